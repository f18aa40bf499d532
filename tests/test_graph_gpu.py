"""The per-layer surgery step (route vote, sync-free list build, prefill
forward), the fused one-launch routed prefill and a serving decode step
captured in a HIP graph: every replay, with
new inputs copied into the captured buffers and eager work plus
synchronisations between replays, equals the eager result bit for bit (the
kernels are deterministic and launch nothing outside the captured stream)."""

import pytest
import torch

import sparse_workloads as wl
from ultrametric import block_list_prefill, ultrametric_decode
from ultrametric.kernel_decode import decode_workspace_bytes

pytestmark = pytest.mark.gpu
DEV = "cuda"


def test_surgery_layer_step_in_graph():
    g = torch.Generator().manual_seed(1)
    B, H, Hkv, S, D, L, p, rb, r = 1, 8, 2, 2048, 128, 4, 4, 128, 2
    q = torch.empty(B, H, S, D, dtype=torch.bfloat16, device=DEV)
    k = torch.empty(B, Hkv, S, D, dtype=torch.bfloat16, device=DEV)
    v = torch.empty_like(k)
    a = torch.empty(B, H, S, L, p, device=DEV)

    def fill():
        for t in (q, k, v, a):
            t.copy_(torch.randn(t.shape, generator=g).to(t.dtype))

    def step():
        return block_list_prefill(q, k, v, a, r, p=p, route_block=rb, local_window=16)

    fill()
    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    for _ in range(3):
        fill()
        eager = step()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_decode_step_in_graph():
    # few sequences: the split-KV path with its merge kernel and a static workspace
    w = wl.config4(device=DEV, B=6, min_len=2000, max_len=9000)
    kw = dict(req_depth=w.req_depth, local_blocks=w.local_blocks, sink_block=w.sink_block)
    B, H, D = w.q.shape
    need = decode_workspace_bytes(B, H, D, w.block_tables.shape[1], w.k_cache.shape[1])
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    q = w.q.clone()
    ctx = w.context_lens.clone()

    def step():
        return ultrametric_decode(q, w.k_cache, w.v_cache, w.block_tables, ctx, w.router, w.q_router,
                                  workspace=ws, **kw)

    step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = step()
    g = torch.Generator().manual_seed(2)
    for i in range(3):
        q.copy_(torch.randn(q.shape, generator=g).to(q.dtype))
        ctx.copy_(w.context_lens - i * 37)            # the sequences grow back and forth
        eager = step().clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_fused_routed_prefill_in_graph():
    # routed_block_attention with the arity: list build and prefill in one launch, no host read
    from ultrametric import routed_block_attention
    g = torch.Generator().manual_seed(4)
    Z, H, N, D, rb = 1, 4, 2048, 128, 128
    q = torch.empty(Z, H, N, D, dtype=torch.bfloat16, device=DEV)
    k = torch.empty_like(q)
    v = torch.empty_like(q)
    router = torch.empty(Z, H, N // rb, 3, dtype=torch.int32, device=DEV)

    def fill():
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=g).to(t.dtype))
        router.copy_(torch.randint(0, 4, router.shape, generator=g, dtype=torch.int32))

    def step():
        return routed_block_attention(q, k, v, router, 2, route_block=rb, is_causal=True, sink_block=True, arity=4)

    with torch.no_grad():
        fill()
        step()
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = step()
        for _ in range(3):
            fill()
            eager = step()
            torch.cuda.synchronize()
            graph.replay()
            torch.cuda.synchronize()
            assert torch.equal(out, eager)
