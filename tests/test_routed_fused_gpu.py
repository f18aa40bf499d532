"""The fused routed prefill (sa_routed_block_sparse_fwd: list build inside the
forward kernel) against the two-launch path it replaces: build_block_lists
(sync-free, `arity`) then block_list_attention. Lists, counts and the output
must be identical bit for bit (same lists, same kernel arithmetic). Cases the
fused kernel does not cover (soft bias, fp32, NB above one key block per
thread, gradients) take the two-launch path through the same API."""

import pytest
import torch

from ultrametric import block_list_attention, build_block_lists, routed_block_attention
from ultrametric.block_list import _routed_fused

pytestmark = pytest.mark.gpu
DEV = "cuda"

CASES = [
    # Z, H, Hkv, N, D, rb, TD, p (ids in [0, p)), arity, depth, causal, sink, local, dtype, id dtype
    (1, 4, 2, 1024, 128, 128, 3, 4, 4, 2, True, True, 0, torch.bfloat16, torch.int32),
    (2, 2, 2, 1000, 64, 64, 3, 2, 2, [1, 3], False, True, 1, torch.float16, torch.int64),
    (1, 3, 3, 640, 32, 32, 2, 2, 2, 1, True, False, 2, torch.bfloat16, torch.int32),
    (1, 2, 1, 2048, 128, 256, 4, 4, 4, 3, True, True, 1, torch.bfloat16, torch.int32),
    (1, 2, 2, 512, 64, 128, 3, 2, 2, 0, True, False, 0, torch.float16, torch.int32),
    (1, 4, 4, 8192, 128, 128, 3, 4, 4, 2, True, True, 0, torch.bfloat16, torch.int32),
    (1, 2, 2, 777, 128, 64, 3, 5, 4, 2, True, True, 0, torch.bfloat16, torch.int64),   # ids >= arity alias
]


def inputs(Z, H, Hkv, N, D, rb, TD, p, dtype, id_dtype, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Z, H, N, D, generator=g).to(dtype).to(DEV)
    k = torch.randn(Z, Hkv, N, D, generator=g).to(dtype).to(DEV)
    v = torch.randn(Z, Hkv, N, D, generator=g).to(dtype).to(DEV)
    router = torch.randint(0, p, (Z, H, -(-N // rb), TD), generator=g).to(id_dtype).to(DEV)
    return q, k, v, router


@pytest.mark.parametrize("case", CASES, ids=[f"case{i}" for i in range(len(CASES))])
def test_fused_equals_two_launches(case):
    Z, H, Hkv, N, D, rb, TD, p, arity, depth, causal, sink, local, dtype, id_dtype = case
    q, k, v, router = inputs(Z, H, Hkv, N, D, rb, TD, p, dtype, id_dtype, seed=N + D + rb)
    kw = dict(is_causal=causal, sink_block=sink, local_blocks=local)
    with torch.no_grad():
        fused = _routed_fused(q, k, v, router, depth, route_block=rb, sm_scale=None, arity=arity, **kw)
        assert fused is not None
        out, bl = fused
        ref_bl = build_block_lists(router, depth, arity=arity, **kw)
        ref = block_list_attention(q, k, v, ref_bl, route_block=rb, is_causal=causal)
        assert torch.equal(bl.counts, ref_bl.counts)
        assert torch.equal(bl.lists, ref_bl.lists)
        assert bl.max_count == ref_bl.max_count
        assert torch.equal(out, ref)
        api = routed_block_attention(q, k, v, router, depth, route_block=rb, arity=arity, **kw)
        assert torch.equal(api, ref)


def test_fused_with_scale_and_strided_q():
    Z, H, N, D, rb = 1, 2, 1024, 128, 128
    q, k, v, router = inputs(Z, H, H, N, D, rb, 3, 4, torch.bfloat16, torch.int32, seed=5)
    qs = q.transpose(1, 2).contiguous().transpose(1, 2)        # (Z, N, H, D) memory, (Z, H, N, D) view
    with torch.no_grad():
        out = routed_block_attention(qs, k, v, router, 2, route_block=rb, is_causal=True, sink_block=True,
                                     sm_scale=0.05, arity=4)
        bl = build_block_lists(router, 2, is_causal=True, sink_block=True, arity=4)
        ref = block_list_attention(q, k, v, bl, route_block=rb, is_causal=True, sm_scale=0.05)
    assert torch.equal(out, ref)


@pytest.mark.parametrize("what", ["nb_too_large", "fp32", "soft_bias", "grad"])
def test_uncovered_cases_take_the_two_launch_path(what):
    Z, H, D = 1, 2, 64
    N, rb, dtype = (4096, 32, torch.bfloat16) if what == "nb_too_large" else (512, 64, torch.bfloat16)
    if what == "fp32":
        dtype = torch.float32
    q, k, v, router = inputs(Z, H, H, N, D, rb, 3, 2, dtype, torch.int32, seed=11)
    kw = dict(is_causal=True, sink_block=True)
    bl = build_block_lists(router, 1, arity=2, **kw)
    sb = torch.randn(Z, H, bl.counts.shape[-1], bl.max_count, device=DEV) if what == "soft_bias" else None
    if what == "nb_too_large":
        with torch.no_grad():
            assert _routed_fused(q, k, v, router, 1, route_block=rb, sm_scale=None, arity=2, local_blocks=0,
                                 **kw) is None
    if what == "grad":
        q.requires_grad_(True)
        out = routed_block_attention(q, k, v, router, 1, route_block=rb, arity=2, **kw)
        out.float().sum().backward()
        assert q.grad is not None
        ref = block_list_attention(q.detach(), k, v, bl, route_block=rb, is_causal=True)
        assert torch.equal(out.detach(), ref)
        return
    with torch.no_grad():
        out = routed_block_attention(q, k, v, router, 1, route_block=rb, arity=2, soft_block_bias=sb, **kw)
        ref = block_list_attention(q, k, v, bl, route_block=rb, is_causal=True, soft_block_bias=sb)
    assert torch.equal(out, ref)
