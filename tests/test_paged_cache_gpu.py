"""GPU parity of the serving decode over a real paged cache
(ultrametric.paged_cache): page reservation, K / V writes (sa_paged_kv_write),
length updates (sa_paged_advance), first-token page codes appended to the
per-sequence code array, and the single-token decode step over it
(ultrametric_decode_seq_codes), the paged replacement of the eager decode
masks of src/llama_surgery/surgery.py:880-955.

Every step is checked against a host model of the cache built from the
tokens alone: the cache's pages hold exactly the tokens written (bit for bit,
read back through the block tables), its codes are the first tokens' codes,
its lengths the token counts, and the decode output matches the float64
oracle (oracle/decode.py, the reference's _ultrametric_decode_reference
semantics with GQA) on the router rebuilt from those first tokens, bf16
tolerance 2e-2. A step captured in a HIP graph replays bit-equal to the
same steps run eagerly on a twin cache."""

import numpy as np
import pytest
import torch

from oracle import decode as od
from paged_host import BPL, P_ARITY, TD, HostModel, oracle_inputs
from ultrametric.paged_cache import PagedKVCache, token_routing_codes

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _check_cache(cache, host, layer=0):
    lens = host.lens()
    assert cache.context_lens[:len(lens)].cpu().tolist() == lens
    kc = cache.k[layer].float().cpu().numpy()
    vc = cache.v[layer].float().cpu().numpy()
    sc = cache.seq_codes[layer].cpu().numpy().astype(np.int64) & 0xFF
    bt = cache.block_tables.cpu().numpy()
    PS = cache.page_size
    for b, n in enumerate(lens):
        for t in range(n):
            page, row = bt[b, t // PS], t % PS
            assert np.array_equal(kc[page, :, row], host.k[b][:, t]), (b, t)
            assert np.array_equal(vc[page, :, row], host.v[b][:, t]), (b, t)
        for l in range(-(-n // PS)):
            lv = host.lv[b][:, l * PS]                        # (H, TD): level 0 most significant
            code = sum(lv[:, i] << (BPL * (TD - 1 - i)) for i in range(TD))
            assert np.array_equal(sc[b, :, l], code), (b, l)
    assert int(cache.status.item()) == 0


def _rand(shape, g, dtype=torch.bfloat16):
    return torch.randn(shape, generator=g).to(dtype)


@pytest.mark.parametrize("req_depth,local,sink", [(4, 4, True), (2, 1, False), (0, 0, False)])
def test_ragged_prefill_then_decode_steps(req_depth, local, sink):
    g = torch.Generator().manual_seed(100 + req_depth)
    B, Hkv, H, D, PS = 5, 2, 8, 128, 16
    cache = PagedKVCache(num_pages=220, page_size=PS, kv_heads=Hkv, head_dim=D, heads=H, tree_depth=TD,
                         bits_per_level=BPL, max_seqs=B, max_pages_per_seq=40, device=DEV)
    host = HostModel(B, Hkv, H, D)
    # ragged prompts: empty, exactly one page, one past a page, longer ones
    lens = [0, 16, 17, 100, 250]
    T = max(lens)
    k = _rand((B, Hkv, T, D), g)
    v = _rand((B, Hkv, T, D), g)
    lv = torch.randint(0, P_ARITY, (B, H, T, TD), generator=g)
    cache.reserve(lens, rows=range(B))
    n_new = torch.tensor(lens, dtype=torch.int32, device=DEV)
    cache.advance(n_new, B, host_counts=lens)
    cache.write(0, k.to(DEV), v.to(DEV), token_routing_codes(lv.to(DEV), BPL), n_new=n_new)
    for b in range(B):
        host.add(b, k[b, :, :lens[b]].float().numpy(), v[b, :, :lens[b]].float().numpy(),
                 lv[b, :, :lens[b]].numpy())
    _check_cache(cache, host)
    # decode steps: every row takes a token, then a step where rows 1 and 4 idle
    for step in range(6):
        active = [1] * B if step != 3 else [1, 0, 1, 1, 0]
        cache.reserve(active, rows=range(B))
        k1, v1 = _rand((B, Hkv, 1, D), g), _rand((B, Hkv, 1, D), g)
        lv1 = torch.randint(0, P_ARITY, (B, H, 1, TD), generator=g)
        if all(active):
            cache.advance(1, B)
            cache.write(0, k1.to(DEV), v1.to(DEV), token_routing_codes(lv1.to(DEV), BPL))
        else:
            nn = torch.tensor(active, dtype=torch.int32, device=DEV)
            cache.advance(nn, B, host_counts=active)
            cache.write(0, k1.to(DEV), v1.to(DEV), token_routing_codes(lv1.to(DEV), BPL), n_new=nn)
        for b in range(B):
            if active[b]:
                host.add(b, k1[b].float().numpy(), v1[b].float().numpy(), lv1[b].numpy())
        q = _rand((B, H, D), g)
        qlv = torch.randint(0, P_ARITY, (B, H, 1, TD), generator=g)
        qc = token_routing_codes(qlv.to(DEV), BPL)[:, :, 0].contiguous()
        out = cache.decode(0, q.to(DEV), qc, req_depth, local_blocks=local, sink_block=sink)
        kc, vc, bt, router = oracle_inputs(cache, host, cache._pages, H)
        ref = od.decode_reference(q.float().numpy(), kc, vc, bt, np.array(host.lens()), router,
                                  qlv[:, :, 0].numpy().astype(np.int32), req_depth, local_blocks=local,
                                  sink_block=sink)
        assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-2, step
        assert cache.lengths == host.lens()
    _check_cache(cache, host)


def test_unaligned_fp16_rows_and_release():
    # D = 16 fp16 rows taken from an offset view: the element-by-element path
    g = torch.Generator().manual_seed(4)
    B, Hkv, H, D, PS = 3, 1, 2, 16, 4
    cache = PagedKVCache(num_pages=12, page_size=PS, kv_heads=Hkv, head_dim=D, heads=H, tree_depth=TD,
                         bits_per_level=BPL, max_seqs=B, max_pages_per_seq=4, dtype=torch.float16, device=DEV)
    host = HostModel(B, Hkv, H, D)
    for step in range(7):
        cache.reserve(1, rows=range(B))
        big_k = _rand((B, Hkv, 1, D + 1), g, torch.float16)
        big_v = _rand((B, Hkv, 1, D + 1), g, torch.float16)
        lv = torch.randint(0, P_ARITY, (B, H, 1, TD), generator=g)
        cache.advance(1, B)
        cache.write(0, big_k.to(DEV)[..., 1:], big_v.to(DEV)[..., 1:], token_routing_codes(lv.to(DEV), BPL))
        for b in range(B):
            host.add(b, big_k[b, :, :, 1:].float().numpy(), big_v[b, :, :, 1:].float().numpy(), lv[b].numpy())
    _check_cache(cache, host)
    free = cache.free_pages()
    cache.release([1])
    assert cache.free_pages() == free + 2 and cache.lengths[1] == 0
    assert (cache.block_tables[1] == -1).all() and int(cache.context_lens[1]) == 0


def test_write_outside_reserved_pages_is_flagged_not_stored():
    # the block-table slot holds -1: the kernel's bounds check skips the write
    cache = PagedKVCache(num_pages=4, page_size=16, kv_heads=1, head_dim=64, heads=1, tree_depth=TD,
                         bits_per_level=BPL, max_seqs=1, max_pages_per_seq=2, device=DEV)
    k = torch.ones(1, 1, 1, 64, dtype=torch.bfloat16, device=DEV)
    cache.advance(1, 1)
    cache.write(0, k, k)
    assert int(cache.k.abs().sum()) == 0
    with pytest.raises(RuntimeError, match="reserved"):
        cache.check_status()
    assert int(cache.status.item()) == 0


def test_decode_step_graph_replays_bit_equal():
    g = torch.Generator().manual_seed(9)
    B, Hkv, H, D, PS, layers = 4, 2, 8, 128, 16, 2
    kw = dict(num_pages=160, page_size=PS, kv_heads=Hkv, head_dim=D, heads=H, tree_depth=TD, bits_per_level=BPL,
              max_seqs=B, max_pages_per_seq=32, layers=layers, device=DEV)
    caches = [PagedKVCache(**kw), PagedKVCache(**kw)]
    lens = [30, 1, 64, 200]
    T = max(lens)
    pk, pv = _rand((layers, B, Hkv, T, D), g), _rand((layers, B, Hkv, T, D), g)
    plv = torch.randint(0, P_ARITY, (layers, B, H, T, TD), generator=g)
    nn = torch.tensor(lens, dtype=torch.int32, device=DEV)
    steps = 5
    for c in caches:
        c.reserve(lens, rows=range(B))
        c.advance(nn, B, host_counts=lens)
        for l in range(layers):
            c.write(l, pk[l].to(DEV), pv[l].to(DEV), token_routing_codes(plv[l].to(DEV), BPL), n_new=nn)
        c.reserve(steps + 1, rows=range(B))         # pages for the warmup step and the replays
    # static inputs of the captured step
    q_s = torch.empty(layers, B, H, D, dtype=torch.bfloat16, device=DEV)
    k_s = torch.empty(layers, B, Hkv, 1, D, dtype=torch.bfloat16, device=DEV)
    v_s = torch.empty_like(k_s)
    c_s = torch.empty(layers, B, H, 1, dtype=torch.int32, device=DEV)
    qc_s = torch.empty(layers, B, H, dtype=torch.int32, device=DEV)

    def fill():
        q_s.copy_(_rand(q_s.shape, g))
        k_s.copy_(_rand(k_s.shape, g))
        v_s.copy_(_rand(v_s.shape, g))
        c_s.copy_(token_routing_codes(torch.randint(0, P_ARITY, (layers * B, H, 1, TD), generator=g).to(DEV),
                                      BPL).view(layers, B, H, 1))
        qc_s.copy_(token_routing_codes(torch.randint(0, P_ARITY, (layers * B, H, 1, TD), generator=g).to(DEV),
                                       BPL).view(layers, B, H))

    def step(c):
        c.advance(1, B)
        outs = []
        for l in range(layers):
            c.write(l, k_s[l], v_s[l], c_s[l])
            outs.append(c.decode(l, q_s[l], qc_s[l], 4, local_blocks=4, sink_block=True))
        return torch.stack(outs)

    fill()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):                   # warmup step on both caches
        step(caches[0])
        step(caches[1])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out_g = step(caches[0])
    # capture does not run the step: cache 1 runs it eagerly now, the graph replays it
    eager = step(caches[1])
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(out_g, eager)
    for _ in range(steps - 1):
        fill()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        eager = step(caches[1])
        torch.cuda.synchronize()
        assert torch.equal(out_g, eager)
    a, b = caches
    assert torch.equal(a.context_lens, b.context_lens)
    assert a.context_lens.cpu().tolist() == [x + steps + 1 for x in lens]
    for name in ("k", "v", "seq_codes"):
        assert torch.equal(getattr(a, name), getattr(b, name)), name
    assert int(a.status.item()) == 0 and int(b.status.item()) == 0
