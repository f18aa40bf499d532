"""GPU parity: HIP sparse paged decode vs the float64 decode oracle
(oracle/decode.py), including the reference's test grid
(tests/test_llama_surgery.py:355-398: fp32, D=16, 6 pages of 8 tokens, tree
depths 1..10, local_blocks=1, sink), GQA, ragged/zero context lengths,
multi-split sequences, out-of-range block-table entries and BASELINE
config 4 (checked on a subset of sequences, plus properties on all)."""

import numpy as np
import pytest
import torch

import sparse_workloads as wl
from oracle import decode as od
from ultrametric import ultrametric_decode

pytestmark = pytest.mark.gpu
DEV = "cuda"
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 2e-3}


def run(args, **kw):
    q, kc, vc, bt, ctx, r, qr = (torch.as_tensor(a).to(DEV) for a in args)
    return ultrametric_decode(q, kc, vc, bt, ctx, r, qr, **kw)


def oracle(args, dtype, **kw):
    q, kc, vc, bt, ctx, r, qr = args
    f = lambda t: t.float().numpy() if isinstance(t, torch.Tensor) else t  # noqa: E731
    return od.decode_reference(f(q), f(kc), f(vc), np.asarray(bt), np.asarray(ctx), np.asarray(r),
                               np.asarray(qr), **kw)


def make(B, H, Hkv, D, page, pages, TD, p, lens, dtype, seed, max_pages=None):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(B, H, D, generator=g).to(dtype)
    kc = torch.randn(pages, Hkv, page, D, generator=g).to(dtype)
    vc = torch.randn(pages, Hkv, page, D, generator=g).to(dtype)
    mp = max_pages or max(1, max(-(-l // page) for l in lens))
    bt = torch.stack([torch.randperm(pages, generator=g)[:mp] for _ in range(B)]).to(torch.int32)
    ctx = torch.tensor(lens, dtype=torch.int32)
    r = torch.randint(0, p, (pages, H, TD), generator=g, dtype=torch.int32)
    qr = torch.randint(0, p, (B, H, TD), generator=g, dtype=torch.int32)
    return [q, kc, vc, bt, ctx, r, qr]


@pytest.mark.parametrize("tree_depth", [1, 3, 5, 6, 7, 10])
def test_reference_grid_fp32(tree_depth):
    torch.manual_seed(100 + tree_depth)
    B, H, D, num_blocks, bs = 2, 4, 16, 6, 8
    q = torch.randn(B, H, D)
    kc = torch.randn(num_blocks, H, bs, D)
    vc = torch.randn(num_blocks, H, bs, D)
    bt = torch.arange(num_blocks, dtype=torch.int32).unsqueeze(0).repeat(B, 1)
    ctx = torch.tensor([40, 35], dtype=torch.int32)
    r = torch.randint(0, 2, (num_blocks, H, tree_depth), dtype=torch.int32)
    qr = torch.randint(0, 2, (B, H, tree_depth), dtype=torch.int32)
    args = [q, kc, vc, bt, ctx, r, qr]
    rd = min(3, tree_depth)
    out = run(args, req_depth=rd, local_blocks=1, sink_block=True)
    ref = oracle(args, torch.float32, req_depth=rd, local_blocks=1, sink_block=True)
    assert out.shape == (B, H, D)
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-5


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H,Hkv", [(4, 4), (8, 2), (32, 8), (8, 1), (6, 2), (10, 2), (28, 4), (32, 2)])
@pytest.mark.parametrize("D", [64, 128])
def test_gqa_ragged(dtype, H, Hkv, D):
    args = make(B=5, H=H, Hkv=Hkv, D=D, page=16, pages=80, TD=4, p=2,
                lens=[0, 1, 17, 300, 1000], dtype=dtype, seed=H * 7 + D)
    for kw in (dict(req_depth=2, local_blocks=2, sink_block=True), dict(req_depth=4), dict(req_depth=0),
               dict(req_depth=9, sink_block=True)):
        out = run(args, **kw)
        ref = oracle(args, dtype, **kw)
        err = np.abs(out.float().cpu().numpy() - ref).max()
        assert err <= TOL[dtype], (kw, err)
        assert torch.all(out[0] == 0)          # ctx = 0 -> zeros


def test_multi_split_long_sequences():
    # 5000 pages of 4 tokens: more than one split of 256 pages per sequence
    args = make(B=2, H=8, Hkv=2, D=128, page=4, pages=5000, TD=2, p=2, lens=[19999, 4097],
                dtype=torch.bfloat16, seed=11)
    for kw in (dict(req_depth=2, local_blocks=3, sink_block=True), dict(req_depth=0)):
        out = run(args, **kw)
        ref = oracle(args, torch.bfloat16, **kw)
        assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-2


@pytest.mark.parametrize("B,max_len", [(300, 200), (37, 3000)])
def test_many_sequences_balanced_slices(B, max_len):
    # equal unit slices over 512 workgroups cut many segments: zero-length sequences
    # interspersed, every sequence checked against the oracle
    g = torch.Generator().manual_seed(B)
    lens = torch.randint(0, max_len, (B,), generator=g)
    lens[::7] = 0
    lens[1] = max_len
    args = make(B=B, H=4, Hkv=2, D=32, page=8, pages=max(64, -(-max_len // 8) + 8), TD=3, p=2,
                lens=[int(x) for x in lens], dtype=torch.float32, seed=B + 1)
    for kw in (dict(req_depth=1, local_blocks=2, sink_block=True), dict(req_depth=3), dict(req_depth=0)):
        out = run(args, **kw)
        ref = oracle(args, torch.float32, **kw)
        assert np.abs(out.cpu().numpy() - ref).max() <= 1e-5, kw
        assert torch.all(out[lens == 0] == 0)


def test_more_sequences_than_balanced_limit():
    # > 4096 sequences: one workgroup per (sequence, kv head), no workspace
    B = 4100
    g = torch.Generator().manual_seed(5)
    lens = [int(x) for x in torch.randint(0, 40, (B,), generator=g)]
    args = make(B=B, H=4, Hkv=2, D=32, page=16, pages=32, TD=2, p=2, lens=lens, dtype=torch.float32, seed=6,
                max_pages=3)
    out = run(args, req_depth=1, local_blocks=1, sink_block=True)
    sub = list(range(0, B, 97))
    sargs = [a[sub] if i in (0, 3, 4, 6) else a for i, a in enumerate(args)]
    ref = oracle(sargs, torch.float32, req_depth=1, local_blocks=1, sink_block=True)
    assert np.abs(out[sub].cpu().numpy() - ref).max() <= 1e-5


def test_out_of_range_pages_are_skipped():
    args = make(B=2, H=4, Hkv=4, D=32, page=8, pages=10, TD=2, p=2, lens=[70, 40], dtype=torch.float32,
                seed=3)
    bt = args[3].clone()
    bt[0, 2] = 10_000     # outside the cache: treated as not selected
    bt[1, 1] = -5
    args[3] = bt
    out = run(args, req_depth=0)
    ok = args[3].clone()
    # the oracle on the same selection: drop those pages by pointing them at a zero-length view
    q, kc, vc, _, ctx, r, qr = args
    ref = np.zeros(out.shape)
    for b, bad in ((0, 2), (1, 1)):
        n = -(-int(ctx[b]) // 8)
        keep = [l for l in range(n) if l != bad]
        ks = np.concatenate([kc[ok[b, l], :, :min(8, int(ctx[b]) - l * 8)].numpy() for l in keep], 1)
        vs = np.concatenate([vc[ok[b, l], :, :min(8, int(ctx[b]) - l * 8)].numpy() for l in keep], 1)
        for h in range(4):
            s = ks[h] @ q[b, h].numpy().astype(np.float64) / np.sqrt(32)
            w = np.exp(s - s.max())
            ref[b, h] = (w / w.sum()) @ vs[h]
    assert np.abs(out.cpu().numpy() - ref).max() <= 1e-5


def test_config4_subset_and_properties():
    w = wl.config4(device=DEV)
    kw = dict(req_depth=w.req_depth, local_blocks=w.local_blocks, sink_block=w.sink_block)
    out = ultrametric_decode(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.router,
                             w.q_router, **kw)
    assert out.shape == (64, 32, 128) and torch.isfinite(out).all()
    # exact check on 4 sequences: slice their pages out of the cache
    for b in (0, 17, 40, 63):
        n = -(-int(w.context_lens[b]) // 16)
        phys = w.block_tables[b, :n].long()
        kc, vc, rt = w.k_cache[phys].cpu(), w.v_cache[phys].cpu(), w.router[phys].cpu()
        bt = torch.arange(n, dtype=torch.int32)[None]
        args = [w.q[b:b + 1].cpu(), kc, vc, bt, w.context_lens[b:b + 1].cpu(), rt, w.q_router[b:b + 1].cpu()]
        ref = oracle(args, torch.bfloat16, **kw)
        assert np.abs(out[b:b + 1].float().cpu().numpy() - ref).max() <= 2e-2, b
    # determinism: a second call is bit-identical
    out2 = ultrametric_decode(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.router,
                              w.q_router, **kw)
    assert torch.equal(out, out2)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_range_and_half_boundaries(dtype):
    # phase A runs 1024-page halves of 2048-page ranges at G = 4: sequences of
    # 1024 / 1025 / 2047 / 2048 / 2049 pages end a half, start one, fill a range
    # or spill into the next
    page = 16
    lens = [1024 * page, 1024 * page + 1, 2047 * page, 2048 * page, 2048 * page + 5]
    args = make(B=5, H=8, Hkv=2, D=64, page=page, pages=2100, TD=4, p=2, lens=lens, dtype=dtype, seed=77)
    for kw in (dict(req_depth=3, local_blocks=2, sink_block=True), dict(req_depth=4)):
        out = run(args, **kw)
        ref = oracle(args, dtype, **kw)
        assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL[dtype], kw
