"""GPU parity for the packed routing-code decode path: sa_pack_page_codes is
bit-exact against oracle.decode.pack_codes, and ultrametric_decode_packed
matches the float64 decode oracle, and the int32-level entry point bit for
bit (both walk the same page ranges: up to 2048 pages per range at G = 4)."""

import numpy as np
import pytest
import torch

import sparse_workloads as wl
from oracle import decode as od
from ultrametric import ultrametric_decode
from ultrametric.kernel_decode import pack_routing_codes, ultrametric_decode_packed

from test_decode_gpu import make, oracle, run, TOL

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("TD,bpl", [(1, 1), (4, 2), (6, 5), (8, 4), (16, 2), (32, 1), (2, 16)])
def test_pack_matches_oracle(TD, bpl):
    g = torch.Generator().manual_seed(TD * 31 + bpl)
    r = torch.randint(0, 1 << bpl, (257, 5, TD), generator=g, dtype=torch.int32)
    r[0] = (1 << bpl) - 1
    got = pack_routing_codes(r.to(DEV), bpl).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, od.pack_codes(r.numpy(), bpl))
    # strided (non-contiguous) router view
    rt = torch.randint(0, 1 << bpl, (5, 40, TD), generator=g, dtype=torch.int32).to(DEV).transpose(0, 1)
    got = pack_routing_codes(rt, bpl).cpu().numpy().view(np.uint32)
    assert np.array_equal(got, od.pack_codes(rt.cpu().numpy(), bpl))


def packed(args, TD, bpl, **kw):
    q, kc, vc, bt, ctx, r, qr = (torch.as_tensor(a).to(DEV) for a in args)
    pc, qc = pack_routing_codes(r, bpl), pack_routing_codes(qr, bpl)
    return ultrametric_decode_packed(q, kc, vc, bt, ctx, pc, qc, TD, bpl, **kw)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("TD,p,bpl", [(4, 2, 1), (8, 4, 2), (3, 5, 3)])
def test_packed_decode_matches_oracle(dtype, TD, p, bpl):
    args = make(B=5, H=8, Hkv=2, D=64, page=16, pages=80, TD=TD, p=p, lens=[0, 1, 17, 300, 1000], dtype=dtype,
                seed=TD * 13 + p)
    for kw in (dict(req_depth=2, local_blocks=2, sink_block=True), dict(req_depth=TD), dict(req_depth=0),
               dict(req_depth=1), dict(req_depth=TD + 3, sink_block=True)):
        out = packed(args, TD, bpl, **kw)
        ref = oracle(args, dtype, **kw)
        assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL[dtype], kw
        assert torch.equal(out, run(args, **kw)), kw


def test_packed_multi_split_and_bad_pages():
    args = make(B=2, H=8, Hkv=2, D=128, page=4, pages=5000, TD=6, p=2, lens=[19999, 4097],
                dtype=torch.bfloat16, seed=12)
    bt = args[3].clone()
    bt[0, 7] = 10_000
    bt[1, 3] = -1
    args[3] = bt
    for kw in (dict(req_depth=2, local_blocks=3, sink_block=True), dict(req_depth=5)):
        assert torch.equal(packed(args, 6, 1, **kw), run(args, **kw)), kw


def test_packed_config4():
    w = wl.config4(device=DEV)
    kw = dict(req_depth=w.req_depth, local_blocks=w.local_blocks, sink_block=w.sink_block)
    TD = w.router.shape[-1]
    bpl = max(1, int(w.router.max().item()).bit_length())
    pc, qc = pack_routing_codes(w.router, bpl), pack_routing_codes(w.q_router, bpl)
    out = ultrametric_decode_packed(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, pc, qc, TD,
                                    bpl, **kw)
    ref = ultrametric_decode(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.router,
                             w.q_router, **kw)
    # same selection, same 2048-page ranges, same order: equal bit for bit
    assert torch.equal(out, ref)
    # exact against the oracle on a few sequences (their pages sliced out)
    for b in (0, 31, 63):
        n = -(-int(w.context_lens[b]) // 16)
        phys = w.block_tables[b, :n].long()
        args = [w.q[b:b + 1].cpu(), w.k_cache[phys].cpu(), w.v_cache[phys].cpu(),
                torch.arange(n, dtype=torch.int32)[None], w.context_lens[b:b + 1].cpu(), w.router[phys].cpu(),
                w.q_router[b:b + 1].cpu()]
        assert np.abs(out[b:b + 1].float().cpu().numpy() - oracle(args, torch.bfloat16, **kw)).max() <= 2e-2, b


def test_packed_argument_errors():
    r = torch.zeros(4, 2, 9, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        pack_routing_codes(r, 4)          # 9 levels x 4 bits > 32
    with pytest.raises(ValueError):
        pack_routing_codes(r, 0)


def seq_packed(args, TD, bpl, **kw):
    from ultrametric.kernel_decode import sequence_page_codes, ultrametric_decode_seq_codes
    q, kc, vc, bt, ctx, r, qr = (torch.as_tensor(a).to(DEV) for a in args)
    sc = sequence_page_codes(pack_routing_codes(r, bpl), bt, bits=kw.pop("bits", TD * bpl))
    return ultrametric_decode_seq_codes(q, kc, vc, bt, ctx, sc, pack_routing_codes(qr, bpl), TD, bpl, **kw)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("TD,p,bpl,H,Hkv", [(4, 2, 1, 8, 2), (8, 4, 2, 8, 8), (3, 5, 3, 8, 1), (4, 2, 2, 4, 2)])
def test_seq_codes_decode_matches_oracle(dtype, TD, p, bpl, H, Hkv):
    # ragged and zero lengths, page tables wider than the sequences (unread columns)
    args = make(B=5, H=H, Hkv=Hkv, D=64, page=16, pages=300, TD=TD, p=p, lens=[0, 1, 17, 2999, 1000],
                dtype=dtype, seed=TD * 7 + p + H)
    for kw in (dict(req_depth=2, local_blocks=2, sink_block=True), dict(req_depth=TD), dict(req_depth=0),
               dict(req_depth=TD + 3, sink_block=True)):
        for bits in (TD * bpl, 16, 32):          # narrowest width and wider storage
            out = seq_packed(args, TD, bpl, bits=bits, **kw)
            ref = oracle(args, dtype, **kw)
            assert np.abs(out.float().cpu().numpy() - ref).max() <= TOL[dtype], (kw, bits)
            assert torch.all(out[0] == 0)


def test_seq_codes_long_and_bad_pages():
    # 5000 pages of 4 tokens: several 2048-page ranges (and splits); out-of-range table entries
    args = make(B=2, H=8, Hkv=2, D=128, page=4, pages=5000, TD=6, p=2, lens=[19999, 9000],
                dtype=torch.bfloat16, seed=13)
    bt = args[3].clone()
    bt[0, 7] = 10_000
    bt[1, 3] = -1
    args[3] = bt
    for kw in (dict(req_depth=2, local_blocks=3, sink_block=True), dict(req_depth=5)):
        out = seq_packed(args, 6, 1, **kw)
        ref = packed(args, 6, 1, **kw)
        assert (out.float() - ref.float()).abs().max().item() <= 2e-2, kw


def test_seq_codes_config4_equals_packed():
    from ultrametric.kernel_decode import sequence_page_codes, ultrametric_decode_seq_codes
    w = wl.config4(device=DEV)
    kw = dict(req_depth=w.req_depth, local_blocks=w.local_blocks, sink_block=w.sink_block)
    TD = w.router.shape[-1]
    pc, qc = pack_routing_codes(w.router, 2), pack_routing_codes(w.q_router, 2)
    ref = ultrametric_decode_packed(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, pc, qc, TD, 2,
                                    **kw)
    for bits in (8, 32):
        sc = sequence_page_codes(pc, w.block_tables, bits=bits)
        out = ultrametric_decode_seq_codes(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, sc, qc, TD,
                                           2, **kw)
        assert torch.equal(out, ref), bits     # same selection, same 2048-page ranges, same order
