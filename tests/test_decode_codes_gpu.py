"""GPU parity for the packed routing-code decode path: sa_pack_page_codes is
bit-exact against oracle.decode.pack_codes, and ultrametric_decode_packed
matches the float64 decode oracle (and the int32-level entry point bit for
bit, as both run the same attention code on the same selection)."""

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
    assert torch.equal(out, ref)


def test_packed_argument_errors():
    r = torch.zeros(4, 2, 9, dtype=torch.int32, device=DEV)
    with pytest.raises(ValueError):
        pack_routing_codes(r, 4)          # 9 levels x 4 bits > 32
    with pytest.raises(ValueError):
        pack_routing_codes(r, 0)
