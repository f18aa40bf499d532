"""The no-allocation decode entry point (sa_sparse_paged_decode_seq_codes_noalloc,
split-KV partials in the library's per-GPU scratch array) against the
workspace entry point it mirrors (sa_sparse_paged_decode_seq_codes), through
the C ABI: bit-equal outputs on two calls in a row, the second on a smaller
input, shapes chosen so that the partials are in use (B x H_kv below the
launch's workgroup target, so the pages are split)."""

import pytest
import torch

import sparse_workloads as wl
from ultrametric import _native as nat
from ultrametric.kernel_decode import pack_routing_codes, sequence_page_codes

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _case(B, min_len, max_len, seed):
    w = wl.config4(seed=seed, device=torch.device(DEV), B=B, min_len=min_len, max_len=max_len)
    bpl = 2
    pc = pack_routing_codes(w.router, bpl)
    qc = pack_routing_codes(w.q_router, bpl)
    bt = w.block_tables.to(torch.int32).contiguous()
    sc = sequence_page_codes(pc, bt, bits=w.q_router.shape[-1] * bpl)
    ctx = w.context_lens.to(torch.int32).contiguous()
    return w, bt, ctx, sc, qc, bpl


def _args(w, bt, ctx, sc, qc, bpl, out):
    B, H, D = w.q.shape
    P, Hkv, PS, _ = w.k_cache.shape
    head = (nat.ptr(w.q), nat.ptr(w.k_cache), nat.ptr(w.v_cache), nat.ptr(bt), nat.ptr(ctx), nat.ptr(sc),
            sc.element_size(), nat.ptr(qc), nat.ptr(out), B, H, Hkv, D, PS, w.q_router.shape[-1], bpl,
            bt.shape[1], P, w.req_depth, w.local_blocks, int(w.sink_block), nat.strides(w.q),
            nat.strides(w.k_cache), nat.strides(w.v_cache), nat.strides(bt), nat.strides(sc), nat.strides(qc),
            nat.strides(out))
    return head, (B, H, Hkv, D, bt.shape[1])


def _run_both(case):
    w, bt, ctx, sc, qc, bpl = case
    lib = nat.lib()
    out_ws = torch.empty_like(w.q)
    out_na = torch.full_like(w.q, float("nan"))
    head, (B, H, Hkv, D, mp) = _args(w, bt, ctx, sc, qc, bpl, out_ws)
    need = lib.sa_decode_workspace_bytes(B, H, Hkv, D, mp)
    assert 0 < need <= lib.sa_noalloc_scratch_bytes()
    ws = torch.empty(need, dtype=torch.uint8, device=DEV)
    dt = nat.DTYPE_CODES[w.q.dtype]
    stream = nat.stream(torch.device(DEV))
    nat.check(lib.sa_sparse_paged_decode_seq_codes(*head, nat.ptr(ws), need, dt, stream))
    head_na, _ = _args(w, bt, ctx, sc, qc, bpl, out_na)
    nat.check(lib.sa_sparse_paged_decode_seq_codes_noalloc(*head_na, dt, stream))
    torch.cuda.synchronize()
    return out_ws, out_na


def test_noalloc_matches_workspace_entry_point_twice():
    big = _case(8, 24576, 32768, seed=31)      # 8 splits per (sequence, kv head)
    small = _case(4, 5120, 6144, seed=32)      # 2 splits: fewer partials than the first call left
    for case in (big, small):
        out_ws, out_na = _run_both(case)
        assert torch.isfinite(out_na).all()
        assert torch.equal(out_ws, out_na)


def test_noalloc_rejects_partials_beyond_the_scratch():
    lib = nat.lib()
    cap = lib.sa_noalloc_scratch_bytes()
    # 511 (sequence, kv head) pairs split 2 ways, 8 query heads each, D = 256:
    # 511 * 8 * 2 * 258 * 4 bytes > 8 MiB; rejected on the host before any launch
    B, H, Hkv, D, mp = 511, 8, 1, 256, 300
    need = lib.sa_decode_workspace_bytes(B, H, Hkv, D, mp)
    assert need > cap
    t = torch.zeros(1, device=DEV)
    s3 = nat.strides(torch.zeros(1, 1, 1))
    s4 = nat.strides(torch.zeros(1, 1, 1, 1))
    s2 = nat.strides(torch.zeros(1, 1))
    rc = lib.sa_sparse_paged_decode_seq_codes_noalloc(
        nat.ptr(t), nat.ptr(t), nat.ptr(t), nat.ptr(t), nat.ptr(t), nat.ptr(t), 1, nat.ptr(t), nat.ptr(t),
        B, H, Hkv, D, 16, 4, 2, mp, 1, 4, 0, 0, s3, s4, s4, s2, s3, s2, s3, nat.DTYPE_CODES[torch.bfloat16],
        nat.stream(torch.device(DEV)))
    assert rc == nat.SA_EINVAL
    assert "no-allocation scratch" in lib.sa_last_error().decode()
