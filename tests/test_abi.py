"""C-ABI library checks that need no GPU: it loads, exports every symbol that
include/sparse_attn.h declares, reports its ABI version, and rejects bad
arguments on the host with the documented status codes. The Python layer
raises instead of falling back to the CPU."""

import ctypes
import os
import re

import pytest
import torch

from ultrametric import _native as nat

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "sparse_attn.h")


def declared_symbols():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"\b(sa_[a-z_0-9]+)\s*\(", text)))


def test_library_loads_and_exports_header_symbols():
    assert os.path.exists(nat.LIB_PATH), "build libsparseattn.so first (__graft_entry__.build())"
    lib = ctypes.CDLL(nat.LIB_PATH)
    syms = declared_symbols()
    assert len(syms) >= 7
    for s in syms:
        assert hasattr(lib, s), s
    assert set(syms) == set(nat.EXPORTED_SYMBOLS)
    assert nat.lib().sa_abi_version() == 1


def test_host_side_argument_errors():
    lib = nat.lib()
    st = (ctypes.c_int64 * 4)(1, 1, 1, 1)
    # NULL router
    rc = lib.sa_build_block_lists(None, 3, st, 1, 1, 4, 2, None, 1, 2, 1, 0, 0, 0, None, 4, None, None)
    assert rc == nat.SA_EINVAL and b"NULL" in lib.sa_last_error()
    # bad router dtype
    rc = lib.sa_build_block_lists(ctypes.c_void_p(16), 0, st, 1, 1, 4, 2, None, 1, 2, 1, 0, 0, 0, None, 4,
                                  ctypes.c_void_p(16), None)
    assert rc == nat.SA_EINVAL
    # depth out of range
    rc = lib.sa_build_block_lists(ctypes.c_void_p(16), 3, st, 1, 1, 4, 2, None, 3, 2, 1, 0, 0, 0, None, 4,
                                  ctypes.c_void_p(16), None)
    assert rc == nat.SA_EINVAL
    # NB beyond the LDS code table
    rc = lib.sa_build_block_lists(ctypes.c_void_p(16), 3, st, 1, 1, 9000, 2, None, 1, 2, 1, 0, 0, 0, None, 4,
                                  ctypes.c_void_p(16), None)
    assert rc == nat.SA_EUNSUPPORTED
    # forward: head_dim not a power of two, route block too small, D too large
    p = ctypes.c_void_p(256)
    for D, rb, code in ((48, 64, nat.SA_EINVAL), (64, 8, nat.SA_EINVAL), (512, 64, nat.SA_EUNSUPPORTED)):
        rc = lib.sa_block_sparse_fwd(p, p, p, p, None, p, p, None, 0, 1, 1, 1, 64, D, rb, 1, st, st, st, st,
                                     None, 0.1, 1, 0, None)
        assert rc == code, (D, rb)
    # decode: H not a multiple of H_kv, too small workspace
    st3 = (ctypes.c_int64 * 3)(1, 1, 1)
    st2 = (ctypes.c_int64 * 2)(1, 1)
    stk = (ctypes.c_int64 * 4)(2 * 16 * 64, 16 * 64, 64, 1)
    args = [p] * 8 + [1, 7, 2, 64, 16, 4, 4, 10, 4, 0, 0, st3, stk, stk, st2, st3, st3, st3, p, 0, 1, None]
    assert lib.sa_sparse_paged_decode(*args) == nat.SA_EINVAL
    args[9] = 8
    args[14] = 300  # 300 pages for 2 (sequence, kv head) pairs: split-KV, needs a workspace
    assert lib.sa_sparse_paged_decode(*args) == nat.SA_EINVAL
    assert b"workspace" in lib.sa_last_error()
    assert lib.sa_decode_workspace_bytes(2, 8, 8, 64, 300) == 2 * 8 * 2 * 66 * 4
    # enough (sequence, kv head) pairs to fill the GPU: one workgroup each, no workspace
    assert lib.sa_decode_workspace_bytes(64, 32, 8, 128, 2048) == 0


def test_route_vote_argument_errors():
    lib = nat.lib()
    p = ctypes.c_void_p(16)
    st5 = (ctypes.c_int64 * 5)(1, 1, 1, 1, 1)
    out = ctypes.c_void_p(16)
    # r beyond the levels, zero route block, too many branches, bad dtype
    assert lib.sa_route_block_vote(p, 0, st5, 1, 1, 8, 2, 2, 3, 4, out, None) == nat.SA_EINVAL
    assert lib.sa_route_block_vote(p, 0, st5, 1, 1, 8, 2, 2, 1, 0, out, None) == nat.SA_EINVAL
    assert lib.sa_route_block_vote(p, 0, st5, 1, 1, 8, 2, 65, 1, 4, out, None) == nat.SA_EUNSUPPORTED
    assert lib.sa_route_block_vote(p, 3, st5, 1, 1, 8, 2, 2, 1, 4, out, None) == nat.SA_EINVAL
    # empty problem: no launch, OK
    assert lib.sa_route_block_vote(p, 0, st5, 0, 1, 8, 2, 2, 1, 4, out, None) == nat.SA_OK



def test_packed_code_argument_errors():
    lib = nat.lib()
    p = ctypes.c_void_p(16)
    st3 = (ctypes.c_int64 * 3)(8, 4, 1)
    # bits per level out of [1, 16]; TD * bits beyond 32; empty problem is OK
    assert lib.sa_pack_page_codes(p, st3, 4, 2, 4, 0, p, None) == nat.SA_EINVAL
    assert lib.sa_pack_page_codes(p, st3, 4, 2, 4, 17, p, None) == nat.SA_EINVAL
    assert lib.sa_pack_page_codes(p, st3, 4, 2, 9, 4, p, None) == nat.SA_EINVAL
    assert lib.sa_pack_page_codes(p, st3, 0, 2, 4, 4, p, None) == nat.SA_OK
    st = [(ctypes.c_int64 * 4)(1, 1, 1, 1) for _ in range(7)]
    args = [p] * 8 + [1, 4, 4, 64, 16, 4]
    tail = [8, 8, 2, 0, 0] + st + [None, 0, 1, None]
    assert lib.sa_sparse_paged_decode_codes(*args, 0, *tail) == nat.SA_EINVAL
    assert lib.sa_sparse_paged_decode_codes(*args, 9, *tail) == nat.SA_EINVAL

def test_python_layer_raises_on_cpu_tensors():
    from ultrametric import block_list_attention, build_block_lists, ultrametric_decode
    r = torch.zeros(1, 1, 4, 2, dtype=torch.int32)
    with pytest.raises(RuntimeError, match="HIP"):
        build_block_lists(r, 1, arity=2)
    q = torch.zeros(1, 1, 64, 32)
    bl = (torch.zeros(1, 1, 1, 1, dtype=torch.int32), torch.ones(1, 1, 1, dtype=torch.int32), 1)
    with pytest.raises(RuntimeError, match="HIP"):
        block_list_attention(q, q, q, bl, route_block=64)
    with pytest.raises(RuntimeError, match="HIP"):
        ultrametric_decode(torch.zeros(1, 1, 16), torch.zeros(1, 1, 4, 16), torch.zeros(1, 1, 4, 16),
                           torch.zeros(1, 1, dtype=torch.int32), torch.ones(1, dtype=torch.int32),
                           torch.zeros(1, 1, 2, dtype=torch.int32), torch.zeros(1, 1, 2, dtype=torch.int32), 1)


def test_python_validation_matches_reference_errors():
    from ultrametric import block_list_attention, build_block_lists
    with pytest.raises(ValueError):
        build_block_lists(torch.zeros(2, 3, 4, dtype=torch.int32), 1)          # not 4-D
    with pytest.raises(ValueError):
        build_block_lists(torch.zeros(1, 2, 4, 3, dtype=torch.int32), 4, arity=2)
    q = torch.zeros(1, 2, 64, 48)
    bl = (torch.zeros(1, 2, 1, 1, dtype=torch.int32), torch.ones(1, 2, 1, dtype=torch.int32), 1)
    with pytest.raises(ValueError, match="head_dim"):
        block_list_attention(q, q, q, bl, route_block=64)
    q = torch.zeros(1, 2, 64, 32)
    with pytest.raises(ValueError, match="route_block"):
        block_list_attention(q, q, q, bl, route_block=48)
    with pytest.raises(ValueError, match="block_lists built for"):
        block_list_attention(q, q, q, bl, route_block=32)
    with pytest.raises(ValueError, match="divide"):
        block_list_attention(q, q, q, bl, route_block=64, block_m=48)


def test_empty_problems_accept_null_data():
    # zero-size tensors hand over NULL data pointers; an empty problem is a
    # no-op (no launch, no device call) whatever the pointers
    lib = nat.lib()
    s = [(ctypes.c_int64 * 5)(1, 1, 1, 1, 1) for _ in range(8)]
    N0 = None
    assert lib.sa_build_block_lists(N0, 3, s[0], 0, 2, 4, 2, None, 1, 2, 1, 1, 0, 0, N0, 4, N0, None) == nat.SA_OK
    assert lib.sa_build_block_lists_mask(N0, s[0], 1, 0, 4, 1, 0, 0, N0, 4, N0, None) == nat.SA_OK
    assert lib.sa_transpose_block_lists(N0, N0, 4, 0, 2, 4, N0, 4, N0, None) == nat.SA_OK
    for Z, H, N in ((0, 2, 64), (1, 0, 64), (1, 2, 0)):
        assert lib.sa_block_sparse_fwd(N0, N0, N0, N0, N0, N0, N0, N0, 0, Z, H, 1 if H == 0 else H, N, 64, 64, 1,
                                       s[0], s[1], s[2], s[3], None, 0.1, 1, 1, None) == nat.SA_OK, (Z, H, N)
    assert lib.sa_route_block_vote(N0, 0, s[0], 0, 2, 64, 3, 2, 1, 32, N0, None) == nat.SA_OK
    assert lib.sa_pack_page_codes(N0, s[0], 0, 4, 3, 2, N0, None) == nat.SA_OK
    assert lib.sa_ternary_pack(N0, 1, s[0], 0, 64, 0, N0, N0, None) == nat.SA_OK
    assert lib.sa_ternary_prefill_fwd(N0, N0, N0, N0, N0, 0, N0, N0, 1, N0, 0, 2, 2, 256, 64, 0,
                                      *s[:6], None) == nat.SA_OK
    dec = [N0] * 8 + [0, 8, 2, 64, 16, 3, 2, 4, 2, 0, 0] + s[:7] + [N0, 0, 1, None]
    assert lib.sa_sparse_paged_decode(*dec) == nat.SA_OK
    assert lib.sa_block_sparse_bwd_plan_bytes(0, 2, 2, 64, 64, 1) == 0


def test_routed_fwd_argument_errors():
    lib = nat.lib()
    p = ctypes.c_void_p(256)

    def call(router_dtype=3, TD=3, depth=2, base=4, local=0, Z=1, H=2, N=1024, D=128, rb=128, dtype=1):
        rs = (ctypes.c_int64 * 4)(H * 400 * TD, 400 * TD, TD, 1)
        qs = (ctypes.c_int64 * 4)(H * N * D, N * D, D, 1)      # contiguous (Z, H, N, D)
        return lib.sa_routed_block_sparse_fwd(p, p, p, p, None, p, router_dtype, rs, TD, None, depth, base, 1,
                                              local, p, p, Z, H, H, N, D, rb, qs, qs, qs, qs, 0.1, dtype, 1, None)
    assert call(router_dtype=0) == nat.SA_EINVAL          # float router ids
    assert call(TD=0) == nat.SA_EINVAL
    assert call(depth=4) == nat.SA_EINVAL                 # depth beyond TD
    assert call(base=1) == nat.SA_EINVAL
    assert call(local=-1) == nat.SA_EINVAL
    assert call(dtype=0) == nat.SA_EUNSUPPORTED           # fp32: the MFMA path only
    assert call(N=40000) == nat.SA_EUNSUPPORTED           # NB = 313 > 256 key blocks per workgroup
    assert b"NB" in lib.sa_last_error()
    assert call(Z=0) == nat.SA_OK                         # empty problem: no launch
