"""Pins oracle/ternary.py (see its header): packing layout and round trip,
the quantizer, reduction to the block-sparse attention oracle, the shift
regions, and a single-visible-key closed form."""

import math

import numpy as np

from oracle import attention as oa
from oracle import ternary as ot


def test_pack_layout_and_round_trip():
    t = np.zeros(16)
    t[0], t[1], t[15] = 1, -1, 1
    w = ot.pack_ternary(t[None])[0, 0]
    assert int(np.uint32(w)) == (1 | (2 << 2) | (1 << 30))
    rng = np.random.default_rng(0)
    x = rng.integers(-1, 2, (3, 5, 64)).astype(np.float64)
    assert np.array_equal(ot.unpack_ternary(ot.pack_ternary(x), 64), x)
    # code 3 (never written by pack) reads as 3
    assert ot.unpack_ternary(np.array([[3]], dtype=np.int32), 16)[0, 0] == 3


def test_quantizer_closed_form():
    x = np.array([[4.0, -4.0, 0.5, -0.5, 1.5, -1.5, 0.0, 2.0]])
    t, g = ot.ternary_quantize(x)
    assert g[0, 0] == np.abs(x).mean()                # 1.75, threshold 0.875
    assert t.tolist() == [[1, -1, 0, 0, 1, -1, 0, 1]]


def _case(Z, H, N, D, seed, TD=3, p=2):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((Z, H, N, D))
    kt = rng.integers(-1, 2, (Z, H, N, D))
    vt = rng.integers(-1, 2, (Z, H, N, D))
    ks = rng.uniform(0.2, 1.5, (Z, H, N))
    vs = rng.uniform(0.2, 1.5, (Z, H, N))
    router = rng.integers(0, p, (Z, H, math.ceil(N / 128), TD))
    return q, kt, vt, ks, vs, router


def test_unit_scales_reduce_to_block_sparse_reference():
    q, kt, vt, _, _, router = _case(1, 2, 300, 32, 1)
    one = np.ones((1, 2, 300))
    got = ot.ternary_attention_ref(q, ot.pack_ternary(kt), ot.pack_ternary(vt), one, one, router,
                                   local_window=128, req_depth=2)
    sel = ot.block_selection(router, 2, 128, 3)
    want = oa.block_sparse_attention_ref(q, kt.astype(np.float64), vt.astype(np.float64), sel, 128,
                                         is_causal=True)[0]
    assert np.abs(got - want).max() < 1e-12


def test_scales_fold_into_k_and_v():
    q, kt, vt, ks, vs, router = _case(1, 1, 200, 16, 2)
    got = ot.ternary_attention_ref(q, ot.pack_ternary(kt), ot.pack_ternary(vt), ks, vs, router)
    sel = ot.block_selection(router, 2, 128, 2)
    want = oa.block_sparse_attention_ref(q, kt * ks[..., None], vt * vs[..., None], sel, 128, is_causal=True)[0]
    assert np.abs(got - want).max() < 1e-12


def test_shift_regions_are_independent():
    # every block visited (req_depth 0): the shifted tail attends only to itself,
    # causally, so the output equals two separate causal calls
    q, kt, vt, ks, vs, router = _case(1, 1, 256, 16, 3)
    kp, vp = ot.pack_ternary(kt), ot.pack_ternary(vt)
    got = ot.ternary_attention_ref(q, kp, vp, ks, vs, router, req_depth=0, shift_size=100)
    head = ot.ternary_attention_ref(q[:, :, :156], kp[:, :, :156], vp[:, :, :156], ks[:, :, :156], vs[:, :, :156],
                                    router, req_depth=0)
    k = kt * ks[..., None]
    v = vt * vs[..., None]
    qt, kk, vv = q[0, 0, 156:], k[0, 0, 156:], v[0, 0, 156:]
    s = qt @ kk.T / 4.0 + np.triu(np.full((100, 100), -np.inf), 1)
    w = np.exp(s - s.max(-1, keepdims=True))
    tail = (w / w.sum(-1, keepdims=True)) @ vv
    assert np.abs(got[0, 0, :156] - head[0, 0]).max() < 1e-12
    assert np.abs(got[0, 0, 156:] - tail).max() < 1e-12


def test_first_query_sees_only_itself():
    q, kt, vt, ks, vs, router = _case(1, 1, 128, 16, 4)
    got = ot.ternary_attention_ref(q, ot.pack_ternary(kt), ot.pack_ternary(vt), ks, vs, router)
    assert np.allclose(got[0, 0, 0], vt[0, 0, 0] * vs[0, 0, 0])
