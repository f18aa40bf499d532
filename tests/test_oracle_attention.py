"""Pins the attention oracle (oracle/attention.py) on the CPU.

  * a pure-Python per-row loop (math.exp, explicit visibility test) on tiny
    inputs, against both the gathered block form and the full token-mask form;
  * closed forms: a single visible key returns its V row; identical keys
    return the mean of the visible V rows; causal row 0 returns v0 with
    lse = q0.k0*scale; a row with no visible key returns 0 / -inf;
  * the reference's fp32 torch formulation (the CPU baseline) agrees with the
    float64 oracle to fp32 rounding;
  * GQA by head grouping equals the repeated-K/V call.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import blocks as ob


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


@pytest.mark.parametrize("N,rb,depth,causal,sink,local", [
    (40, 16, 1, False, False, 0), (40, 16, 2, True, False, 0), (48, 16, 1, True, True, 1),
    (33, 16, 0, True, False, 0)])
def test_against_python_loop(N, rb, depth, causal, sink, local):
    Z, H, D = 1, 2, 8
    q, k, v = rnd((Z, H, N, D), 1), rnd((Z, H, N, D), 2), rnd((Z, H, N, D), 3)
    NB = -(-N // rb)
    router = np.random.default_rng(N).integers(0, 2, size=(Z, H, NB, 3))
    bm = ob.block_mask_reference(router, depth, is_causal=causal, sink_block=sink, local_blocks=local)
    out, lse = oa.block_sparse_attention_ref(q, k, v, bm, rb, is_causal=causal)
    tm = oa.token_mask_from_blocks(bm, rb, N, causal)
    out2, lse2 = oa.masked_attention(q, k, v, tm)
    scale = 1 / math.sqrt(D)
    for h in range(H):
        for i in range(N):
            vis = [bool(bm[0, h, i // rb, j // rb]) and (not causal or j <= i) for j in range(N)]
            o, l = oa.brute_force_row(q[0, h, i].tolist(), k[0, h].tolist(), v[0, h].tolist(), vis, scale)
            assert np.allclose(out[0, h, i], o, atol=1e-12)
            assert np.allclose(out2[0, h, i], o, atol=1e-12)
            assert (l == -math.inf and lse[0, h, i] == -math.inf) or abs(lse[0, h, i] - l) < 1e-12
            assert (l == -math.inf and lse2[0, h, i] == -math.inf) or abs(lse2[0, h, i] - l) < 1e-12


def test_closed_forms():
    Z, H, N, D, rb = 1, 1, 32, 4, 16
    q, v = rnd((Z, H, N, D), 4), rnd((Z, H, N, D), 5)
    k = np.tile(rnd((1, 1, 1, D), 6), (1, 1, N, 1))           # identical keys
    bm = np.zeros((1, 1, 2, 2), dtype=bool)
    bm[0, 0, 1, 0] = True                                      # row block 1 sees block 0 only
    out, lse = oa.block_sparse_attention_ref(q, k, v, bm, rb, is_causal=True)
    assert np.allclose(out[0, 0, :16], 0) and np.all(lse[0, 0, :16] == -np.inf)   # empty rows
    assert np.allclose(out[0, 0, 16:], v[0, 0, :16].mean(0))  # identical keys -> mean of V
    # causal row 0 with the diagonal block: out = v0, lse = q0.k0 * scale
    bm2 = np.ones((1, 1, 2, 2), dtype=bool)
    k2 = rnd((Z, H, N, D), 7)
    out2, lse2 = oa.block_sparse_attention_ref(q, k2, v, bm2, rb, is_causal=True)
    assert np.allclose(out2[0, 0, 0], v[0, 0, 0])
    assert abs(lse2[0, 0, 0] - q[0, 0, 0] @ k2[0, 0, 0] / 2.0) < 1e-12
    # single visible key (block of one token at the tail): N = 17, rb = 16
    q3, k3, v3 = rnd((1, 1, 17, D), 8), rnd((1, 1, 17, D), 9), rnd((1, 1, 17, D), 10)
    bm3 = np.zeros((1, 1, 2, 2), dtype=bool)
    bm3[0, 0, 0, 1] = True
    out3, _ = oa.block_sparse_attention_ref(q3, k3, v3, bm3, 16)
    assert np.allclose(out3[0, 0, :16], v3[0, 0, 16])


def test_pair_bias_shifts_blocks():
    Z, H, N, D, rb = 1, 1, 32, 4, 16
    q, k, v = rnd((Z, H, N, D), 11), rnd((Z, H, N, D), 12), rnd((Z, H, N, D), 13)
    bm = np.ones((1, 1, 2, 2), dtype=bool)
    bias = np.zeros((1, 1, 2, 2))
    bias[0, 0, :, 1] = -1e9                                     # kill block 1 via the bias
    out, _ = oa.block_sparse_attention_ref(q, k, v, bm, rb, pair_bias=bias)
    bm_only0 = bm.copy()
    bm_only0[0, 0, :, 1] = False
    ref, _ = oa.block_sparse_attention_ref(q, k, v, bm_only0, rb)
    assert np.allclose(out, ref)


def test_gqa_grouping_equals_repeat():
    Z, H, Hkv, N, D, rb = 1, 4, 2, 32, 8, 16
    q, k, v = rnd((Z, H, N, D), 14), rnd((Z, Hkv, N, D), 15), rnd((Z, Hkv, N, D), 16)
    bm = np.random.default_rng(0).random((Z, H, 2, 2)) < 0.7
    a, la = oa.block_sparse_attention_ref(q, k, v, bm, rb, is_causal=True)
    b, lb = oa.block_sparse_attention_ref(q, np.repeat(k, 2, axis=1), np.repeat(v, 2, axis=1), bm, rb,
                                          is_causal=True)
    assert np.array_equal(a, b) and np.array_equal(la, lb)


def test_torch_fp32_baseline_agrees():
    H, N, D, rb = 2, 256, 32, 64
    q, k, v = (torch.from_numpy(rnd((H, N, D), s)).float() for s in (17, 18, 19))
    bm = torch.from_numpy(np.random.default_rng(1).random((H, 4, 4)) < 0.5)
    idx = torch.arange(4)
    bm[:, idx, idx] = True
    out = oa.masked_attention_torch_fp32(q, k, v, bm, rb, True, chunk=100)
    ref, _ = oa.block_sparse_attention_ref(q.numpy()[None], k.numpy()[None], v.numpy()[None],
                                           bm.numpy()[None], rb, is_causal=True)
    assert np.abs(out.numpy() - ref[0]).max() < 1e-5
