"""Pins oracle/attention.py:block_sparse_attention_grad_ref (the analytic
backward of src/ultrametric/block_list.py:494-681,758-880) against torch
float64 autograd through the masked-dense formulation (block_list.py:371-378
with a token-level block bias, as tests/test_block_list.py:260-351 build their
reference) and against central finite differences on a tiny case."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import blocks as ob


def torch_reference_grads(q, k, v, bm, rb, dout, causal, pair_bias, group):
    N, D = q.shape[2], q.shape[3]
    qt, kt, vt = (torch.from_numpy(x).double().requires_grad_(True) for x in (q, k, v))
    pb = torch.from_numpy(pair_bias).double().requires_grad_(True)
    tm = torch.from_numpy(oa.token_mask_from_blocks(bm, rb, N, is_causal=causal))
    tb = pb.repeat_interleave(rb, -2).repeat_interleave(rb, -1)[..., :N, :N]
    kr = kt.repeat_interleave(group, 1)
    vr = vt.repeat_interleave(group, 1)
    s = qt @ kr.transpose(-1, -2) / math.sqrt(D) + tb
    s = s.masked_fill(~tm, float("-inf"))
    p = torch.softmax(s, -1).nan_to_num(0.0)
    (p @ vr).backward(torch.from_numpy(dout).double())
    return qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy(), pb.grad.numpy()


@pytest.mark.parametrize("N,rb,causal,H,Hkv", [(100, 32, True, 2, 2), (128, 64, False, 2, 1), (96, 32, True, 4, 2)])
def test_grad_ref_matches_torch_autograd(N, rb, causal, H, Hkv):
    rng = np.random.default_rng(N + H)
    Z, D = 1, 16
    q = rng.standard_normal((Z, H, N, D))
    k = rng.standard_normal((Z, Hkv, N, D))
    v = rng.standard_normal((Z, Hkv, N, D))
    dout = rng.standard_normal((Z, H, N, D))
    NB = -(-N // rb)
    router = rng.integers(0, 2, size=(Z, H, NB, 3), dtype=np.int32)
    bl = ob.build_block_lists(router, 1, is_causal=causal, sink_block=True)
    bm = ob.lists_to_mask(bl.lists, bl.counts)
    pair_bias = rng.standard_normal((Z, H, NB, NB)) * bm
    dq, dk, dv, dpb = oa.block_sparse_attention_grad_ref(q, k, v, bm, rb, dout, is_causal=causal,
                                                         pair_bias=pair_bias)
    tq, tk, tv, tpb = torch_reference_grads(q, k, v, bm, rb, dout, causal, pair_bias, H // Hkv)
    for a, b in ((dq, tq), (dk, tk), (dv, tv)):
        assert np.abs(a - b).max() < 1e-10
    assert np.abs((dpb - tpb) * bm).max() < 1e-10


def test_grad_ref_finite_differences():
    rng = np.random.default_rng(5)
    Z, H, N, D, rb = 1, 1, 20, 4, 8
    q, k, v, dout = (rng.standard_normal((Z, H, N, D)) for _ in range(4))
    NB = -(-N // rb)
    bm = np.tril(np.ones((NB, NB), dtype=bool))[None, None]
    bm[..., 2, 1] = False
    pb = rng.standard_normal((Z, H, NB, NB)) * bm
    dq, dk, dv, dpb = oa.block_sparse_attention_grad_ref(q, k, v, bm, rb, dout, is_causal=True, pair_bias=pb)

    def loss(q_, k_, v_, pb_):
        o, _ = oa.block_sparse_attention_ref(q_, k_, v_, bm, rb, is_causal=True, pair_bias=pb_)
        return float((o * dout).sum())

    eps = 1e-6
    for arr, grad in ((q, dq), (k, dk), (v, dv), (pb, dpb)):
        for idx in [(0, 0, 3, 1), (0, 0, 17, 2), (0, 0, 9, 0)] if arr.ndim == 4 and arr.shape[2] == N else \
                [(0, 0, 1, 0), (0, 0, 2, 2), (0, 0, 2, 0)]:
            a0 = arr[idx]
            arr[idx] = a0 + eps
            lp = loss(q, k, v, pb)
            arr[idx] = a0 - eps
            lm = loss(q, k, v, pb)
            arr[idx] = a0
            assert abs((lp - lm) / (2 * eps) - grad[idx]) < 1e-6, idx


def test_grad_ref_delta_from_stored_output():
    # `out` replaces the exact output in delta = rowsum(dO * out) (block_list.py:784-785).
    # With the exact output it changes nothing. With a perturbed one, sum_j dS_ij =
    # dO_i . O_i - delta_i = dO_i . (O_i - out_i): the bias gradient of a pair that holds
    # all of a row's visible keys (here: one block per row) is that sum over its rows.
    rng = np.random.default_rng(11)
    Z, H, N, D, rb = 1, 2, 24, 8, 8
    q, k, v, dout = (rng.standard_normal((Z, H, N, D)) for _ in range(4))
    NB = N // rb
    bm = np.broadcast_to(np.eye(NB, dtype=bool), (Z, H, NB, NB)).copy()
    o, _ = oa.block_sparse_attention_ref(q, k, v, bm, rb, is_causal=True)
    base = oa.block_sparse_attention_grad_ref(q, k, v, bm, rb, dout, is_causal=True)
    same = oa.block_sparse_attention_grad_ref(q, k, v, bm, rb, dout, is_causal=True, out=o)
    for a, b in zip(base, same):
        assert np.allclose(a, b, rtol=0, atol=1e-12)
    assert np.abs(base[3]).max() < 1e-12
    stored = o + rng.standard_normal(o.shape) * 1e-3
    dpb = oa.block_sparse_attention_grad_ref(q, k, v, bm, rb, dout, is_causal=True, out=stored)[3]
    for h in range(H):
        for qb in range(NB):
            r = slice(qb * rb, (qb + 1) * rb)
            want = float((dout[0, h, r] * (o[0, h, r] - stored[0, h, r])).sum())
            assert abs(dpb[0, h, qb, qb] - want) < 1e-12
