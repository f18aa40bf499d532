"""Masked-dense attention oracle — test infrastructure only.

Restates, on the CPU:
  * ``token_mask_from_blocks``     src/ultrametric/block_list.py:361-368
  * ``masked_reference_attention`` src/ultrametric/block_list.py:371-378, in
    float64 (numpy), also returning the natural-log LSE of the scaled masked
    scores that _block_list_fwd_kernel stores (block_list.py:463-470);
    rows with no visible key give out = 0 and lse = -inf (block_list.py:463-470,
    kernel.py:577-579 nan_to_num).
  * the query-chunked evaluation of benchmarks/benchmark_block_list.py:105-123,
    so that N = 8192 never materialises an (N, N) mask per head at once.
  * GQA by head grouping: query head h reads kv head h // (H / H_kv), the
    same as repeat_kv (src/llama_surgery/surgery.py:77-86) followed by the
    reference call.
  * ``masked_attention_torch_fp32`` — the reference's own fp32 torch
    formulation (block_list.py:371-378, chunked as benchmark_block_list.py:105-123)
    used only as the timed CPU baseline.

Pinned by (tests/test_oracle_attention.py): a pure-Python per-row loop with
math.exp on tiny inputs, and closed forms — a single visible key returns its
V row, identical keys return the mean of the visible V rows, causal row 0
returns v0 with lse = q0.k0*scale, an empty row returns 0 / -inf.
"""

from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np


def token_mask_from_blocks(block_mask: np.ndarray, route_block: int, seq_len: int,
                           is_causal: bool = False) -> np.ndarray:
    """block_list.py:361-368 — (..., NB, NB) block mask -> (..., N, N) token mask."""
    m = np.repeat(np.repeat(block_mask, route_block, axis=-2), route_block, axis=-1)
    m = m[..., :seq_len, :seq_len]
    if is_causal:
        m = m & np.tril(np.ones((seq_len, seq_len), dtype=bool))
    return m


def _rows_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray,
                    scale: float, bias: Optional[np.ndarray] = None) -> Tuple[np.ndarray, np.ndarray]:
    """float64 softmax(q k^T * scale + bias, masked) v and natural LSE for a row chunk."""
    if k.shape[0] == 0:
        return np.zeros((q.shape[0], v.shape[-1])), np.full(q.shape[0], -np.inf)
    s = (q @ k.T) * scale
    if bias is not None:
        s = s + bias
    s = np.where(mask, s, -np.inf)
    m = s.max(-1, keepdims=True)
    m_safe = np.where(np.isfinite(m), m, 0.0)
    e = np.exp(s - m_safe)
    l = e.sum(-1, keepdims=True)
    out = np.where(l > 0, (e @ v) / np.where(l > 0, l, 1.0), 0.0)
    with np.errstate(divide="ignore"):
        lse = np.where(l[:, 0] > 0, np.log(np.where(l[:, 0] > 0, l[:, 0], 1.0)) + m_safe[:, 0], -np.inf)
    return out, lse


def block_sparse_attention_ref(q: np.ndarray, k: np.ndarray, v: np.ndarray, block_mask: np.ndarray,
                               route_block: int, *, is_causal: bool = False,
                               sm_scale: Optional[float] = None,
                               pair_bias: Optional[np.ndarray] = None,
                               heads: Optional[list] = None) -> Tuple[np.ndarray, np.ndarray]:
    """Masked-dense attention over a block mask, float64.

    Each query route block attends the tokens of its active key blocks only;
    columns outside them are -inf in the masked-dense formulation
    (block_list.py:371-378) and contribute exp(-inf) = 0, so gathering the
    active columns gives the same softmax at the cost of the active pairs.
    (Pinned against ``masked_attention`` with the full token mask.)

    q: (Z, H, N, D); k, v: (Z, H_kv, N, D); block_mask: (Z, H, NB, NB) bool;
    pair_bias: optional (Z, H, NB, NB) additive logit bias per block pair
    (the soft_block_bias of a listed pair, block_list.py:431-447).
    heads: optional list of (z, h) to evaluate (others stay 0 / -inf).
    Returns (out float64 (Z, H, N, D), lse float64 (Z, H, N)).
    """
    Z, H, N, D = q.shape
    Hkv = k.shape[1]
    group = H // Hkv
    NB = block_mask.shape[-1]
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    out = np.zeros((Z, H, N, D), dtype=np.float64)
    lse = np.full((Z, H, N), -np.inf, dtype=np.float64)
    todo = heads if heads is not None else [(z, h) for z in range(Z) for h in range(H)]
    for z, h in todo:
        kh = h // group
        kf = k[z, kh].astype(np.float64)
        vf = v[z, kh].astype(np.float64)
        for qb in range(NB):
            r0, r1 = qb * route_block, min(N, (qb + 1) * route_block)
            if r0 >= N:
                break
            kbs = np.nonzero(block_mask[z, h, qb])[0]
            cols = np.concatenate([np.arange(kb * route_block, min(N, (kb + 1) * route_block))
                                   for kb in kbs]) if kbs.size else np.zeros(0, np.int64)
            cols = cols[cols < N]
            rows = np.arange(r0, r1)
            m = np.ones((rows.size, cols.size), dtype=bool)
            if is_causal:
                m &= rows[:, None] >= cols[None, :]
            bias = None
            if pair_bias is not None and cols.size:
                bias = pair_bias[z, h, qb][cols // route_block][None, :].astype(np.float64)
            o, l = _rows_attention(q[z, h, r0:r1].astype(np.float64), kf[cols], vf[cols], m, scale, bias)
            out[z, h, r0:r1] = o
            lse[z, h, r0:r1] = l
    return out, lse


def block_sparse_attention_grad_ref(q: np.ndarray, k: np.ndarray, v: np.ndarray, block_mask: np.ndarray,
                                    route_block: int, dout: np.ndarray, *, is_causal: bool = False,
                                    sm_scale: Optional[float] = None,
                                    pair_bias: Optional[np.ndarray] = None,
                                    out: Optional[np.ndarray] = None):
    """Gradients of ``block_sparse_attention_ref``'s output, float64
    (the analytic backward of block_list.py:494-681,758-880):
    with P = softmax(S) over the visible columns of a row,
      dV += P^T dO, dS = P * (dO V^T - rowsum(dO * O)),
      dQ += scale dS K, dK += scale dS^T Q,
    and the gradient of the per-block-pair logit bias is the sum of dS over
    the pair. k / v may carry H_kv | H heads (their gradients sum over the
    query heads that read them).
    Returns (dq, dk, dv, d_pair_bias (Z, H, NB, NB)) as float64.
    ``out``: the forward output as the forward stored it (e.g. rounded to
    bf16). When given, delta = rowsum(dO * out) is taken from it, as the
    reference's backward does (block_list.py:784-785); otherwise from the
    exact float64 output. The two differ by the output's rounding, which
    matters for sums of dS that cancel exactly (a bias gradient over a row
    whose visible keys all lie in one block is 0 with the exact output).
    """
    Z, H, N, D = q.shape
    Hkv = k.shape[1]
    group = H // Hkv
    NB = block_mask.shape[-1]
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    dq = np.zeros((Z, H, N, D))
    dk = np.zeros((Z, Hkv, N, D))
    dv = np.zeros((Z, Hkv, N, D))
    dpb = np.zeros((Z, H, NB, NB))
    for z in range(Z):
        for h in range(H):
            kh = h // group
            kf = k[z, kh].astype(np.float64)
            vf = v[z, kh].astype(np.float64)
            for qb in range(NB):
                r0, r1 = qb * route_block, min(N, (qb + 1) * route_block)
                if r0 >= N:
                    break
                kbs = np.nonzero(block_mask[z, h, qb])[0]
                if kbs.size == 0:
                    continue
                cols = np.concatenate([np.arange(kb * route_block, min(N, (kb + 1) * route_block)) for kb in kbs])
                cols = cols[cols < N]
                if cols.size == 0:
                    continue
                rows = np.arange(r0, r1)
                m = np.ones((rows.size, cols.size), dtype=bool)
                if is_causal:
                    m &= rows[:, None] >= cols[None, :]
                qf = q[z, h, r0:r1].astype(np.float64)
                s = qf @ kf[cols].T * scale
                if pair_bias is not None:
                    s = s + pair_bias[z, h, qb][cols // route_block][None, :].astype(np.float64)
                s = np.where(m, s, -np.inf)
                mx = s.max(-1, keepdims=True)
                mx = np.where(np.isfinite(mx), mx, 0.0)
                e = np.where(m, np.exp(s - mx), 0.0)
                den = e.sum(-1, keepdims=True)
                pm = np.where(den > 0, e / np.where(den > 0, den, 1.0), 0.0)
                do = dout[z, h, r0:r1].astype(np.float64)
                o = pm @ vf[cols] if out is None else out[z, h, r0:r1].astype(np.float64)
                dp = do @ vf[cols].T
                ds = pm * (dp - (do * o).sum(-1, keepdims=True))
                dq[z, h, r0:r1] += scale * ds @ kf[cols]
                np.add.at(dk[z, kh], cols, scale * ds.T @ qf)
                np.add.at(dv[z, kh], cols, pm.T @ do)
                colb = cols // route_block
                for kb in kbs:
                    dpb[z, h, qb, kb] += ds[:, colb == kb].sum()
    return dq, dk, dv, dpb


def masked_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, token_mask: np.ndarray,
                     sm_scale: Optional[float] = None) -> Tuple[np.ndarray, np.ndarray]:
    """block_list.py:371-378 with an explicit (Z, H, N, N) token mask, float64."""
    Z, H, N, D = q.shape
    group = H // k.shape[1]
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    out = np.zeros((Z, H, N, D))
    lse = np.full((Z, H, N), -np.inf)
    for z in range(Z):
        for h in range(H):
            o, l = _rows_attention(q[z, h].astype(np.float64), k[z, h // group].astype(np.float64),
                                   v[z, h // group].astype(np.float64), token_mask[z, h], scale)
            out[z, h], lse[z, h] = o, l
    return out, lse


def masked_attention_torch_fp32(q, k, v, block_mask, route_block: int, is_causal: bool,
                                chunk: int = 2048):
    """The reference's fp32 masked-dense formulation on CPU torch (CPU baseline only).

    block_list.py:371-378 (matmul, masked_fill(-inf), softmax, matmul) evaluated
    per head and per query chunk as benchmarks/benchmark_block_list.py:105-123.
    q: (H, N, D) torch tensor; k, v: (H_kv, N, D); block_mask: (H, NB, NB) bool.
    """
    import torch

    H, N, D = q.shape
    group = H // k.shape[0]
    scale = 1.0 / math.sqrt(D)
    col_blk = torch.arange(N) // route_block
    cols = torch.arange(N)
    out = torch.empty(H, N, D, dtype=torch.float32)
    for h in range(H):
        kf = k[h // group].float()
        vf = v[h // group].float()
        for s0 in range(0, N, chunk):
            e0 = min(N, s0 + chunk)
            rows = torch.arange(s0, e0)
            sc = torch.matmul(q[h, s0:e0].float(), kf.transpose(-2, -1)) * scale
            m = block_mask[h][rows // route_block][:, col_blk]
            if is_causal:
                m = m & (rows[:, None] >= cols[None, :])
            sc = sc.masked_fill(~m, float("-inf"))
            out[h, s0:e0] = torch.matmul(torch.softmax(sc, dim=-1), vf)
    return out


def brute_force_row(qrow, keys, vals, visible, scale):
    """Pure-Python softmax-weighted average for one query row (pinning only)."""
    scores = [sum(a * b for a, b in zip(qrow, keys[j])) * scale for j in range(len(keys)) if visible[j]]
    idx = [j for j in range(len(keys)) if visible[j]]
    if not idx:
        return [0.0] * len(qrow), -math.inf
    mx = max(scores)
    ws = [math.exp(s - mx) for s in scores]
    tot = sum(ws)
    out = [sum(w * vals[j][d] for w, j in zip(ws, idx)) / tot for d in range(len(qrow))]
    return out, mx + math.log(tot)
