"""Ternary packed-KV prefill oracle — test infrastructure only.

Restates, in float64 numpy:
  * ternary_quantize (src/llama_surgery/surgery.py:15-28): gamma = mean |x| per
    row, values > gamma/2 -> +1, < -gamma/2 -> -1, else 0; returns
    (ternary, gamma);
  * pack_ternary / unpack_ternary (surgery.py:35-76): 16 values per int32,
    value i in bits [2i, 2i + 2), code 0 -> 0, 1 -> +1, 2 -> -1;
  * _ternary_ultrametric_fwd_kernel (src/llama_surgery/kernel.py:147-249) with
    its launcher (:348-420): causal attention over 128-token blocks; key block
    n <= m is visited iff the routing vectors of blocks m and n agree on the
    first req_depth levels, or n == 0 (sink), or m - n <= ceil(local_window /
    128) (local); k = unpack(K) * k_scale (per key row), v = unpack(V) *
    v_scale; keys j are visible to query i iff j <= i and both lie on the same
    side of N - shift_size; scale 1/sqrt(D); router rows past its length are
    zero (the launcher's padding).
Divergence, on purpose: a row whose first visited block has no visible key
makes the reference's online softmax produce NaN (exp(-inf - -inf), :222-225);
the restatement uses the all-masked guard of block_list.py:455-461 instead and
returns the softmax over the row's visible keys.

Pinned by (tests/test_oracle_ternary.py): pack/unpack round trip and the bit
layout on hand-made words; the quantizer on closed-form rows; with unit
scales and shift_size = 0 the attention equals oracle.attention's
block-sparse reference on the unpacked K / V with the same block mask; a
shifted sequence equals two independent calls on the two regions; a query
whose only visible key is itself returns that key's scaled V row.
"""

from __future__ import annotations

import math

import numpy as np


def ternary_quantize(x):
    """surgery.py:15-28 forward: (ternary in {-1, 0, 1}, gamma (..., 1)) in float64."""
    x = np.asarray(x, dtype=np.float64)
    gamma = np.abs(x).mean(-1, keepdims=True)
    thr = 0.5 * gamma
    t = np.zeros_like(x)
    t[x > thr] = 1.0
    t[x < -thr] = -1.0
    return t, gamma


def pack_ternary(t):
    """surgery.py:35-55: (..., D) in {-1, 0, 1}, D % 16 == 0 -> (..., D / 16) int32."""
    t = np.asarray(t)
    assert t.shape[-1] % 16 == 0
    code = np.zeros(t.shape, dtype=np.uint32)
    code[t == 1] = 1
    code[t == -1] = 2
    code = code.reshape(*t.shape[:-1], t.shape[-1] // 16, 16)
    word = np.zeros(code.shape[:-1], dtype=np.uint32)
    for i in range(16):
        word |= code[..., i] << np.uint32(2 * i)
    return word.view(np.int32)


def unpack_ternary(packed, D):
    """surgery.py:57-76 (code 3 is read as 3, as the kernel's k_val.to(float) does)."""
    w = np.asarray(packed).view(np.uint32)
    vals = np.stack([(w >> np.uint32(2 * i)) & np.uint32(3) for i in range(16)], -1).astype(np.float64)
    vals = vals.reshape(*w.shape[:-1], D)
    vals[vals == 2] = -1.0
    return vals


def block_selection(router, req_depth, local_window, NB):
    """(Z, H, NB, NB) bool: the visited (m, n) block pairs, n <= m (kernel.py:197-208)."""
    Z, H, nr, TD = router.shape
    r = np.zeros((Z, H, NB, TD), dtype=np.int64)
    r[:, :, :min(nr, NB)] = router[:, :, :NB]
    lw = math.ceil(local_window / 128)
    d = min(max(int(req_depth), 0), TD)
    sel = np.zeros((Z, H, NB, NB), dtype=bool)
    for m in range(NB):
        for n in range(m + 1):
            match = (r[:, :, m, :d] == r[:, :, n, :d]).all(-1)
            sel[:, :, m, n] = match | (n == 0) | ((m - n) <= lw)
    return sel


def ternary_attention_ref(q, k_packed, v_packed, k_scale, v_scale, router, local_window=128, req_depth=2,
                          shift_size=0):
    """float64 (Z, H, N, D) output of the ternary prefill (see module doc)."""
    q = np.asarray(q, dtype=np.float64)
    Z, H, N, D = q.shape
    NB = math.ceil(N / 128)
    k = unpack_ternary(k_packed, D) * np.asarray(k_scale, dtype=np.float64)[..., None]
    v = unpack_ternary(v_packed, D) * np.asarray(v_scale, dtype=np.float64)[..., None]
    sel = block_selection(np.asarray(router), req_depth, local_window, NB)
    pos = np.arange(N)
    region = pos >= N - shift_size
    vis_tok = (pos[:, None] >= pos[None, :]) & (region[:, None] == region[None, :])
    scale = 1.0 / math.sqrt(D)
    out = np.zeros((Z, H, N, D))
    for z in range(Z):
        for h in range(H):
            blk = np.repeat(np.repeat(sel[z, h], 128, 0), 128, 1)[:N, :N]
            vis = vis_tok & blk
            s = q[z, h] @ k[z, h].T * scale
            s = np.where(vis, s, -np.inf)
            mx = s.max(-1, keepdims=True)
            mx = np.where(np.isfinite(mx), mx, 0.0)
            w = np.where(vis, np.exp(s - mx), 0.0)
            den = w.sum(-1, keepdims=True)
            out[z, h] = np.where(den > 0, (w @ v[z, h]) / np.where(den > 0, den, 1.0), 0.0)
    return out
