"""Sparse paged decode oracle — test infrastructure only.

Restates ``_ultrametric_decode_reference`` (src/ultrametric/kernel_decode.py:129-185)
in float64 numpy, with:
  * ctx_len <= 0 -> zeros (kernel_decode.py:145-147; the Triton kernel leaves
    such rows unwritten, :50-51, so the CPU reference defines them);
  * r = clamp(req_depth, 0, TD) (kernel_decode.py:141);
  * selection on the PHYSICAL page's routing vector (kernel_decode.py:149-152,
    :76-81), sink = logical page 0, local = last local_blocks logical pages
    (:154-157, :88-89);
  * GQA by head grouping: k/v caches carry H_kv heads and query head h reads
    kv head h // (H / H_kv) — equal to calling the reference with the caches
    repeat_interleave'd to H heads.

Pinned by (tests/test_oracle_decode.py): req_depth = 0 with no sink/local
equals dense paged attention over the concatenated valid tokens (the loop of
benchmarks/benchmark_serving.py:11-73 restated in pure Python), ctx = 0 gives
zeros, a sequence of one page with one token returns that token's V row,
and GQA equals the H_kv = H call on repeated caches.
"""

from __future__ import annotations

import math

import numpy as np


def decode_reference(q, k_cache, v_cache, block_tables, context_lens, router, q_router,
                     req_depth, local_blocks=0, sink_block=False):
    """kernel_decode.py:129-185 (+ GQA grouping), float64. Returns (B, H, D) float64."""
    B, H, D = q.shape
    Hkv = k_cache.shape[1]
    group = H // Hkv
    tree_depth = q_router.shape[-1]
    r = min(max(int(req_depth), 0), tree_depth)
    page = k_cache.shape[2]
    scale = 1.0 / math.sqrt(D)
    out = np.zeros((B, H, D), dtype=np.float64)
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        n = (ctx + page - 1) // page
        phys = block_tables[b, :n].astype(np.int64)
        for h in range(H):
            if r > 0:
                match = (router[phys, h, :r] == q_router[b, h, :r][None, :]).all(-1)
            else:
                match = np.ones(n, dtype=bool)
            if sink_block and n > 0:
                match[0] = True
            if local_blocks > 0:
                match[max(0, n - local_blocks):] = True
            if not match.any():
                continue
            kh = h // group
            ks, vs = [], []
            for l in range(n):
                if match[l]:
                    valid = min(page, ctx - l * page)
                    ks.append(k_cache[phys[l], kh, :valid].astype(np.float64))
                    vs.append(v_cache[phys[l], kh, :valid].astype(np.float64))
            kc = np.concatenate(ks, 0)
            vc = np.concatenate(vs, 0)
            s = kc @ q[b, h].astype(np.float64) * scale
            w = np.exp(s - s.max())
            out[b, h] = (w / w.sum()) @ vc
    return out


def routed_page_bytes(block_tables, context_lens, router, q_router, H_kv, page_size, head_dim,
                      elem_bytes, req_depth, local_blocks=0, sink_block=False):
    """Algorithmic decode bytes: each (sequence, kv head, physical page) selected by any
    query head of the group counts once, valid tokens x D x (K and V) x elem_bytes.
    Also returns the number of such unique pages."""
    B = len(context_lens)
    H = router.shape[1]
    group = H // H_kv
    tree_depth = q_router.shape[-1]
    r = min(max(int(req_depth), 0), tree_depth)
    total_tokens = 0
    pages = 0
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        n = (ctx + page_size - 1) // page_size
        phys = block_tables[b, :n].astype(np.int64)
        valid = np.minimum(page_size, ctx - np.arange(n) * page_size)
        forced = np.zeros(n, dtype=bool)
        if sink_block:
            forced[0] = True
        if local_blocks > 0:
            forced[max(0, n - local_blocks):] = True
        for g in range(H_kv):
            sel = forced.copy()
            for h in range(g * group, (g + 1) * group):
                if r > 0:
                    sel |= (router[phys, h, :r] == q_router[b, h, :r][None, :]).all(-1)
                else:
                    sel[:] = True
            total_tokens += int(valid[sel].sum())
            pages += int(sel.sum())
    return total_tokens * head_dim * 2 * elem_bytes, pages


def dense_paged_loop(q, k_cache, v_cache, block_tables, context_lens):
    """Pure-Python dense paged attention (benchmarks/benchmark_serving.py:11-73 with every
    page selected), for pinning decode_reference at req_depth = 0."""
    B, H, D = q.shape
    page = k_cache.shape[2]
    group = H // k_cache.shape[1]
    scale = 1.0 / math.sqrt(D)
    out = [[[0.0] * D for _ in range(H)] for _ in range(B)]
    for b in range(B):
        ctx = int(context_lens[b])
        if ctx <= 0:
            continue
        for h in range(H):
            scores, rows = [], []
            for t in range(ctx):
                pg = int(block_tables[b][t // page])
                krow = k_cache[pg][h // group][t % page]
                scores.append(sum(float(a) * float(c) for a, c in zip(q[b][h], krow)) * scale)
                rows.append(v_cache[pg][h // group][t % page])
            mx = max(scores)
            w = [math.exp(s - mx) for s in scores]
            tot = sum(w)
            out[b][h] = [sum(wi * float(r[d]) for wi, r in zip(w, rows)) / tot for d in range(D)]
    return np.array(out)


def pack_codes(router, bits_per_level):
    """Packed routing code per (row, head): level l in bits [bpl*(TD-1-l), bpl*(TD-l)).

    No reference counterpart (the reference decode compares int32 levels one by
    one, kernel_decode.py:76-81); this states the packing that the packed decode
    entry point consumes. Pinned by brute force (tests/test_oracle_decode.py):
    for every depth r, the top bpl*r bits of two codes agree iff the first r
    levels agree, and unpacking recovers every level.
    """
    router = np.asarray(router, dtype=np.int64)
    td = router.shape[-1]
    assert 1 <= bits_per_level <= 16 and td * bits_per_level <= 32
    assert (router >= 0).all() and (router < (1 << bits_per_level)).all()
    code = np.zeros(router.shape[:-1], dtype=np.uint64)
    for lev in range(td):
        code = (code << np.uint64(bits_per_level)) | router[..., lev].astype(np.uint64)
    return code.astype(np.uint32)


def prefix_mask(tree_depth, bits_per_level, req_depth):
    """uint32 mask of the top bits_per_level * r bits, r = clamp(req_depth, 0, TD)."""
    r = min(max(int(req_depth), 0), tree_depth)
    if r == 0:
        return np.uint32(0)
    shift = bits_per_level * (tree_depth - r)
    return np.uint32((0xFFFFFFFF << shift) & 0xFFFFFFFF)
