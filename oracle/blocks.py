"""Block-list oracle (numpy) — test infrastructure only.

Restates, on the CPU:
  * ``_depth_tensor``            src/ultrametric/block_list.py:93-104
  * ``_apply_structural_masks``  src/ultrametric/block_list.py:107-118
  * ``build_block_lists``        src/ultrametric/block_list.py:170-278
    (code semantics :211-229, element-wise path :256-258, compaction :263-278)
  * ``build_transposed_block_lists`` src/ultrametric/block_list.py:281-327
  * ``block_mask_reference``     src/ultrametric/block_list.py:334-358

Pinned by (tests/test_oracle_blocks.py): a pure-Python brute force over
(i, j) pairs on tiny inputs (independent of the vectorised code path here),
the reference's known-answer tests (tests/test_block_list.py:50-70,131-183:
depth 0 is dense, causal counts 1..NB, a binary tree router at depth r keeps
NB/2^r blocks per row and is block-diagonal at full depth, the diagonal is
always listed, sync-free == syncing on the valid prefix), and the code-alias
rule of the sync-free mode read from block_list.py:212-229.
"""

from __future__ import annotations

import math
from typing import NamedTuple, Optional, Sequence, Union

import numpy as np

DepthLike = Union[int, Sequence[int], np.ndarray]


class BlockListsNP(NamedTuple):
    lists: np.ndarray   # (Z, H, NB, max_count) int32, ascending, zero padded
    counts: np.ndarray  # (Z, H, NB) int32
    max_count: int


def depth_array(req_depth: DepthLike, num_heads: int, tree_depth: int) -> np.ndarray:
    """block_list.py:93-104 — int or per-head depths -> validated (H,) int64."""
    if isinstance(req_depth, (int, np.integer)):
        depth = np.full((num_heads,), int(req_depth), dtype=np.int64)
    else:
        depth = np.asarray(req_depth, dtype=np.int64).reshape(-1)
        if depth.size != num_heads:
            raise ValueError(f"req_depth has {depth.size} entries, expected {num_heads}")
    if depth.size and (depth.min() < 0 or depth.max() > tree_depth):
        raise ValueError(f"req_depth must be in [0, {tree_depth}]")
    return depth


def apply_structural_masks(match: np.ndarray, *, is_causal: bool, sink_block: bool,
                           local_blocks: int) -> np.ndarray:
    """block_list.py:107-118 — local band OR, then sink column OR, then causal AND."""
    nb = match.shape[-1]
    idx = np.arange(nb)
    match = match.copy()
    if local_blocks > 0:
        match |= np.abs(idx[:, None] - idx[None, :]) <= local_blocks
    if sink_block:
        match[..., 0] = True
    if is_causal:
        match &= idx[:, None] >= idx[None, :]
    return match


def compact(match: np.ndarray, max_count: int) -> BlockListsNP:
    """block_list.py:263-278 — k-th active key block of a row to slot k, zeros after."""
    Z, H, NB, NB2 = match.shape
    counts = match.sum(-1).astype(np.int32)
    lists = np.zeros((Z, H, NB, max_count), dtype=np.int32)
    zz, hh, ii, jj = np.nonzero(match)          # row-major => ascending j per row
    pos = np.cumsum(match, axis=-1)[zz, hh, ii, jj] - 1
    keep = pos < max_count
    lists[zz[keep], hh[keep], ii[keep], pos[keep]] = jj[keep]
    return BlockListsNP(lists, counts, int(max_count))


def routing_match(router: np.ndarray, req_depth: DepthLike, *, arity: Optional[int] = None) -> np.ndarray:
    """Block-pair match of build_block_lists before structural masks (block_list.py:196-258).

    Codes: base = max(2, arity) when sync-free, else max(2, max(id)+1); a block's
    code is sum_l id_l * [l < depth_h] * base^l in wrapping int64 arithmetic
    (the reference's torch int64 ops); used iff TD*log2(base) < 62, otherwise
    the first depth_h levels are compared element-wise.
    """
    Z, H, NB, TD = router.shape
    r = router.astype(np.int64)
    sync_free = arity is not None
    if sync_free and isinstance(req_depth, (int, np.integer)):
        if not 0 <= int(req_depth) <= TD:
            raise ValueError(f"req_depth must be in [0, {TD}]")
        depth = np.full((H,), int(req_depth), dtype=np.int64)
    else:
        depth = depth_array(req_depth, H, TD)
    if sync_free:
        base = max(2, int(arity))
    else:
        if r.size and r.min() < 0:
            raise ValueError("router_indices must be non-negative branch ids")
        base = max(2, int(r.max()) + 1) if r.size else 2
    keep = np.arange(TD)[None, :] < depth[:, None]              # (H, TD)
    if TD * math.log2(base) < 62:
        powers = np.array([base ** l for l in range(TD)], dtype=np.uint64)
        terms = r.astype(np.uint64) * keep[None, :, None, :].astype(np.uint64) * powers
        code = terms.sum(-1, dtype=np.uint64)                    # wraps mod 2^64
        return code[..., :, None] == code[..., None, :]
    eq = (r[:, :, :, None, :] == r[:, :, None, :, :]) | ~keep[None, :, None, None, :]
    return eq.all(-1)


def build_block_lists(router: np.ndarray, req_depth: DepthLike, *, is_causal: bool = False,
                      sink_block: bool = False, local_blocks: int = 0,
                      arity: Optional[int] = None) -> BlockListsNP:
    """block_list.py:170-278 — routing vectors -> BlockLists (sync-free iff arity given)."""
    if router.ndim != 4:
        raise ValueError("router_indices must be (Z, H, NB, TD)")
    NB = router.shape[2]
    match = routing_match(router, req_depth, arity=arity)
    match = apply_structural_masks(match, is_causal=is_causal, sink_block=sink_block,
                                   local_blocks=local_blocks)
    counts = match.sum(-1)
    max_count = NB if arity is not None else (int(counts.max()) if counts.size else 0)
    return compact(match, max_count)


def block_lists_from_mask(mask: np.ndarray, *, is_causal: bool = False, sink_block: bool = False,
                          local_blocks: int = 0, sync_free: bool = True) -> BlockListsNP:
    """Compaction of a given block mask (block_list.py:263-278 applied to `match`)."""
    match = apply_structural_masks(mask.astype(bool), is_causal=is_causal, sink_block=sink_block,
                                   local_blocks=local_blocks)
    NB = match.shape[-1]
    counts = match.sum(-1)
    max_count = NB if sync_free else (int(counts.max()) if counts.size else 0)
    return compact(match, max_count)


def block_mask_reference(router: np.ndarray, req_depth: DepthLike, *, is_causal: bool = False,
                         sink_block: bool = False, local_blocks: int = 0) -> np.ndarray:
    """block_list.py:334-358 — explicit per-head prefix comparison, then structural masks."""
    Z, H, NB, TD = router.shape
    depth = depth_array(req_depth, H, TD)
    out = np.empty((Z, H, NB, NB), dtype=bool)
    for h, d in enumerate(depth.tolist()):
        if d == 0:
            out[:, h] = True
        else:
            rh = router[:, h, :, :d]
            out[:, h] = (rh[:, :, None, :] == rh[:, None, :, :]).all(-1)
    return apply_structural_masks(out, is_causal=is_causal, sink_block=sink_block,
                                  local_blocks=local_blocks)


def lists_to_mask(lists: np.ndarray, counts: np.ndarray, num_key_blocks: Optional[int] = None) -> np.ndarray:
    """Dense (Z, H, NB_Q, NB_K) bool mask of the listed pairs (first counts[row] entries)."""
    Z, H, NB = counts.shape
    NBK = NB if num_key_blocks is None else num_key_blocks
    mask = np.zeros((Z, H, NB, NBK), dtype=bool)
    if lists.shape[-1] == 0:
        return mask
    t = np.arange(lists.shape[-1])
    valid = t[None, None, None, :] < counts[..., None]
    zz, hh, ii, tt = np.nonzero(valid)
    mask[zz, hh, ii, lists[zz, hh, ii, tt]] = True
    return mask


def build_transposed_block_lists(lists: np.ndarray, counts: np.ndarray,
                                 num_key_blocks: Optional[int] = None) -> BlockListsNP:
    """block_list.py:281-327 — per key block, the ascending query blocks that list it."""
    Z, H, NBQ = counts.shape
    NBK = NBQ if num_key_blocks is None else num_key_blocks
    if NBQ == 0 or NBK == 0 or lists.shape[-1] == 0:
        return BlockListsNP(np.zeros((Z, H, NBK, 0), np.int32), np.zeros((Z, H, NBK), np.int32), 0)
    m_kq = np.swapaxes(lists_to_mask(lists, counts, NBK), -1, -2)
    qc = m_kq.sum(-1)
    return compact(m_kq, int(qc.max()) if qc.size else 0)
