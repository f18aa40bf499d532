"""Surgery-side block routing and prefill (the model caller of the hot path).

Mirrors ``SurgicalLlamaAttention._block_list_prefill``
(src/llama_surgery/surgery.py:521-601), the only model-side caller of the
block-list kernel in the reference, as free functions over the same inputs
(the reference reads them from its module and config):

* ``route_block_vote`` — one routing vector per route block: per level, the
  branch most of the block's tokens pick (token choice = argmax over the p
  branch scores, first maximum on ties; block winner = lowest branch id on
  ties; surgery.py:543-547), or with ``route_block = 1`` the per-row argmax of
  direct block assignments (surgery.py:536-541). One HIP kernel
  (``sa_route_block_vote``) replaces the reference's argmax / one_hot / pad /
  view / sum / argmax chain.
* ``block_list_prefill`` — the causal prefill: vote, sync-free list build with
  causal + sink + ceil(local_window / route_block) local blocks and
  arity = p (surgery.py:550-564), then ``block_list_attention`` with the
  caller's softmax scale (surgery.py:599-601). K / V may carry fewer heads
  (GQA): the kernel indexes kv head h // (H / H_kv) instead of materialising
  ``repeat_kv`` (surgery.py:77-86). Optional statistics follow
  surgery.py:589-595.

Gradients with respect to q, k and v flow through block_list_attention's
backward. When grad is enabled and the routing scores require grad, the
router's straight-through soft-bias term is built as the reference does
(surgery.py:566-588): block-mean assignments, their expected tree distance
(``expected_block_distance``, topology.py:456-485), soft logits
(max_dist - distance) / 0.5 gathered at each row's listed blocks, and the
zero-valued bias g - g.detach() passed to block_list_attention as
``soft_block_bias``; the kernel's backward returns its gradient, which
autograd carries to the scores.
"""

from __future__ import annotations

from typing import Optional

import torch

from . import _native as nat
from .block_list import block_list_attention, build_block_lists

__all__ = ["route_block_vote", "block_list_prefill", "local_blocks_of", "RouteCache", "expected_block_distance",
           "ste_soft_block_bias"]

_SCORE_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def local_blocks_of(local_window: int, route_block: int) -> int:
    """Local band in blocks for a token window (surgery.py:550-551)."""
    return -(-int(local_window) // int(route_block)) if local_window > 0 else 0


def expected_block_distance(block_assignments: torch.Tensor, p: int = 2) -> torch.Tensor:
    """(B, H, NB, L, p) soft branch probabilities -> (B, H, NB, NB) expected tree
    distance (topology.py:456-485): with m_l(i, j) = sum_p a_i[l, p] a_j[l, p] the
    chance that blocks i and j take the same branch at level l, the chance that
    they share levels 0..l is taken as min(m_0, ..., m_l), and the distance is
    L minus the sum of those over l. When the input requires grad, the backward
    also sees a tie-breaking term 0.05 * 2^(l - (L - 1)) * m_l per level (its
    forward value cancels), as the reference adds. ``p`` is the arity (the
    last dimension); the formula does not otherwise use it."""
    if block_assignments.dim() != 5:
        raise ValueError(f"block_assignments must be (B, H, NB, L, p); got {tuple(block_assignments.shape)}")
    a = block_assignments
    L = a.shape[-2]
    # (B, H, L, NB, p) @ (B, H, L, p, NB) -> m[b, h, l, i, j], in the input's precision
    al = a.permute(0, 1, 3, 2, 4).contiguous()
    m = torch.matmul(al, al.transpose(-1, -2).contiguous())
    m = m.permute(0, 1, 3, 4, 2)                                  # (B, H, NB, NB, L)
    shared = torch.cummin(m, dim=-1).values
    if m.requires_grad:
        w = 0.05 * torch.pow(2.0, torch.arange(L, device=m.device, dtype=m.dtype) - (L - 1))
        tie = m * w
        shared = shared + (tie - tie.detach())
    return L - shared.sum(dim=-1)


def _block_mean(assignments: torch.Tensor, S: int, route_block: int) -> torch.Tensor:
    """(B, H, S, L, p) -> (B, H, NB, L, p): the mean over each route block's tokens
    (a last block shorter than route_block averages its valid tokens only)."""
    B, H, _, L, P = assignments.shape
    NB = -(-S // route_block)
    a = assignments[:, :, :S]
    pad = NB * route_block - S
    if pad:
        a = torch.cat([a, a.new_zeros(B, H, pad, L, P)], dim=2)
    n = torch.full((NB,), float(route_block), dtype=a.dtype, device=a.device)
    n[-1] = S - (NB - 1) * route_block
    return a.view(B, H, NB, route_block, L, P).sum(dim=3) / n.view(1, 1, NB, 1, 1)


def ste_soft_block_bias(block_assignments: torch.Tensor, lists: torch.Tensor, r: int, p: int,
                        max_dist: Optional[float] = None) -> torch.Tensor:
    """The router's straight-through soft bias (surgery.py:577-588): logits
    (max_dist - expected_block_distance) / 0.5 gathered at each row's listed
    blocks (entries clamped into [0, NB)), returned as g - g.detach(): zero in
    the forward pass, gradient 1 with respect to g. ``max_dist`` defaults to
    L - r, as the reference's config default."""
    L = block_assignments.shape[-2]
    NB = block_assignments.shape[2]
    md = float(max_dist) if max_dist is not None else float(L - int(r))
    dist = expected_block_distance(block_assignments.float(), p=p)
    logits = (md - dist) / 0.5
    idx = lists.clamp(min=0, max=max(NB - 1, 0)).to(torch.int64)
    g = torch.gather(logits, dim=-1, index=idx)
    return g - g.detach()


def route_block_vote(assignments: torch.Tensor, r: int, route_block: int) -> torch.Tensor:
    """(B, H, S, L, p) branch scores -> (B, H, ceil(S / route_block), r) int32 routing ids."""
    if assignments.dim() != 5:
        raise ValueError(f"assignments must be (B, H, S, levels, p); got {tuple(assignments.shape)}")
    B, H, S, L, P = assignments.shape
    r = int(r)
    if not 0 <= r <= L:
        raise ValueError(f"r={r} must lie in [0, {L}]")
    if route_block < 1:
        raise ValueError("route_block must be >= 1")
    dev = nat.require_device(assignments)
    a = assignments if assignments.dtype in _SCORE_DTYPES else assignments.float()
    NB = -(-S // route_block)
    out = torch.empty((B, H, NB, r), dtype=torch.int32, device=dev)
    if out.numel() == 0:
        return out
    with torch.cuda.device(dev):
        rc = nat.lib().sa_route_block_vote(nat.ptr(a), nat.dtype_code(a.dtype, _SCORE_DTYPES), nat.strides(a),
                                           B, H, S, L, P, r, int(route_block), nat.ptr(out), nat.stream(dev))
    nat.check(rc)
    return out


class RouteCache:
    """Cross-layer reuse of routing (surgery.py:295-315, ``surgical_route_stride``).

    With ``stride`` s > 1, layer l with l % s != 0 reuses the block lists of its
    anchor layer (l // s) * s, provided the anchor was built with the same
    (B, H, NB, r, route_block, local_window, p); the reference caches the
    anchor's routing assignments under the same rule, this cache keeps the
    anchor's block lists, so that non-anchor layers launch neither the vote
    nor the list build. Anchor layers always route and store their lists.
    """

    def __init__(self, stride: int = 1):
        self.stride = max(1, int(stride))
        self._lists = {}

    def clear(self):
        self._lists.clear()

    def lookup(self, layer_idx: int, key: tuple):
        if self.stride > 1 and layer_idx % self.stride != 0:
            hit = self._lists.get((layer_idx // self.stride) * self.stride)
            if hit is not None and hit[0] == key:
                return hit[1]
        return None

    def store(self, layer_idx: int, key: tuple, lists):
        if layer_idx % self.stride == 0:
            self._lists[layer_idx] = (key, lists)


def block_list_prefill(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, assignments: torch.Tensor, r: int,
                       *, p: int, route_block: int = 128, local_window: int = 16,
                       sm_scale: Optional[float] = None, block_assignments: Optional[torch.Tensor] = None,
                       return_stats: bool = False, route_cache: Optional[RouteCache] = None,
                       layer_idx: Optional[int] = None, max_dist: Optional[float] = None):
    """Causal block-list prefill with block-granular tree routing.

    q: (B, H, S, D); k, v: (B, H_kv, S, D). ``assignments``: (B, H, S, L, p)
    per-token branch scores, or (B, H, NB, L, p) per-block scores when
    NB != S (direct block routing); ``block_assignments`` of shape
    (B, H, NB, L, p) take precedence, as in the reference. ``r``: routed
    levels (req_depth). Returns the attention output, plus a dict with
    ``mean_allowed_keys``, ``mean_causal_keys`` and ``block_density``
    (surgery.py:589-595; host reads) when ``return_stats``. With ``route_cache``
    and ``layer_idx``, non-anchor layers reuse their anchor's lists (see
    RouteCache) and ``assignments`` is not read for them. When grad is
    enabled and ``assignments`` requires grad, the straight-through soft bias
    (``ste_soft_block_bias``, ``max_dist`` defaulting to L - r) is added, so
    the scores receive the reference's router gradient (surgery.py:566-588).
    """
    B, H, S, _ = q.shape
    RB = int(route_block)
    NB = -(-S // RB)
    key = (B, H, NB, int(r), RB, int(local_window), int(p))
    bl = None
    if route_cache is not None and layer_idx is not None:
        bl = route_cache.lookup(int(layer_idx), key)
    if bl is None:
        if int(r) == 0:
            # no routed level: every block matches (the list build needs a
            # routing vector of at least one level; depth 0 never reads it)
            route = torch.zeros((B, H, NB, 1), dtype=torch.int32, device=q.device)
        elif block_assignments is not None and block_assignments.shape[2] == NB:
            route = route_block_vote(block_assignments[:, :, :NB], r, 1)
        elif assignments.shape[2] == NB and NB != S:
            route = route_block_vote(assignments[:, :, :NB], r, 1)
        else:
            route = route_block_vote(assignments[:, :, :S], r, RB)
        bl = build_block_lists(route, r, is_causal=True, sink_block=True,
                               local_blocks=local_blocks_of(local_window, RB), arity=p)
        if route_cache is not None and layer_idx is not None:
            route_cache.store(int(layer_idx), key, bl)
    soft_bias = None
    if torch.is_grad_enabled() and assignments is not None and assignments.requires_grad:
        if block_assignments is not None and block_assignments.shape[2] == NB:
            blk = block_assignments[:, :, :NB]
        elif assignments.shape[2] == NB and NB != S:
            blk = assignments[:, :, :NB]
        else:
            blk = _block_mean(assignments, S, RB)
        soft_bias = ste_soft_block_bias(blk, bl.lists, r, p, max_dist=max_dist)
    out = block_list_attention(q, k, v, bl, route_block=RB, is_causal=True, sm_scale=sm_scale,
                               soft_block_bias=soft_bias)
    if not return_stats:
        return out
    lens = torch.full((NB,), RB, dtype=torch.float32, device=q.device)
    lens[-1] = S - (NB - 1) * RB
    c = bl.counts.to(torch.float32)
    allowed = ((c - 1) * RB * lens + lens * (lens + 1) / 2).sum(-1)
    stats = {
        "mean_allowed_keys": (allowed.mean() / S).item(),
        "mean_causal_keys": (S + 1) / 2,
        "block_density": (c.sum() / (B * H * NB * (NB + 1) / 2)).item(),
    }
    return out, stats
