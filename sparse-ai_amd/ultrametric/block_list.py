"""Block-list sparse attention on MI355X (drop-in for src/ultrametric/block_list.py).

Same public names, signatures, argument meaning and exception types as the
reference module; the work runs in hand-written HIP kernels for gfx950
(libsparseattn.so, see include/sparse_attn.h) launched on torch's current
stream:

* ``build_block_lists`` (block_list.py:170-278) — routing vectors -> per-row
  ascending lists of active key blocks. One compaction kernel computes the
  mixed-radix codes, the structural masks and the ballot/prefix compaction;
  the sync-free mode (``arity`` given) performs no host<->device sync.
* ``block_lists_from_mask`` — the same compaction from an explicit per-head
  (Z, H, NB, NB) block mask (extension).
* ``block_list_attention`` (block_list.py:968-1061) — flash-style forward
  over the lists (bf16/fp16 on MFMA, fp32 in true fp32), with GQA-native
  K/V (k, v may carry H_kv | H heads).
* ``routed_block_attention`` (block_list.py:1064-1083).
* ``build_transposed_block_lists`` (block_list.py:281-327).

``block_mask_reference``, ``token_mask_from_blocks`` and
``masked_reference_attention`` keep the reference's independent torch
formulations (block_list.py:334-378) for callers' correctness checks; no
function above calls them.

There is no CPU fallback: CPU tensors or a missing library raise RuntimeError.

``block_list_attention`` is differentiable in q, k, v and ``soft_block_bias``
(the reference's sparse autograd, block_list.py:494-961): the backward
computes delta = rowsum(dO * O) inside the dQ kernel, which walks each query
tile's list; dK and dV walk each key tile's transposed list; the soft-bias
gradient of a (query block, list slot) is the sum of dS over that pair. The
one host read of the backward is the work plan's three counts, at the point
where the reference reads max(q_counts) (block_list.py:320).
"""

from __future__ import annotations

import contextlib
import math
from typing import NamedTuple, Optional, Sequence, Union

import torch

from . import _native as nat

HAS_TRITON = nat.available()  # name kept for callers: "the kernel backend is present"
HAS_HIP = HAS_TRITON

DepthLike = Union[int, Sequence[int], torch.Tensor]

__all__ = [
    "HAS_TRITON",
    "HAS_HIP",
    "BlockLists",
    "build_block_lists",
    "block_lists_from_mask",
    "build_transposed_block_lists",
    "block_list_attention",
    "routed_block_attention",
    "block_mask_reference",
    "token_mask_from_blocks",
    "masked_reference_attention",
]


class BlockLists(NamedTuple):
    """Active key route-blocks per query route-block (block_list.py:78-90).

    lists:     (Z, H, NB, max_count) int32, ascending; entries >= counts are 0.
    counts:    (Z, H, NB) int32.
    max_count: int (= NB for the sync-free builder).
    """

    lists: torch.Tensor
    counts: torch.Tensor
    max_count: int


def _depth_tensor(req_depth: DepthLike, num_heads: int, tree_depth: int,
                  device: torch.device) -> torch.Tensor:
    """block_list.py:93-104: normalise req_depth to (H,) int64 and validate (host sync)."""
    if isinstance(req_depth, int):
        depth = torch.full((num_heads,), req_depth, dtype=torch.int64, device=device)
    else:
        depth = torch.as_tensor(req_depth, dtype=torch.int64, device=device).reshape(-1)
        if depth.numel() != num_heads:
            raise ValueError(f"req_depth has {depth.numel()} entries, expected {num_heads} (one per head)")
    if depth.numel() and (int(depth.min()) < 0 or int(depth.max()) > tree_depth):
        raise ValueError(f"req_depth must be in [0, {tree_depth}], got {depth.tolist()}")
    return depth.contiguous()


def _apply_structural_masks(match: torch.Tensor, *, is_causal: bool, sink_block: bool,
                            local_blocks: int) -> torch.Tensor:
    """block_list.py:107-118 (used by the torch reference helpers only)."""
    nb = match.shape[-1]
    idx = torch.arange(nb, device=match.device)
    if local_blocks > 0:
        match = match | ((idx.view(-1, 1) - idx.view(1, -1)).abs() <= local_blocks)
    if sink_block:
        match = match.clone()
        match[..., 0] = True
    if is_causal:
        match = match & (idx.view(-1, 1) >= idx.view(1, -1))
    return match


def _launch_build(router: torch.Tensor, depth_dev: Optional[torch.Tensor], depth_uniform: int,
                  base: int, use_codes: bool, is_causal: bool, sink_block: bool, local_blocks: int,
                  lists: Optional[torch.Tensor], cols: int, counts: torch.Tensor) -> None:
    Z, H, NB, TD = router.shape
    dev = router.device
    lib = nat.lib()
    with torch.cuda.device(dev):
        rc = lib.sa_build_block_lists(
            nat.ptr(router), nat.DTYPE_CODES[router.dtype], nat.strides(router), Z, H, NB, TD,
            nat.ptr(depth_dev), int(depth_uniform), int(base), int(use_codes), int(bool(is_causal)),
            int(bool(sink_block)), int(local_blocks), nat.ptr(lists), int(cols), nat.ptr(counts),
            nat.stream(dev))
    nat.check(rc)


@torch.no_grad()
def build_block_lists(
    router_indices: torch.Tensor,
    req_depth: DepthLike,
    *,
    is_causal: bool = False,
    sink_block: bool = False,
    local_blocks: int = 0,
    arity: Optional[int] = None,
) -> BlockLists:
    """Per-row active key-block lists from per-block routing vectors (block_list.py:170-278).

    router_indices: (Z, H, NB, TD) integer branch ids. Blocks i, j match iff
    their routing vectors agree on the first ``req_depth[h]`` levels; then the
    local band, sink column and causal triangle are applied in that order.
    ``arity`` given => sync-free: ids are not validated, ``max_count = NB``.
    Otherwise the ids are validated and the lists are cut to max(counts)
    (two host reads, as in the reference).
    """
    if router_indices.dim() != 4:
        raise ValueError(f"router_indices must be (Z, H, NB, TD), got {tuple(router_indices.shape)}")
    Z, H, NB, TD = router_indices.shape
    device = router_indices.device
    sync_free = arity is not None
    if sync_free and isinstance(req_depth, int):
        if not 0 <= req_depth <= TD:
            raise ValueError(f"req_depth must be in [0, {TD}], got {req_depth}")
        depth_dev, depth_uniform = None, int(req_depth)
    else:
        depth_dev, depth_uniform = _depth_tensor(req_depth, H, TD, device), 0
    r = router_indices
    if r.dtype not in (torch.int32, torch.int64):
        r = r.to(torch.int64)

    if sync_free:
        base = max(2, int(arity))
    else:
        if r.numel() and int(r.min()) < 0:
            raise ValueError("router_indices must be non-negative branch ids")
        base = max(2, int(r.max()) + 1) if r.numel() else 2
    use_codes = TD * math.log2(base) < 62
    nat.require_device(router_indices)

    counts = torch.empty((Z, H, NB), dtype=torch.int32, device=device)
    if sync_free:
        lists = torch.empty((Z, H, NB, NB), dtype=torch.int32, device=device)
        if counts.numel():
            _launch_build(r, depth_dev, depth_uniform, base, use_codes, is_causal, sink_block,
                          local_blocks, lists, NB, counts)
        return BlockLists(lists, counts, NB)

    if counts.numel() == 0:
        return BlockLists(torch.zeros((Z, H, NB, 0), dtype=torch.int32, device=device), counts, 0)
    _launch_build(r, depth_dev, depth_uniform, base, use_codes, is_causal, sink_block,
                  local_blocks, None, 0, counts)
    max_count = int(counts.max())
    lists = torch.empty((Z, H, NB, max_count), dtype=torch.int32, device=device)
    _launch_build(r, depth_dev, depth_uniform, base, use_codes, is_causal, sink_block,
                  local_blocks, lists, max_count, counts)
    return BlockLists(lists, counts, max_count)


@torch.no_grad()
def block_lists_from_mask(
    block_mask: torch.Tensor,
    *,
    is_causal: bool = False,
    sink_block: bool = False,
    local_blocks: int = 0,
    sync_free: bool = True,
) -> BlockLists:
    """Compact an explicit (Z, H, NB, NB) bool/uint8 block mask into BlockLists.

    The compaction of block_list.py:263-278 applied to a caller-supplied
    ``match`` (structural masks are applied on top, in the reference order).
    ``sync_free`` pads rows to NB columns; otherwise lists are cut to
    max(counts) with one host read.
    """
    if block_mask.dim() != 4 or block_mask.shape[-1] != block_mask.shape[-2]:
        raise ValueError(f"block_mask must be (Z, H, NB, NB), got {tuple(block_mask.shape)}")
    nat.require_device(block_mask)
    Z, H, NB, _ = block_mask.shape
    m = block_mask
    if m.dtype == torch.bool:
        m = m.view(torch.uint8)
    elif m.dtype != torch.uint8:
        m = (m != 0).view(torch.uint8)
    device = m.device
    counts = torch.empty((Z, H, NB), dtype=torch.int32, device=device)
    lib = nat.lib()

    def launch(lists, cols):
        with torch.cuda.device(device):
            rc = lib.sa_build_block_lists_mask(nat.ptr(m), nat.strides(m), Z, H, NB, int(bool(is_causal)),
                                               int(bool(sink_block)), int(local_blocks), nat.ptr(lists),
                                               int(cols), nat.ptr(counts), nat.stream(device))
        nat.check(rc)

    if sync_free:
        lists = torch.empty((Z, H, NB, NB), dtype=torch.int32, device=device)
        if counts.numel():
            launch(lists, NB)
        return BlockLists(lists, counts, NB)
    if counts.numel() == 0:
        return BlockLists(torch.zeros((Z, H, NB, 0), dtype=torch.int32, device=device), counts, 0)
    launch(None, 0)
    max_count = int(counts.max())
    lists = torch.empty((Z, H, NB, max_count), dtype=torch.int32, device=device)
    launch(lists, max_count)
    return BlockLists(lists, counts, max_count)


@torch.no_grad()
def build_transposed_block_lists(
    block_lists: BlockLists,
    num_key_blocks: Optional[int] = None,
) -> BlockLists:
    """Query blocks per key block (block_list.py:281-327).

    The listed (qb, kb) pairs are scattered into a device block mask, which
    is transposed and compacted by the HIP compaction kernel.
    """
    lists, counts, max_count = block_lists
    Z, H, NB_Q = counts.shape
    NB_K = num_key_blocks if num_key_blocks is not None else NB_Q
    device = lists.device
    nat.require_device(lists, counts)
    if NB_Q == 0 or NB_K == 0 or max_count == 0:
        return BlockLists(torch.zeros((Z, H, NB_K, 0), dtype=torch.int32, device=device),
                          torch.zeros((Z, H, NB_K), dtype=torch.int32, device=device), 0)
    if NB_K != NB_Q:
        raise RuntimeError("build_transposed_block_lists: only square block grids are supported")
    if NB_Q <= _TRANSPOSE_MAX_NB:
        l32 = lists.to(torch.int32).contiguous()
        c32 = counts.to(torch.int32).contiguous()
        t_counts = torch.empty((Z, H, NB_K), dtype=torch.int32, device=device)
        _launch_transpose(l32, c32, max_count, None, 0, t_counts)
        t_max = int(t_counts.max()) if t_counts.numel() else 0     # host read, as block_list.py:320
        t_lists = torch.empty((Z, H, NB_K, max(t_max, 1)), dtype=torch.int32, device=device)
        _launch_transpose(l32, c32, max_count, t_lists, max(t_max, 1), t_counts)
        return BlockLists(t_lists[..., :t_max].contiguous(), t_counts, t_max)
    t_idx = torch.arange(max_count, device=device).view(1, 1, 1, max_count)
    valid = t_idx < counts.unsqueeze(-1)
    safe_kb = torch.where(valid, lists.to(torch.int64), torch.full_like(lists, NB_K, dtype=torch.int64))
    match_qk = torch.zeros((Z, H, NB_Q, NB_K + 1), dtype=torch.bool, device=device)
    match_qk.scatter_(-1, safe_kb, valid)
    match_kq = match_qk[..., :NB_K].transpose(-2, -1)
    return block_lists_from_mask(match_kq, sync_free=False)


_TRANSPOSE_MAX_NB = 8192  # sa_transpose_block_lists limit (the builder's); larger grids use torch scatter + compaction


def _launch_transpose(lists, counts, max_count, t_lists, t_cols, t_counts):
    Z, H, NB = counts.shape
    dev = counts.device
    with torch.cuda.device(dev):
        rc = nat.lib().sa_transpose_block_lists(nat.ptr(lists) if max_count > 0 else None, nat.ptr(counts),
                                                int(max_count), Z, H, NB, nat.ptr(t_lists), int(t_cols),
                                                nat.ptr(t_counts), nat.stream(dev))
    nat.check(rc)


def _transposed_lists_sync_free(lists, counts, max_count, nb):
    """Transposed lists of width nb (no host read): the layout of
    build_transposed_block_lists before its cut to max(q_counts)."""
    Z, H, _ = counts.shape
    device = lists.device
    if nb == 0 or max_count == 0:
        return (torch.zeros((Z, H, nb, 0), dtype=torch.int32, device=device),
                torch.zeros((Z, H, nb), dtype=torch.int32, device=device), 0)
    if nb <= _TRANSPOSE_MAX_NB:
        t_lists = torch.empty((Z, H, nb, nb), dtype=torch.int32, device=device)
        t_counts = torch.empty((Z, H, nb), dtype=torch.int32, device=device)
        _launch_transpose(lists.to(torch.int32).contiguous(), counts.to(torch.int32).contiguous(), max_count,
                          t_lists, nb, t_counts)
        return t_lists, t_counts, nb
    t_idx = torch.arange(max_count, device=device).view(1, 1, 1, max_count)
    valid = t_idx < counts.unsqueeze(-1)
    safe_kb = torch.where(valid, lists.to(torch.int64), torch.full_like(lists, nb, dtype=torch.int64))
    match_qk = torch.zeros((Z, H, counts.shape[2], nb + 1), dtype=torch.bool, device=device)
    match_qk.scatter_(-1, safe_kb, valid)
    tl = block_lists_from_mask(match_qk[..., :nb].transpose(-2, -1), sync_free=True)
    return tl.lists, tl.counts, tl.max_count


# ----------------------------------------------------------------------------
# Forward
# ----------------------------------------------------------------------------

def _launch_fwd(q, k, v, out, lse, lists, counts, max_count, soft_block_bias, route_block,
                is_causal, scale):
    Z, H, N, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    dt = nat.dtype_code(q.dtype, (torch.float32, torch.bfloat16, torch.float16))
    sb = soft_block_bias
    sb_code = 0
    if sb is not None:
        if sb.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            sb = sb.float()
        sb_code = nat.DTYPE_CODES[sb.dtype]
    lib = nat.lib()
    with torch.cuda.device(dev):
        rc = lib.sa_block_sparse_fwd(
            nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(out), nat.ptr(lse), nat.ptr(lists),
            nat.ptr(counts), nat.ptr(sb), sb_code, Z, H, Hkv, N, D, int(route_block), int(max_count),
            nat.strides(q), nat.strides(k), nat.strides(v), nat.strides(out),
            nat.strides(sb) if sb is not None else None, float(scale), dt, int(bool(is_causal)),
            nat.stream(dev))
    nat.check(rc)


def block_list_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    block_lists: BlockLists,
    *,
    route_block: int = 128,
    is_causal: bool = False,
    sm_scale: Optional[float] = None,
    block_m: Optional[int] = None,
    block_n: Optional[int] = None,
    num_warps: int = 4,
    num_stages: int = 3,
    return_lse: bool = False,
    soft_block_bias: Optional[torch.Tensor] = None,
):
    """Block-sparse attention over precomputed block lists (block_list.py:968-1061).

    q: (Z, H, N, D); k, v: (Z, H_kv, N, D) with H_kv dividing H (GQA; the
    reference requires H_kv == H). D a power of two >= 16 (<= 256 here),
    route_block a power of two >= 16. ``block_m`` / ``block_n`` /
    ``num_warps`` / ``num_stages`` are the reference's Triton tile knobs: the
    HIP kernels pick their own tiles, but given values must still divide
    route_block (block_list.py:738-739). Returns out, or (out, lse) with lse
    the natural-log LSE of the scaled scores, (Z, H, N) fp32, -inf for rows
    with no visible key. Differentiable in q, k, v and ``soft_block_bias``
    (block_list.py:883-961): the backward recomputes P from the saved LSE.
    """
    if not HAS_TRITON:
        raise RuntimeError("block_list_attention requires the HIP backend (libsparseattn.so)")
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4 or k.shape != v.shape \
            or q.shape[0] != k.shape[0] or q.shape[2:] != k.shape[2:] \
            or k.shape[1] == 0 or q.shape[1] % k.shape[1] != 0:
        raise ValueError(f"q, k, v must share shape (Z, H, N, D) (k, v may have H_kv | H heads); "
                         f"got {q.shape}, {k.shape}, {v.shape}")
    if not (q.dtype == k.dtype == v.dtype):
        raise ValueError("q, k, v must share dtype")
    Z, H, N, D = q.shape
    if D < 16 or D & (D - 1):
        raise ValueError(f"head_dim must be a power of two >= 16, got {D}")
    if route_block < 16 or route_block & (route_block - 1):
        raise ValueError(f"route_block must be a power of two >= 16, got {route_block}")
    for name, val in (("block_m", block_m), ("block_n", block_n)):
        if val is not None and (val <= 0 or route_block % val):
            raise ValueError(f"block_m ({block_m}) and block_n ({block_n}) must divide route_block ({route_block})")

    lists, counts, max_count = block_lists
    nb = -(-N // route_block)
    if tuple(counts.shape) != (Z, H, nb) or tuple(lists.shape[:3]) != (Z, H, nb):
        raise ValueError(f"block_lists built for {tuple(counts.shape)}, expected {(Z, H, nb)} "
                         f"(N={N}, route_block={route_block})")
    if lists.shape[-1] != max_count:
        raise ValueError("lists.shape[-1] must equal max_count")
    if soft_block_bias is not None and tuple(soft_block_bias.shape) != (Z, H, nb, max_count):
        raise ValueError(
            f"soft_block_bias must have shape {(Z, H, nb, max_count)}, got {tuple(soft_block_bias.shape)}")
    nat.require_device(q, k, v, lists, counts)
    if soft_block_bias is not None:
        nat.require_device(q, soft_block_bias)

    lists = lists.to(torch.int32).contiguous()
    counts = counts.to(torch.int32).contiguous()
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    needs_grad = torch.is_grad_enabled() and (
        q.requires_grad or k.requires_grad or v.requires_grad
        or (soft_block_bias is not None and soft_block_bias.requires_grad))
    if needs_grad:
        return _BlockListAttentionFn.apply(q, k, v, soft_block_bias, lists, counts, int(max_count),
                                           int(route_block), bool(is_causal), float(scale), bool(return_lse))
    out = torch.empty((Z, H, N, D), dtype=q.dtype, device=q.device)
    lse = torch.empty((Z, H, N), dtype=torch.float32, device=q.device) if return_lse else None
    _launch_fwd(q, k, v, out, lse, lists, counts, max_count,
                soft_block_bias.detach() if soft_block_bias is not None else None,
                route_block, is_causal, scale)
    return (out, lse) if return_lse else out


# ----------------------------------------------------------------------------
# Backward
# ----------------------------------------------------------------------------

_SIDE_STREAMS = {}


def _side_stream(dev: torch.device) -> torch.cuda.Stream:
    """A second stream per device (default priority) for backward work that does not
    feed dQ."""
    idx = dev.index if dev.index is not None else torch.cuda.current_device()
    st = _SIDE_STREAMS.get(idx)
    if st is None:
        st = torch.cuda.Stream(device=idx)
        _SIDE_STREAMS[idx] = st
    return st


def _launch_bwd(dout, q, k, v, out, lse, lists, counts, max_count, soft_block_bias, route_block,
                is_causal, scale):
    """dq, dk, dv (and the soft-bias gradient) of block-list attention
    (block_list.py:758-880): delta = rowsum(dout * out), dQ over the forward
    lists, dK / dV over the transposed lists."""
    Z, H, N, D = q.shape
    Hkv = k.shape[1]
    dev = q.device
    nb = -(-N // route_block)
    dt = nat.dtype_code(q.dtype, (torch.float32, torch.bfloat16, torch.float16))
    if dout.dtype != q.dtype:
        dout = dout.to(q.dtype)
    sb = soft_block_bias
    sb_code = 0
    if sb is not None:
        if sb.dtype not in (torch.float32, torch.bfloat16, torch.float16):
            sb = sb.float()
        sb_code = nat.DTYPE_CODES[sb.dtype]
    sb_st = nat.strides(sb) if sb is not None else None
    lib = nat.lib()
    lists_p = nat.ptr(lists) if max_count > 0 else None
    mfma = not (q.dtype == torch.float32 or route_block < 32 or Z * H * N == 0)

    # MFMA path: the transposed lists and the dK/dV work plan do not feed dQ, so they
    # are built on a second stream while dQ runs on the caller's stream, which waits
    # for them before dK/dV. The plan's item counts are the backward's one host read
    # (the reference reads max(q_counts) at this point, block_list.py:320).
    main = torch.cuda.current_stream(dev)
    if mfma:
        side = _side_stream(dev)
        side.wait_stream(main)
        where = torch.cuda.stream(side)
    else:
        where = contextlib.nullcontext()
    with where:
        t_lists, t_counts, t_max = _transposed_lists_sync_free(lists, counts, max_count, nb)
        t_lists_p = nat.ptr(t_lists) if t_max > 0 else None
        if mfma:
            nbytes = int(lib.sa_block_sparse_bwd_plan_bytes(Z, H, Hkv, N, int(route_block), int(t_max)))
            plan = torch.empty(nbytes, dtype=torch.uint8, device=dev)
            info = torch.empty(3, dtype=torch.int32, device=dev)
            with torch.cuda.device(dev):
                rc = lib.sa_block_sparse_bwd_plan(lists_p, nat.ptr(counts), int(max_count), t_lists_p,
                                                  nat.ptr(t_counts), int(t_max), nat.ptr(sb), sb_code, sb_st, Z, H,
                                                  Hkv, N, int(route_block), nat.ptr(plan), nbytes, nat.ptr(info),
                                                  nat.stream(dev))
            nat.check(rc)
            info_host = torch.empty(3, dtype=torch.int32, pin_memory=True)
            info_host.copy_(info, non_blocking=True)
            ready = torch.cuda.Event()
            ready.record(side)

    dq = torch.empty_like(q)
    dk = torch.empty_like(k)
    dv = torch.empty_like(v)
    delta = torch.empty((Z, H, N), dtype=torch.float32, device=dev)
    dsb = torch.zeros((Z, H, nb, max_count), dtype=torch.float32, device=dev) if sb is not None else None

    def launch(phases, plan=None, n_work=0, n_multi=0, partials=None):
        with torch.cuda.device(dev):
            rc = lib.sa_block_sparse_bwd(
                nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(out), nat.ptr(dout), nat.ptr(lse),
                lists_p, nat.ptr(counts), int(max_count), t_lists_p, nat.ptr(t_counts), int(t_max),
                nat.ptr(sb), sb_code, sb_st,
                nat.ptr(delta), nat.ptr(dq), nat.ptr(dk), nat.ptr(dv), nat.ptr(dsb),
                nat.ptr(plan), int(n_work), int(n_multi), nat.ptr(partials), int(phases),
                Z, H, Hkv, N, D, int(route_block),
                nat.strides(q), nat.strides(k), nat.strides(v), nat.strides(out), nat.strides(dout),
                nat.strides(dq), nat.strides(dk), nat.strides(dv), float(scale), dt, int(bool(is_causal)),
                nat.stream(dev))
        nat.check(rc)

    if not mfma:
        launch(3)
        return dq, dk, dv, dsb
    launch(1)                       # dQ (with delta) reads only the forward lists
    main.wait_stream(side)
    for t in (t_lists, t_counts, plan):
        t.record_stream(main)
    ready.synchronize()
    n_work, n_multi, n_multi_items = info_host.tolist()
    partials = None
    if n_multi:
        bk = 128 if route_block >= 128 else route_block
        partials = torch.empty(n_multi_items * 2 * bk * D, dtype=torch.float32, device=dev)
    launch(2, plan, n_work, n_multi, partials)
    return dq, dk, dv, dsb


class _BlockListAttentionFn(torch.autograd.Function):
    """Autograd wrapper of the HIP forward / backward (block_list.py:883-961)."""

    @staticmethod
    def forward(ctx, q, k, v, soft_block_bias, lists, counts, max_count, route_block, is_causal, scale,
                return_lse):
        Z, H, N, D = q.shape
        out = torch.empty((Z, H, N, D), dtype=q.dtype, device=q.device)
        lse = torch.empty((Z, H, N), dtype=torch.float32, device=q.device)
        sb = soft_block_bias.detach() if soft_block_bias is not None else None
        _launch_fwd(q, k, v, out, lse, lists, counts, max_count, sb, route_block, is_causal, scale)
        ctx.save_for_backward(q, k, v, out, lse, lists, counts, sb)
        ctx.max_count, ctx.route_block, ctx.is_causal, ctx.scale = max_count, route_block, is_causal, scale
        ctx.sb_dtype = soft_block_bias.dtype if soft_block_bias is not None else None
        if return_lse:
            ctx.mark_non_differentiable(lse)
            return out, lse
        return out

    @staticmethod
    def backward(ctx, dout, *unused):
        q, k, v, out, lse, lists, counts, sb = ctx.saved_tensors
        dq, dk, dv, dsb = _launch_bwd(dout, q, k, v, out, lse, lists, counts, ctx.max_count, sb,
                                      ctx.route_block, ctx.is_causal, ctx.scale)
        if dsb is not None and ctx.sb_dtype is not None:
            dsb = dsb.to(ctx.sb_dtype)
        return (dq if ctx.needs_input_grad[0] else None,
                dk if ctx.needs_input_grad[1] else None,
                dv if ctx.needs_input_grad[2] else None,
                dsb if ctx.needs_input_grad[3] else None,
                None, None, None, None, None, None, None)


def routed_block_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    router_indices: torch.Tensor,
    req_depth: DepthLike,
    *,
    route_block: int = 128,
    is_causal: bool = False,
    sink_block: bool = False,
    local_blocks: int = 0,
    sm_scale: Optional[float] = None,
    soft_block_bias: Optional[torch.Tensor] = None,
    arity: Optional[int] = None,
) -> torch.Tensor:
    """Build the block lists, then run the kernel (block_list.py:1064-1083).

    ``arity`` (extension; the branch count, ids in [0, arity)) builds the lists
    sync-free, as ``build_block_lists(..., arity=arity)``. Then, without a soft
    bias and when no input needs a gradient, the build runs inside the forward
    kernel: one launch (``sa_routed_block_sparse_fwd``) instead of two.
    """
    if arity is not None and soft_block_bias is None and not (
            torch.is_grad_enabled() and (q.requires_grad or k.requires_grad or v.requires_grad)):
        fused = _routed_fused(q, k, v, router_indices, req_depth, route_block=route_block, is_causal=is_causal,
                              sink_block=sink_block, local_blocks=local_blocks, sm_scale=sm_scale, arity=arity)
        if fused is not None:
            return fused[0]
    bl = build_block_lists(router_indices, req_depth, is_causal=is_causal,
                           sink_block=sink_block, local_blocks=local_blocks, arity=arity)
    return block_list_attention(q, k, v, bl, route_block=route_block,
                                is_causal=is_causal, sm_scale=sm_scale,
                                soft_block_bias=soft_block_bias)


def _routed_fused(q, k, v, router_indices, req_depth, *, route_block, is_causal, sink_block, local_blocks,
                  sm_scale, arity):
    """(out, BlockLists) from one sa_routed_block_sparse_fwd launch, or None when the
    inputs are outside what it covers (the caller then builds the lists and calls
    block_list_attention, which also raises the reference's errors)."""
    if not HAS_TRITON or router_indices.dim() != 4 or q.dim() != 4 or k.dim() != 4 or k.shape != v.shape:
        return None
    Z, H, N, D = q.shape
    if (q.dtype not in (torch.bfloat16, torch.float16) or not (q.dtype == k.dtype == v.dtype)
            or k.shape[0] != Z or k.shape[2:] != q.shape[2:] or k.shape[1] == 0 or H % k.shape[1] != 0
            or route_block < 32 or route_block & (route_block - 1) or D & (D - 1) or D < 16):
        return None
    Zr, Hr, NB, TD = router_indices.shape
    if (Zr, Hr, NB) != (Z, H, -(-N // route_block)) or TD < 1:
        return None
    base = max(2, int(arity))
    if not TD * math.log2(base) < 62:
        return None
    if isinstance(req_depth, int):
        if not 0 <= req_depth <= TD:
            return None
        depth_dev, depth_uniform = None, int(req_depth)
    else:
        depth_dev, depth_uniform = _depth_tensor(req_depth, H, TD, q.device), 0
    r = router_indices if router_indices.dtype in (torch.int32, torch.int64) else router_indices.to(torch.int64)
    dev = nat.require_device(q, k, v, r)
    out = torch.empty((Z, H, N, D), dtype=q.dtype, device=dev)
    lists = torch.empty((Z, H, NB, NB), dtype=torch.int32, device=dev)
    counts = torch.empty((Z, H, NB), dtype=torch.int32, device=dev)
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(D)
    with torch.cuda.device(dev):
        rc = nat.lib().sa_routed_block_sparse_fwd(
            nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(out), None, nat.ptr(r), nat.DTYPE_CODES[r.dtype],
            nat.strides(r), TD, nat.ptr(depth_dev), depth_uniform, base, int(bool(sink_block)), int(local_blocks),
            nat.ptr(lists), nat.ptr(counts), Z, H, k.shape[1], N, D, int(route_block), nat.strides(q),
            nat.strides(k), nat.strides(v), nat.strides(out), float(scale), nat.DTYPE_CODES[q.dtype],
            int(bool(is_causal)), nat.stream(dev))
    if rc == nat.SA_EUNSUPPORTED:
        return None
    nat.check(rc)
    return out, BlockLists(lists, counts, NB)


# ----------------------------------------------------------------------------
# Reference formulations kept for callers' checks (block_list.py:334-378).
# ----------------------------------------------------------------------------

@torch.no_grad()
def block_mask_reference(router_indices: torch.Tensor, req_depth: DepthLike, *,
                         is_causal: bool = False, sink_block: bool = False,
                         local_blocks: int = 0) -> torch.Tensor:
    """(Z, H, NB, NB) bool block mask by explicit per-head prefix comparison."""
    Z, H, NB, TD = router_indices.shape
    depth = _depth_tensor(req_depth, H, TD, router_indices.device).tolist()
    out = torch.empty((Z, H, NB, NB), dtype=torch.bool, device=router_indices.device)
    for h, d in enumerate(depth):
        if d == 0:
            out[:, h] = True
        else:
            rh = router_indices[:, h, :, :d]
            out[:, h] = (rh[:, :, None, :] == rh[:, None, :, :]).all(-1)
    return _apply_structural_masks(out, is_causal=is_causal, sink_block=sink_block,
                                   local_blocks=local_blocks)


def token_mask_from_blocks(block_mask: torch.Tensor, route_block: int, seq_len: int,
                           is_causal: bool = False) -> torch.Tensor:
    """Expand a (..., NB, NB) block mask to a (..., N, N) token mask."""
    m = block_mask.repeat_interleave(route_block, dim=-2).repeat_interleave(route_block, dim=-1)
    m = m[..., :seq_len, :seq_len]
    if is_causal:
        m = m & torch.ones(seq_len, seq_len, dtype=torch.bool, device=m.device).tril()
    return m


def masked_reference_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                               token_mask: torch.Tensor,
                               sm_scale: Optional[float] = None) -> torch.Tensor:
    """fp32 masked attention reference; returns q.dtype."""
    scale = sm_scale if sm_scale is not None else 1.0 / math.sqrt(q.shape[-1])
    s = torch.matmul(q.float(), k.float().transpose(-2, -1)) * scale
    s = s.masked_fill(~token_mask, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v.float()).to(q.dtype)
