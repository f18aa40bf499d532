"""Sparse paged decode on MI355X (drop-in for src/ultrametric/kernel_decode.py).

``ultrametric_decode`` keeps the reference signature (kernel_decode.py:188-199)
and runs the HIP split-KV decode kernels of libsparseattn.so on torch's
current stream. Extensions: GQA (k_cache / v_cache may carry H_kv | H heads;
query head h reads kv head h // (H / H_kv)); ``context_lens <= 0`` yields
zeros, as the reference's CPU reference does (kernel_decode.py:145-147).
Block-table entries outside [0, num_pages) are treated as unselected pages
and logical pages beyond block_tables.shape[1] are ignored (memory safety).

``_ultrametric_decode_reference`` keeps the reference's torch loop
(kernel_decode.py:129-185) for callers' checks; ``ultrametric_decode`` never
calls it and has no CPU fallback.
"""

from __future__ import annotations

import torch

from . import _native as nat

HAS_TRITON = nat.available()

__all__ = ["HAS_TRITON", "ultrametric_decode", "_ultrametric_decode_reference", "decode_workspace_bytes",
           "pack_routing_codes", "ultrametric_decode_packed", "sequence_page_codes",
           "ultrametric_decode_seq_codes"]


def decode_workspace_bytes(batch_size: int, num_heads: int, head_dim: int, max_pages: int,
                           num_kv_heads: int = None) -> int:
    """Bytes of split-KV scratch the decode kernels need (0: none).

    ``num_kv_heads`` defaults to ``num_heads`` (no GQA)."""
    hkv = num_heads if num_kv_heads is None else num_kv_heads
    return int(nat.lib().sa_decode_workspace_bytes(batch_size, num_heads, hkv, head_dim, max_pages))


def ultrametric_decode(
    q,
    k_cache,
    v_cache,
    block_tables,
    context_lens,
    router_indices,
    q_router_indices,
    req_depth,
    local_blocks: int = 0,
    sink_block: bool = False,
    workspace: torch.Tensor = None,
):
    """Decode one query token per sequence against routed KV pages.

    q: (B, H, D); k_cache, v_cache: (num_pages, H_kv, page_size, D);
    block_tables: (B, max_pages) int; context_lens: (B,) int;
    router_indices: (num_pages, H, TD) int; q_router_indices: (B, H, TD) int.
    ``workspace`` (optional, uint8, >= decode_workspace_bytes(...)) avoids a
    per-call allocation. Returns (B, H, D) in q.dtype.
    """
    tree_depth = int(q_router_indices.shape[-1])
    assert tree_depth >= 1, "tree_depth must be >= 1"
    rt = router_indices if router_indices.dtype == torch.int32 else router_indices.to(torch.int32)
    qrt = q_router_indices if q_router_indices.dtype == torch.int32 else q_router_indices.to(torch.int32)
    return _decode(q, k_cache, v_cache, block_tables, context_lens, rt, qrt, tree_depth, 0, req_depth,
                   local_blocks, sink_block, workspace)


def pack_routing_codes(router_indices: torch.Tensor, bits_per_level: int) -> torch.Tensor:
    """Pack (rows, H, TD) routing levels into one 32-bit code per (row, head).

    Level l lands in bits [bpl*(TD-1-l), bpl*(TD-l)) (level 0 most significant),
    so a depth-r prefix match of two rows is equality of their top bpl*r bits.
    Every level must lie in [0, 2**bits_per_level); TD * bits_per_level <= 32.
    Returns a (rows, H) int32 tensor holding the uint32 bit patterns. Used once
    per page write (the router of a page does not change), then passed to
    ``ultrametric_decode_packed`` on every step.
    """
    if router_indices.dim() != 3:
        raise ValueError(f"router_indices must be (rows, H, TD); got {tuple(router_indices.shape)}")
    dev = nat.require_device(router_indices)
    rows, H, TD = router_indices.shape
    rt = router_indices if router_indices.dtype == torch.int32 else router_indices.to(torch.int32)
    out = torch.empty((rows, H), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        rc = nat.lib().sa_pack_page_codes(nat.ptr(rt), nat.strides(rt), rows, H, TD, int(bits_per_level),
                                          nat.ptr(out), nat.stream(dev))
    nat.check(rc)
    return out


def ultrametric_decode_packed(q, k_cache, v_cache, block_tables, context_lens, page_codes, q_codes,
                              tree_depth: int, bits_per_level: int, req_depth, local_blocks: int = 0,
                              sink_block: bool = False, workspace: torch.Tensor = None):
    """``ultrametric_decode`` with the routing vectors given as packed codes.

    page_codes: (num_pages, H) and q_codes: (B, H), int32 tensors from
    ``pack_routing_codes(router, bits_per_level)`` of a router with
    ``tree_depth`` levels. Reads one 32-bit word per (page, head) where the
    unpacked form reads tree_depth of them; the output is the same.
    """
    if page_codes.dim() != 2 or q_codes.dim() != 2:
        raise ValueError("page_codes must be (num_pages, H) and q_codes (B, H)")
    if page_codes.dtype != torch.int32 or q_codes.dtype != torch.int32:
        raise ValueError("page_codes / q_codes must be int32 (as pack_routing_codes returns)")
    return _decode(q, k_cache, v_cache, block_tables, context_lens, page_codes, q_codes, int(tree_depth),
                   int(bits_per_level), req_depth, local_blocks, sink_block, workspace)


_CODE_DTYPES = {1: torch.uint8, 2: torch.int16, 4: torch.int32}


def sequence_page_codes(page_codes: torch.Tensor, block_tables: torch.Tensor, bits: int = 32) -> torch.Tensor:
    """(num_pages, H) page codes -> (B, H, max_pages) codes in each sequence's logical page
    order, the layout ``ultrametric_decode_seq_codes`` reads, stored in the narrowest of
    1 / 2 / 4 bytes that holds ``bits`` (= tree depth x bits per level). A serving cache
    appends one column per new page instead of regathering; entries for table slots outside
    [0, num_pages) are arbitrary (the decode never selects those pages)."""
    width = 1 if bits <= 8 else (2 if bits <= 16 else 4)
    idx = block_tables.long().clamp(0, page_codes.shape[0] - 1)
    return page_codes[idx].permute(0, 2, 1).to(_CODE_DTYPES[width]).contiguous()


def ultrametric_decode_seq_codes(q, k_cache, v_cache, block_tables, context_lens, seq_codes, q_codes,
                                 tree_depth: int, bits_per_level: int, req_depth, local_blocks: int = 0,
                                 sink_block: bool = False, workspace: torch.Tensor = None):
    """``ultrametric_decode`` with routing codes stored per sequence, in logical page order:
    seq_codes (B, H, max_pages) uint8 / int16 / int32 (bit patterns of ``pack_routing_codes``,
    see ``sequence_page_codes``), q_codes (B, H) int32. Same output as
    ``ultrametric_decode_packed`` on the same codes."""
    if seq_codes.dim() != 3 or q_codes.dim() != 2:
        raise ValueError("seq_codes must be (B, H, max_pages) and q_codes (B, H)")
    if seq_codes.dtype not in (torch.uint8, torch.int16, torch.int32) or q_codes.dtype != torch.int32:
        raise ValueError("seq_codes must be uint8 / int16 / int32 and q_codes int32")
    if seq_codes.shape[2] != block_tables.shape[1]:
        raise ValueError("seq_codes must have one column per block-table slot")
    return _decode(q, k_cache, v_cache, block_tables, context_lens, seq_codes, q_codes, int(tree_depth),
                   int(bits_per_level), req_depth, local_blocks, sink_block, workspace, seq=True)


def _decode(q, k_cache, v_cache, block_tables, context_lens, rt, qrt, tree_depth, bpl, req_depth,
            local_blocks, sink_block, workspace, seq=False):
    """Shared validation and launch; bpl == 0 selects the int32-level router form."""
    batch_size, num_heads, head_dim = q.shape
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError(f"k_cache / v_cache must be (pages, H_kv, page, D); got {tuple(k_cache.shape)}, "
                         f"{tuple(v_cache.shape)}")
    if k_cache.shape[3] != head_dim or num_heads % k_cache.shape[1] != 0:
        raise ValueError("k_cache head_dim / head count incompatible with q")
    if not (q.dtype == k_cache.dtype == v_cache.dtype):
        raise ValueError("q, k_cache, v_cache must share dtype")
    dev = nat.require_device(q, k_cache, v_cache, block_tables, context_lens, rt, qrt)
    if k_cache.stride(3) != 1:
        k_cache = k_cache.contiguous()
    if v_cache.stride(3) != 1:
        v_cache = v_cache.contiguous()
    bt = block_tables if block_tables.dtype == torch.int32 else block_tables.to(torch.int32)
    ctx = context_lens.to(torch.int32).contiguous()
    num_pages, H_kv, page_size, _ = k_cache.shape
    max_pages = bt.shape[1]
    out = torch.empty((batch_size, num_heads, head_dim), dtype=q.dtype, device=dev)
    need = decode_workspace_bytes(batch_size, num_heads, head_dim, max_pages, H_kv)
    if need == 0:
        workspace = None
    elif workspace is None or workspace.numel() < need:
        workspace = torch.empty(need, dtype=torch.uint8, device=dev)
    dt = nat.dtype_code(q.dtype, (torch.float32, torch.bfloat16, torch.float16))
    lib = nat.lib()
    head = (nat.ptr(q), nat.ptr(k_cache), nat.ptr(v_cache), nat.ptr(bt), nat.ptr(ctx), nat.ptr(rt),
            nat.ptr(qrt), nat.ptr(out), batch_size, num_heads, H_kv, head_dim, page_size, tree_depth)
    tail = (max_pages, num_pages, int(req_depth), int(local_blocks), int(bool(sink_block)),
            nat.strides(q), nat.strides(k_cache), nat.strides(v_cache), nat.strides(bt),
            nat.strides(rt), nat.strides(qrt), nat.strides(out),
            None if workspace is None else nat.ptr(workspace), 0 if workspace is None else workspace.numel(),
            dt, nat.stream(dev))
    with torch.cuda.device(dev):
        if bpl and seq:
            cbytes = rt.element_size()
            rc = lib.sa_sparse_paged_decode_seq_codes(*head[:5], head[5], cbytes, *head[6:], bpl, *tail)
        elif bpl:
            rc = lib.sa_sparse_paged_decode_codes(*head, bpl, *tail)
        else:
            rc = lib.sa_sparse_paged_decode(*head, *tail)
    nat.check(rc)
    return out


def _ultrametric_decode_reference(q, k_cache, v_cache, block_tables, context_lens, router_indices,
                                  q_router_indices, req_depth, local_blocks: int = 0,
                                  sink_block: bool = False):
    """The reference's torch loop (kernel_decode.py:129-185), GQA by head grouping."""
    batch_size, num_heads, head_dim = q.shape
    group = num_heads // k_cache.shape[1]
    tree_depth = q_router_indices.shape[-1]
    r = min(max(int(req_depth), 0), tree_depth)
    block_size = k_cache.shape[2]
    sm_scale = 1.0 / (head_dim ** 0.5)
    out = torch.zeros_like(q)
    for b in range(batch_size):
        ctx_len = int(context_lens[b].item())
        if ctx_len <= 0:
            continue
        num_logical = (ctx_len + block_size - 1) // block_size
        phys_ids = block_tables[b, :num_logical].long()
        for h in range(num_heads):
            q_vec = q[b, h].float()
            if r > 0:
                match = (router_indices[phys_ids, h, :r] == q_router_indices[b, h, :r].unsqueeze(0)).all(dim=-1)
            else:
                match = torch.ones(num_logical, dtype=torch.bool, device=q.device)
            if sink_block and num_logical > 0:
                match[0] = True
            if local_blocks > 0:
                match[max(0, num_logical - local_blocks):] = True
            if not match.any():
                continue
            k_sel, v_sel = [], []
            for l_idx in range(num_logical):
                if not match[l_idx]:
                    continue
                p_idx = int(phys_ids[l_idx].item())
                valid = min(block_size, ctx_len - l_idx * block_size)
                k_sel.append(k_cache[p_idx, h // group, :valid].float())
                v_sel.append(v_cache[p_idx, h // group, :valid].float())
            scores = torch.matmul(torch.cat(k_sel, 0), q_vec) * sm_scale
            out[b, h] = torch.matmul(torch.softmax(scores, dim=-1), torch.cat(v_sel, 0)).to(q.dtype)
    return out
