"""Quick-start block-sparse attention (drop-in for src/ultrametric/kernel.py:520-580).

``block_sparse_attention`` keeps the reference's signature and return value
``(out, lse)``; it pads / truncates the router to ceil(N / route_block)
blocks with branch 0, builds exact-size lists (validating ids, host syncs as
in the reference) and runs the HIP block-list kernel. The reference falls
back to an fp32 torch computation on CPU (kernel.py:574-580); this build has
no CPU fallback and raises RuntimeError for non-HIP tensors.
"""

from __future__ import annotations

import math

import torch

from .block_list import HAS_TRITON, block_list_attention, build_block_lists

__all__ = ["HAS_TRITON", "block_sparse_attention", "routing_to_block_indices"]


def block_sparse_attention(
    q: torch.Tensor,
    k: torch.Tensor,
    v: torch.Tensor,
    router_indices: torch.Tensor,
    req_depth: int = 2,
    p: int = 2,
    is_causal: bool = False,
    route_block: int = 128,
):
    """Block-sparse routed attention forward (inference); returns (out, lse).

    router_indices: (Z, H, num_blocks, tree_depth) non-negative branch ids, one
    routing vector per ``route_block`` tokens; missing blocks are padded with
    branch 0, extra blocks dropped. ``p`` is informational (kernel.py:541).
    """
    Z, H, N, D = q.shape
    router_indices = router_indices.to(torch.int64)
    nb = -(-N // route_block)
    have = router_indices.shape[2]
    if have < nb:
        pad = torch.zeros((Z, H, nb - have, router_indices.shape[-1]), dtype=router_indices.dtype,
                          device=router_indices.device)
        router_indices = torch.cat([router_indices, pad], dim=2)
    elif have > nb:
        router_indices = router_indices[:, :, :nb]
    bl = build_block_lists(router_indices, req_depth, is_causal=is_causal)
    return block_list_attention(q, k, v, bl, route_block=route_block, is_causal=is_causal,
                                return_lse=True)


def routing_to_block_indices(assignments: torch.Tensor, seq_len: int, block_size: int = 128) -> torch.Tensor:
    """Per-block routing ids from one-hot token assignments (kernel.py:152-191).

    As in the reference, each block takes its FIRST token's argmax branch per
    level (not a majority vote). Returns (B, H, num_blocks, levels) int32.
    """
    B, H, S, L, P = assignments.shape
    num_blocks = math.ceil(seq_len / block_size)
    branch_ids = assignments.argmax(dim=-1)
    if S < num_blocks * block_size:
        branch_ids = torch.nn.functional.pad(branch_ids, (0, 0, 0, num_blocks * block_size - S), value=0)
    branch_ids = branch_ids.view(B, H, num_blocks, block_size, L)
    return branch_ids[:, :, :, 0, :].to(torch.int32)
