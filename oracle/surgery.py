"""Surgery-caller oracle (numpy) — test infrastructure only.

Restates, on the CPU, the block routing and statistics of
SurgicalLlamaAttention._block_list_prefill (src/llama_surgery/surgery.py):
  * ``majority_route``   surgery.py:543-547 — per route block and level, the
    branch chosen by most tokens' argmax (one-hot votes summed over the block,
    tokens past S padded with zero votes, argmax of the counts: lowest branch
    id on ties); ``direct_route`` surgery.py:536-541 — argmax per block row.
  * ``local_blocks_of``  surgery.py:550-551 — ceil(local_window / RB), 0 when
    local_window <= 0.
  * ``allowed_key_stats`` surgery.py:589-595 — mean allowed keys per query
    (sum over listed blocks of RB*len, the diagonal block causal), mean causal
    keys (S + 1) / 2 and listed-block density.

Pinned by (tests/test_oracle_surgery.py): the reference test's own independent
construction, a Python loop of bincount + argmax per block and level
(tests/test_surgery_block_list.py:42-55), on its parameter grid; hand-made
blocks whose winner is forced (unanimous, ties between two branches, a tail
block shorter than RB); and the allowed-key mean against the row sums of the
token mask built from the same lists (tests/test_surgery_block_list.py:93-95).
"""

from __future__ import annotations

import numpy as np


def direct_route(block_assign: np.ndarray, r: int) -> np.ndarray:
    """surgery.py:536-541: (B, H, NB, L, p) scores -> (B, H, NB, r) int32 argmax."""
    return block_assign[:, :, :, :r, :].argmax(-1).astype(np.int32)


def majority_route(assign: np.ndarray, r: int, route_block: int) -> np.ndarray:
    """surgery.py:543-547: (B, H, S, L, p) scores -> (B, H, NB, r) int32 majority branches."""
    B, H, S, L, p = assign.shape
    NB = -(-S // route_block)
    idx = assign[:, :, :, :r, :].argmax(-1)                       # (B, H, S, r), first max
    votes = np.eye(p, dtype=np.float64)[idx]                      # (B, H, S, r, p)
    pad = NB * route_block - S
    if pad:
        votes = np.concatenate([votes, np.zeros((B, H, pad, r, p))], axis=2)
    counts = votes.reshape(B, H, NB, route_block, r, p).sum(3)
    return counts.argmax(-1).astype(np.int32)                     # lowest id on ties


def local_blocks_of(local_window: int, route_block: int) -> int:
    """surgery.py:550-551."""
    return -(-local_window // route_block) if local_window > 0 else 0


def allowed_key_stats(counts: np.ndarray, seq_len: int, route_block: int) -> dict:
    """surgery.py:589-595 on (B, H, NB) list counts of causal lists."""
    NB = counts.shape[-1]
    lens = np.full(NB, route_block, dtype=np.float64)
    lens[-1] = seq_len - (NB - 1) * route_block
    c = counts.astype(np.float64)
    allowed = ((c - 1) * route_block * lens + lens * (lens + 1) / 2).sum(-1)
    B, H = counts.shape[:2]
    return {
        "mean_allowed_keys": float(allowed.mean() / seq_len),
        "mean_causal_keys": (seq_len + 1) / 2,
        "block_density": float(c.sum() / (B * H * NB * (NB + 1) / 2)),
    }
