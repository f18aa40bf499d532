"""Seeded synthetic workloads for the BASELINE configurations.

Every generator is deterministic from its seed (torch.Generator on the CPU,
or on the target device for the multi-GB decode caches). Shapes follow
BASELINE.json `configs`; routing patterns follow the reference benchmark
helpers (benchmarks/benchmark_block_list.py:84-98 for the tree layout of
routing ids, MSB level first).
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Optional

import torch


def _gen(seed: int, device="cpu") -> torch.Generator:
    return torch.Generator(device=device).manual_seed(seed)


def randn_qkv(Z, H, N, D, dtype, seed, device="cpu", H_kv=None):
    """Q/K/V ~ N(0, 1) drawn in fp32 on the CPU from `seed`, then cast."""
    g = _gen(seed)
    H_kv = H if H_kv is None else H_kv
    q = torch.randn(Z, H, N, D, generator=g, dtype=torch.float32)
    k = torch.randn(Z, H_kv, N, D, generator=g, dtype=torch.float32)
    v = torch.randn(Z, H_kv, N, D, generator=g, dtype=torch.float32)
    return tuple(t.to(dtype).to(device) for t in (q, k, v))


def leaf_digits(leaf: torch.Tensor, p: int, depth: int) -> torch.Tensor:
    """Base-p digits of leaf ids, most significant (root level) first: (..., depth) int32."""
    return torch.stack([(leaf // p ** (depth - 1 - d)) % p for d in range(depth)], dim=-1).to(torch.int32)


def bernoulli_block_mask(Z, H, NB, density, seed):
    """Per-head Bernoulli(density) over the lower-triangular blocks, diagonal and sink (block 0)
    forced on (configs 1 and 3). Returns (Z, H, NB, NB) bool."""
    g = _gen(seed)
    m = torch.rand(Z, H, NB, NB, generator=g) < density
    m &= torch.ones(NB, NB, dtype=torch.bool).tril()
    idx = torch.arange(NB)
    m[..., idx, idx] = True
    m[..., :, 0] = True
    return m


# ---- config 1 -----------------------------------------------------------------------

def config1(seed=1, device="cpu"):
    """fp32, B=1 H=4 N=1024 D=64, block 64x64, causal, Bernoulli(0.25) mask + diag + sink."""
    Z, H, N, D, RB = 1, 4, 1024, 64, 64
    q, k, v = randn_qkv(Z, H, N, D, torch.float32, seed, device)
    mask = bernoulli_block_mask(Z, H, N // RB, 0.25, seed + 1000).to(device)
    return dict(q=q, k=k, v=v, block_mask=mask, route_block=RB, is_causal=True)


# ---- config 2 -----------------------------------------------------------------------

def tree_leaf_router(Z, H, NB, p, depth, seed):
    """Per head: a random permutation assigns the NB blocks to the NB = p^depth leaves
    of a p-ary tree; router ids are the leaf's digits (root first)."""
    assert NB == p ** depth
    g = _gen(seed)
    leaves = torch.stack([torch.stack([torch.randperm(NB, generator=g) for _ in range(H)])
                          for _ in range(Z)])
    return leaf_digits(leaves, p, depth)  # (Z, H, NB, depth)


def config2(seed=2, device="cpu", dtype=torch.bfloat16, N=8192, H=32):
    """bf16, B=1 H=32 N=8192 D=128, route block 128 (64 blocks = leaves of a p=4 depth-3
    tree, random leaf permutation per head), block (i, j) routed iff LCA depth >= 2,
    plus diagonal and sink, causal. Lists via the sync-free builder (arity 4)."""
    Z, D, RB, p, depth = 1, 128, 128, 4, 3
    NB = N // RB
    q, k, v = randn_qkv(Z, H, N, D, dtype, seed, device)
    router = tree_leaf_router(Z, H, NB, p, depth, seed + 1000).to(device)
    return dict(q=q, k=k, v=v, router=router, req_depth=2, arity=p, sink_block=True,
                route_block=RB, is_causal=True)


# ---- config 3 -----------------------------------------------------------------------

def config3(N, density, seed=3, device="cpu", H=32, dtype=torch.bfloat16):
    """bf16, B=1 H=32 D=128 causal, route block 128, per-head Bernoulli(density) lower
    triangle + diagonal + sink."""
    Z, D, RB = 1, 128, 128
    q, k, v = randn_qkv(Z, H, N, D, dtype, seed, device)
    mask = bernoulli_block_mask(Z, H, N // RB, density, seed + int(density * 1e6)).to(device)
    return dict(q=q, k=k, v=v, block_mask=mask, route_block=RB, is_causal=True)


# ---- config 4 -----------------------------------------------------------------------

@dataclass
class DecodeWorkload:
    q: torch.Tensor
    k_cache: torch.Tensor
    v_cache: torch.Tensor
    block_tables: torch.Tensor
    context_lens: torch.Tensor
    router: torch.Tensor
    q_router: torch.Tensor
    req_depth: int
    local_blocks: int
    sink_block: bool


def config4(seed=4, device="cpu", B=64, H=32, H_kv=8, D=128, page=16, min_len=4096,
            max_len=32768, p=4, depth=4, dtype=torch.bfloat16, kv_seed_device=None):
    """Sparse paged decode: B sequences with KV length ~ U[min_len, max_len], GQA H/H_kv,
    page size `page`, physical pages shuffled; router per (physical page, query head) and
    q_router per (sequence, query head) = base-p digits of a uniform leaf in [0, p^depth);
    req_depth = depth, sink page and last 4 pages forced. K/V ~ N(0, 1) drawn on
    `kv_seed_device` (default: `device`) from the seed."""
    g = _gen(seed)
    lens = torch.randint(min_len, max_len + 1, (B,), generator=g, dtype=torch.int64)
    n_pages = (lens + page - 1) // page
    total = int(n_pages.sum())
    max_pages = int(n_pages.max())
    perm = torch.randperm(total, generator=g).to(torch.int32)
    tables = torch.zeros(B, max_pages, dtype=torch.int32)
    off = 0
    for b in range(B):
        n = int(n_pages[b])
        tables[b, :n] = perm[off:off + n]
        off += n
    leaves = p ** depth
    router = leaf_digits(torch.randint(0, leaves, (total, H), generator=g), p, depth)
    q_router = leaf_digits(torch.randint(0, leaves, (B, H), generator=g), p, depth)
    q = torch.randn(B, H, D, generator=g, dtype=torch.float32).to(dtype)
    kv_dev = kv_seed_device or device
    gk = _gen(seed + 1, kv_dev)
    k_cache = torch.randn(total, H_kv, page, D, generator=gk, dtype=torch.float32, device=kv_dev).to(dtype)
    v_cache = torch.randn(total, H_kv, page, D, generator=gk, dtype=torch.float32, device=kv_dev).to(dtype)
    return DecodeWorkload(q.to(device), k_cache.to(device), v_cache.to(device), tables.to(device),
                          lens.to(torch.int32).to(device), router.to(device), q_router.to(device),
                          req_depth=depth, local_blocks=4, sink_block=True)


# ---- accounting ---------------------------------------------------------------------

def prefill_flops(counts: torch.Tensor, head_dim: int, route_block: int) -> float:
    """Algorithmic FLOPs on computed tiles: 4 * D * RB^2 per listed block pair
    (QK^T and PV, 2 FLOPs per multiply-add), diagonal tiles counted in full."""
    return 4.0 * head_dim * route_block * route_block * float(counts.to(torch.float64).sum())


def useful_prefill_flops(block_mask: torch.Tensor, route_block: int, seq_len: int, head_dim: int,
                         is_causal: bool) -> float:
    """Token-exact FLOPs: 4 * D per visible (query, key) pair."""
    NB = block_mask.shape[-1]
    lens = torch.full((NB,), route_block, dtype=torch.float64)
    lens[-1] = seq_len - (NB - 1) * route_block
    bm = block_mask.to(torch.float64).cpu()
    if not is_causal:
        pairs = (bm * lens[:, None] * lens[None, :]).sum()
    else:
        below = torch.ones(NB, NB, dtype=torch.float64).tril(-1)
        idx = torch.arange(NB)
        pairs = (bm * below * lens[:, None] * lens[None, :]).sum() \
            + (bm[..., idx, idx] * lens * (lens + 1) / 2).sum()
    return 4.0 * head_dim * float(pairs)


def decode_routed_bytes(w: DecodeWorkload, elem_bytes: Optional[int] = None):
    """Algorithmic decode bytes (config 4 metric): every (sequence, kv head, physical page)
    selected by at least one query head of the GQA group counts once, as valid tokens x D x
    (K and V) x element bytes. Returns (bytes, unique pages)."""
    B, H, D = w.q.shape
    Hkv, page = w.k_cache.shape[1], w.k_cache.shape[2]
    G = H // Hkv
    eb = elem_bytes or w.k_cache.element_size()
    r = min(max(int(w.req_depth), 0), w.q_router.shape[-1])
    tokens = 0
    pages = 0
    for b in range(B):
        ctx = int(w.context_lens[b])
        if ctx <= 0:
            continue
        n = (ctx + page - 1) // page
        phys = w.block_tables[b, :n].long()
        if r > 0:
            m = (w.router[phys, :, :r] == w.q_router[b, :, :r][None]).all(-1)
        else:
            m = torch.ones(n, H, dtype=torch.bool, device=w.router.device)
        sel = m.view(n, Hkv, G).any(-1)
        if w.sink_block:
            sel[0] = True
        if w.local_blocks > 0:
            sel[max(0, n - w.local_blocks):] = True
        valid = torch.clamp(ctx - torch.arange(n, device=sel.device) * page, max=page)
        tokens += int((sel * valid[:, None]).sum())
        pages += int(sel.sum())
    return tokens * D * 2 * eb, pages


def lists_to_block_mask(lists: torch.Tensor, counts: torch.Tensor) -> torch.Tensor:
    """(Z, H, NB, NB) bool mask of the listed (query block, key block) pairs."""
    Z, H, NB = counts.shape
    mc = lists.shape[-1]
    t = torch.arange(mc, device=lists.device).view(1, 1, 1, mc)
    valid = t < counts.unsqueeze(-1)
    idx = torch.where(valid, lists.long(), torch.full_like(lists, NB, dtype=torch.long))
    m = torch.zeros(Z, H, NB, NB + 1, dtype=torch.bool, device=lists.device)
    m.scatter_(-1, idx, valid)
    return m[..., :NB]
