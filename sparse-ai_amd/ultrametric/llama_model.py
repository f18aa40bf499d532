"""A Llama-3.1-8B-shaped decoder whose attention runs on the block-list kernels.

This is the model-side caller of the hot path at full size, as the reference's
end-to-end prefill benchmark drives it (experiments/bench_surgery_prefill.py:
81-108 ``AttnTimer``, :146-178 ``run_condition``): ``model(input_ids)`` runs
every decoder layer without the LM head, and each layer's attention is either
dense causal SDPA (the unmodified model, the reference's ``dense_sdpa``
condition) or the surgery prefill (``block_list@r``): per-token tree-routing
scores -> route-block majority vote -> sync-free causal + sink + local block
lists -> block-sparse attention with native GQA
(src/llama_surgery/surgery.py:521-601, ``block_list_prefill`` here).

The reference loads trained Llama-3.1-8B weights and a learned router; there is
no network here, so the weights are random (normal, std 0.02, seeded) in
bf16 and each layer's routing scores are seeded N(0, 1) logits of shape
(B, H, S, levels, p), as the benchmark configuration states. Only the shapes
and the work per token matter for the timing: hidden 4096, 32 layers, 32
query / 8 key-value heads of dimension 128, SwiGLU width 14336, vocabulary
128256, RoPE with theta 5e5 (unscaled), RMSNorm eps 1e-5.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn.functional as F

from .paged_cache import PagedKVCache, token_routing_codes
from .surgery import RouteCache, block_list_prefill

__all__ = ["LlamaShape", "LLAMA31_8B", "SurgeryLlama", "rope_tables", "apply_rope"]


@dataclass(frozen=True)
class LlamaShape:
    hidden: int = 4096
    layers: int = 32
    heads: int = 32
    kv_heads: int = 8
    intermediate: int = 14336
    vocab: int = 128256
    rope_theta: float = 500000.0
    rms_eps: float = 1e-5

    @property
    def head_dim(self) -> int:
        return self.hidden // self.heads


LLAMA31_8B = LlamaShape()


def rope_tables(seq_len: int, head_dim: int, theta: float, device, dtype=torch.float32):
    """cos / sin tables (seq_len, head_dim) of the rotate-half RoPE convention."""
    inv = 1.0 / (theta ** (torch.arange(0, head_dim, 2, device=device, dtype=torch.float32) / head_dim))
    t = torch.arange(seq_len, device=device, dtype=torch.float32)
    f = torch.outer(t, inv)
    emb = torch.cat([f, f], dim=-1)
    return emb.cos().to(dtype), emb.sin().to(dtype)


def apply_rope(x: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor) -> torch.Tensor:
    """x: (B, H, S, D) rotated by position (rotate-half form)."""
    h = x.shape[-1] // 2
    rot = torch.cat([-x[..., h:], x[..., :h]], dim=-1)
    return x * cos + rot * sin


def _rms_norm(x: torch.Tensor, w: torch.Tensor, eps: float) -> torch.Tensor:
    xf = x.float()
    return (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + eps)).to(x.dtype) * w


class SurgeryLlama:
    """Random-init Llama-shaped decoder (no LM head) with switchable attention.

    ``attention``: "sdpa" (dense causal, torch's scaled_dot_product_attention
    with GQA) or "block_list" (the surgery prefill over the HIP kernels).
    ``r``: routed levels; ``p``: branches per level; ``levels``: router depth.
    Weights live on ``device`` in ``dtype``; routing scores are generated per
    (layer, sequence length) from ``seed`` and kept.
    """

    def __init__(self, shape: LlamaShape = LLAMA31_8B, *, device="cuda", dtype=torch.bfloat16, seed: int = 0,
                 r: int = 2, p: int = 4, levels: int = 4, route_block: int = 128, local_window: int = 16,
                 route_stride: int = 1):
        self.shape, self.device, self.dtype = shape, torch.device(device), dtype
        self.r, self.p, self.levels = int(r), int(p), int(levels)
        self.route_block, self.local_window = int(route_block), int(local_window)
        self.route_cache = RouteCache(route_stride)
        self.seed = seed
        g = torch.Generator(device=self.device).manual_seed(seed)
        d, hd = shape.hidden, shape.head_dim

        def w(*s):
            return (torch.randn(*s, generator=g, device=self.device, dtype=torch.float32) * 0.02).to(dtype)

        self.embed = w(shape.vocab, d)
        self.layers: List[dict] = []
        for _ in range(shape.layers):
            self.layers.append({
                "ln1": torch.ones(d, device=self.device, dtype=dtype),
                "wq": w(shape.heads * hd, d), "wk": w(shape.kv_heads * hd, d), "wv": w(shape.kv_heads * hd, d),
                "wo": w(d, shape.heads * hd),
                "ln2": torch.ones(d, device=self.device, dtype=dtype),
                "wg": w(shape.intermediate, d), "wu": w(shape.intermediate, d), "wd": w(d, shape.intermediate),
            })
        self.norm = torch.ones(d, device=self.device, dtype=dtype)
        self._scores = {}
        self._rope = {}
        self.attention = "block_list"
        self.attn_events: Optional[list] = None   # (start, end) CUDA events per layer when set to a list
        self.last_stats: Optional[list] = None
        self._fill: Optional[PagedKVCache] = None  # cache that a forward writes its K / V into
        self.bits_per_level = max(1, (self.p - 1).bit_length())

    # -- routing scores ---------------------------------------------------------------
    def routing_scores(self, layer: int, batch: int, seq_len: int) -> torch.Tensor:
        """Seeded N(0, 1) per-token branch scores (B, H, S, levels, p) of one layer (bf16)."""
        key = (layer, batch, seq_len)
        s = self._scores.get(key)
        if s is None:
            g = torch.Generator(device=self.device).manual_seed(self.seed * 1000003 + layer)
            s = torch.randn(batch, self.shape.heads, seq_len, self.levels, self.p, generator=g,
                            device=self.device, dtype=torch.float32).to(torch.bfloat16)
            self._scores[key] = s
        return s

    def _rope_for(self, seq_len: int):
        t = self._rope.get(seq_len)
        if t is None:
            t = rope_tables(seq_len, self.shape.head_dim, self.shape.rope_theta, self.device, self.dtype)
            self._rope[seq_len] = t
        return t

    # -- blocks ------------------------------------------------------------------------
    def qkv(self, layer: int, x: torch.Tensor):
        """Normed input -> RoPE'd q (B, H, S, D), k, v (B, H_kv, S, D)."""
        L, sh = self.layers[layer], self.shape
        B, S, _ = x.shape
        hd = sh.head_dim
        q = F.linear(x, L["wq"]).view(B, S, sh.heads, hd).transpose(1, 2)
        k = F.linear(x, L["wk"]).view(B, S, sh.kv_heads, hd).transpose(1, 2)
        v = F.linear(x, L["wv"]).view(B, S, sh.kv_heads, hd).transpose(1, 2)
        cos, sin = self._rope_for(S)
        return apply_rope(q, cos, sin), apply_rope(k, cos, sin), v

    def core_attention(self, layer: int, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                       collect_stats: bool = False):
        sh = self.shape
        scale = 1.0 / math.sqrt(sh.head_dim)
        if self.attention == "sdpa":
            # the unmodified model's path: key / value heads repeated to the
            # query heads (transformers' repeat_kv), then torch's fused SDPA
            group = sh.heads // sh.kv_heads
            if group > 1:
                k = k.repeat_interleave(group, dim=1)
                v = v.repeat_interleave(group, dim=1)
            return F.scaled_dot_product_attention(q, k, v, is_causal=True, scale=scale)
        if self.attention != "block_list":
            raise ValueError(f"attention must be 'sdpa' or 'block_list', not {self.attention!r}")
        scores = self.routing_scores(layer, q.shape[0], q.shape[2])
        res = block_list_prefill(q, k, v, scores, self.r, p=self.p, route_block=self.route_block,
                                 local_window=self.local_window, sm_scale=scale, return_stats=collect_stats,
                                 route_cache=self.route_cache, layer_idx=layer)
        if collect_stats:
            out, st = res
            self.last_stats.append(st)
            return out
        return res

    def attention_block(self, layer: int, x: torch.Tensor, collect_stats: bool = False) -> torch.Tensor:
        """Projections, RoPE, routing, attention and output projection of one layer."""
        B, S, _ = x.shape
        q, k, v = self.qkv(layer, x)
        if self._fill is not None:
            levels = self.routing_scores(layer, B, S)[..., :self.levels, :].argmax(-1)   # (B, H, S, levels)
            self._fill.write(layer, k, v, token_routing_codes(levels, self.bits_per_level))
        o = self.core_attention(layer, q, k, v, collect_stats)
        o = o.transpose(1, 2).reshape(B, S, self.shape.heads * self.shape.head_dim)
        return F.linear(o, self.layers[layer]["wo"])

    def mlp(self, layer: int, x: torch.Tensor) -> torch.Tensor:
        L = self.layers[layer]
        return F.linear(F.silu(F.linear(x, L["wg"])) * F.linear(x, L["wu"]), L["wd"])

    @torch.no_grad()
    def __call__(self, input_ids: torch.Tensor, *, layers: Optional[int] = None,
                 collect_stats: bool = False) -> torch.Tensor:
        """Final hidden states (B, S, hidden) of the first ``layers`` decoder layers (all by default)."""
        sh = self.shape
        n = sh.layers if layers is None else int(layers)
        x = F.embedding(input_ids, self.embed)
        self.route_cache.clear()
        if collect_stats:
            self.last_stats = []
        for li in range(n):
            L = self.layers[li]
            h = _rms_norm(x, L["ln1"], sh.rms_eps)
            if self.attn_events is not None:
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                a = self.attention_block(li, h, collect_stats)
                e.record()
                self.attn_events.append((s, e))
            else:
                a = self.attention_block(li, h, collect_stats)
            x = x + a
            x = x + self.mlp(li, _rms_norm(x, L["ln2"], sh.rms_eps))
        return _rms_norm(x, self.norm, sh.rms_eps)

    # -- serving: paged prefill and single-token decode -----------------------------------
    def new_cache(self, max_seqs: int, max_tokens: int, page_size: int = 16, num_pages: Optional[int] = None,
                  layers: Optional[int] = None) -> PagedKVCache:
        """A paged cache for ``layers`` layers (all by default), room for ``max_tokens`` per sequence."""
        sh = self.shape
        max_pages = -(-max_tokens // page_size)
        return PagedKVCache(num_pages or max_seqs * max_pages, page_size, sh.kv_heads, sh.head_dim, heads=sh.heads,
                            tree_depth=self.levels, bits_per_level=self.bits_per_level, max_seqs=max_seqs,
                            max_pages_per_seq=max_pages, layers=sh.layers if layers is None else layers,
                            dtype=self.dtype, device=self.device)

    @torch.no_grad()
    def prefill(self, cache: PagedKVCache, input_ids: torch.Tensor, *, layers: Optional[int] = None) -> torch.Tensor:
        """Prompt forward (the block-list or SDPA condition) that also stores every layer's
        K / V and page codes (first token of each page, from that layer's routing
        scores) in rows 0 .. B-1 of ``cache``, which must be empty there."""
        B, S = input_ids.shape
        if any(cache.lengths[b] for b in range(B)):
            raise ValueError("prefill needs empty cache rows")
        cache.reserve(S, rows=range(B))
        cache.advance(S, B)
        self._fill = cache
        try:
            return self(input_ids, layers=layers)
        finally:
            self._fill = None

    def decode_levels(self, scores: torch.Tensor) -> torch.Tensor:
        """(B, H, levels, p) routing scores of new tokens -> (B, H) int32 packed codes."""
        lv = scores[..., :self.levels, :].argmax(-1).to(torch.int32)
        return token_routing_codes(lv.unsqueeze(2), self.bits_per_level)[:, :, 0]

    def local_pages(self, page_size: int) -> int:
        """Trailing pages that cover the local window ending at the new token."""
        return 0 if self.local_window <= 0 else -(-self.local_window // page_size) + 1

    @torch.no_grad()
    def decode_step(self, cache: PagedKVCache, input_ids: torch.Tensor, scores: torch.Tensor, *,
                    layers: Optional[int] = None) -> torch.Tensor:
        """One new token per row 0 .. B-1: input_ids (B,), scores (layers, B, H, levels, p)
        routing scores of the new tokens. The reference's eager decode mask
        (src/llama_surgery/surgery.py:880-955: the token's branch over r levels equal to
        a past token's, a local window, token 0) becomes page selection over the paged
        cache: a page whose first token's code matches the new token's on r levels,
        page 0 (the sink) and the pages of the local window. Every launch reads its
        sizes from the device (lengths, tables), so the step can be captured in a HIP
        graph once ``cache.reserve`` has pages for it. Returns hidden states (B, hidden)."""
        sh = self.shape
        n = sh.layers if layers is None else int(layers)
        B = input_ids.shape[0]
        pos = cache.context_lens[:B].long()              # position of the new token
        cache.advance(1, B)
        cos, sin = self._rope_for(cache.max_pages * cache.page_size)
        cos, sin = cos[pos][:, None, None, :], sin[pos][:, None, None, :]
        x = F.embedding(input_ids, self.embed)[:, None, :]   # (B, 1, hidden)
        hd = sh.head_dim
        for li in range(n):
            L = self.layers[li]
            h = _rms_norm(x, L["ln1"], sh.rms_eps)
            q = F.linear(h, L["wq"]).view(B, sh.heads, 1, hd)
            k = F.linear(h, L["wk"]).view(B, sh.kv_heads, 1, hd)
            v = F.linear(h, L["wv"]).view(B, sh.kv_heads, 1, hd)
            q, k = apply_rope(q, cos, sin), apply_rope(k, cos, sin)
            codes = self.decode_levels(scores[li])
            cache.write(li, k, v, codes.unsqueeze(-1))
            o = cache.decode(li, q[:, :, 0], codes, self.r, local_blocks=self.local_pages(cache.page_size),
                             sink_block=True)
            x = x + F.linear(o.reshape(B, 1, sh.heads * hd), L["wo"])
            x = x + self.mlp(li, _rms_norm(x, L["ln2"], sh.rms_eps))
        return _rms_norm(x, self.norm, sh.rms_eps)[:, 0]
