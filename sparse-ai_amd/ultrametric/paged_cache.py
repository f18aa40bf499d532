"""Paged KV cache with per-sequence page routing codes: the serving side of
the sparse paged decode.

The reference decodes through a transformers cache that concatenates each
layer's new K / V and an eager token-level mask per step
(src/llama_surgery/surgery.py:880-955: the new token's branch id compared
with every past token's, a local window, token 0 as sink, then a dense
masked softmax over all L keys). Its paged decode kernel
(src/ultrametric/kernel_decode.py:22-124, 188-247) reads a paged layout that
nothing in the reference writes. This module is that writer and the step
around it, at page granularity:

* storage: k / v (layers, P, H_kv, page_size, D); block_tables
  (max_seqs, max_pages) int32; context_lens (max_seqs,) int32; seq_codes
  (layers, max_seqs, H, max_pages) packed routing codes (1, 2 or 4 bytes) in
  logical page order, the layout ``ultrametric_decode_seq_codes`` reads;
* a page's routing code is the code of its first token (the first-token rule
  of ``routing_to_block_indices``, src/ultrametric/kernel.py:152-191), written
  when that token is appended, so a decode step never regathers codes;
* pages come from a host free list (``reserve`` before the steps that need
  them; the captured step itself allocates nothing and reads nothing back);
* a step: ``advance`` (one launch: context_lens += new tokens), then per layer
  ``write`` (one launch: K / V rows and first-token codes) and ``decode``
  (``ultrametric_decode_seq_codes``: routed pages only, split-KV, GQA).

Row b of the tables is the batch row b of the q / k_new tensors given to
``write`` and ``decode``; sequences occupy rows 0 .. B-1 of a step.
"""

from __future__ import annotations

from typing import Optional, Sequence, Union

import torch

from . import _native as nat
from .kernel_decode import _CODE_DTYPES, pack_routing_codes, ultrametric_decode_seq_codes

__all__ = ["PagedKVCache", "token_routing_codes"]

_KV_DTYPES = (torch.float32, torch.bfloat16, torch.float16)


def token_routing_codes(levels: torch.Tensor, bits_per_level: int) -> torch.Tensor:
    """(B, H, T, TD) routing levels of new tokens -> (B, H, T) int32 packed codes
    (the ``pack_routing_codes`` bit layout: level 0 in the most significant field)."""
    if levels.dim() != 4:
        raise ValueError(f"levels must be (B, H, T, TD); got {tuple(levels.shape)}")
    B, H, T, TD = levels.shape
    rows = levels.permute(0, 2, 1, 3).reshape(B * T, H, TD)
    return pack_routing_codes(rows.to(torch.int32), bits_per_level).view(B, T, H).permute(0, 2, 1)


class PagedKVCache:
    """K / V pages, block tables, lengths and page routing codes of up to
    ``max_seqs`` sequences over ``layers`` layers (shared tables and lengths,
    per-layer K / V and codes)."""

    def __init__(self, num_pages: int, page_size: int, kv_heads: int, head_dim: int, *, heads: int,
                 tree_depth: int, bits_per_level: int, max_seqs: int, max_pages_per_seq: int, layers: int = 1,
                 dtype: torch.dtype = torch.bfloat16, device="cuda"):
        if dtype not in _KV_DTYPES:
            raise ValueError(f"dtype must be one of {_KV_DTYPES}")
        if heads % kv_heads:
            raise ValueError("heads must be a multiple of kv_heads")
        bits = tree_depth * bits_per_level
        if not (1 <= bits_per_level and bits <= 32):
            raise ValueError("tree_depth * bits_per_level must lie in [1, 32]")
        self.device = torch.device(device)
        self.num_pages, self.page_size = int(num_pages), int(page_size)
        self.kv_heads, self.head_dim, self.heads = int(kv_heads), int(head_dim), int(heads)
        self.tree_depth, self.bits_per_level = int(tree_depth), int(bits_per_level)
        self.max_seqs, self.max_pages = int(max_seqs), int(max_pages_per_seq)
        self.layers = int(layers)
        shape = (self.layers, self.num_pages, self.kv_heads, self.page_size, self.head_dim)
        self.k = torch.zeros(shape, dtype=dtype, device=self.device)
        self.v = torch.zeros(shape, dtype=dtype, device=self.device)
        # unreserved slots hold -1: a write there is flagged in ``status``, never stored
        self.block_tables = torch.full((self.max_seqs, self.max_pages), -1, dtype=torch.int32, device=self.device)
        self.context_lens = torch.zeros(self.max_seqs, dtype=torch.int32, device=self.device)
        width = 1 if bits <= 8 else (2 if bits <= 16 else 4)
        self.seq_codes = torch.zeros((self.layers, self.max_seqs, self.heads, self.max_pages),
                                     dtype=_CODE_DTYPES[width], device=self.device)
        self.status = torch.zeros(1, dtype=torch.int32, device=self.device)
        # host state: free pages (a stack), each row's pages, each row's length
        self._free = list(range(self.num_pages - 1, -1, -1))
        self._pages = [[] for _ in range(self.max_seqs)]
        self._lens = [0] * self.max_seqs
        self._ws = None

    # -- host bookkeeping ----------------------------------------------------------------
    @property
    def lengths(self):
        """Host copy of the row lengths as ``advance`` left them (graph replays excepted:
        call ``refresh_lengths`` after those)."""
        return list(self._lens)

    def refresh_lengths(self):
        """Reads context_lens back to the host (one device sync)."""
        self._lens = [int(x) for x in self.context_lens.cpu().tolist()]

    def free_pages(self) -> int:
        return len(self._free)

    def reserve(self, tokens: Union[int, Sequence[int]], rows: Optional[Sequence[int]] = None):
        """Allocates pages so that each row can take ``tokens`` more tokens (one int for
        every row of ``rows``, or one per row); writes the new block-table entries."""
        rows = list(range(self.max_seqs)) if rows is None else list(rows)
        extra = [int(tokens)] * len(rows) if isinstance(tokens, int) else [int(t) for t in tokens]
        if len(extra) != len(rows):
            raise ValueError("one token count per row")
        changed = []
        for b, n in zip(rows, extra):
            need = -(-(self._lens[b] + n) // self.page_size)
            if need > self.max_pages:
                raise ValueError(f"row {b}: {self._lens[b] + n} tokens exceed {self.max_pages} pages")
            while len(self._pages[b]) < need:
                if not self._free:
                    raise RuntimeError("paged KV cache is out of pages")
                self._pages[b].append(self._free.pop())
            if need:
                changed.append(b)
        if changed:
            tab = torch.full((len(changed), self.max_pages), -1, dtype=torch.int32)
            for i, b in enumerate(changed):
                tab[i, :len(self._pages[b])] = torch.tensor(self._pages[b], dtype=torch.int32)
            idx = torch.tensor(changed, dtype=torch.long, device=self.device)
            self.block_tables.index_copy_(0, idx, tab.to(self.device))

    def release(self, rows: Sequence[int]):
        """Returns the rows' pages to the free list and sets their lengths to 0."""
        rows = list(rows)
        for b in rows:
            self._free.extend(reversed(self._pages[b]))
            self._pages[b] = []
            self._lens[b] = 0
        if rows:
            idx = torch.tensor(rows, dtype=torch.long, device=self.device)
            self.context_lens.index_fill_(0, idx, 0)
            self.block_tables.index_fill_(0, idx, -1)

    # -- device steps --------------------------------------------------------------------
    def advance(self, n_new: Union[int, torch.Tensor], batch: int, host_counts: Optional[Sequence[int]] = None):
        """context_lens[:batch] += n_new (an int, or a (batch,) int32 device tensor whose
        values ``host_counts`` repeats for the host copy). One launch, no host read."""
        if isinstance(n_new, torch.Tensor):
            if n_new.dtype != torch.int32 or n_new.shape != (batch,) or not n_new.is_contiguous():
                raise ValueError("n_new must be a contiguous (batch,) int32 tensor")
            nat.require_device(n_new, self.context_lens)
            counts = list(host_counts) if host_counts is not None else None
            T, nptr = 0, nat.ptr(n_new)
        else:
            counts, T, nptr = [int(n_new)] * batch, int(n_new), None
        if counts is not None:
            for b in range(batch):
                self._lens[b] += counts[b]
        with torch.cuda.device(self.device):
            rc = nat.lib().sa_paged_advance(nat.ptr(self.context_lens), nptr, int(batch), T,
                                            nat.stream(self.device))
        nat.check(rc)

    def write(self, layer: int, k_new: torch.Tensor, v_new: torch.Tensor, token_codes: Optional[torch.Tensor] = None,
              n_new: Optional[torch.Tensor] = None):
        """Writes k_new / v_new (B, H_kv, T, D) as the last tokens of rows 0 .. B-1 (lengths
        already advanced), and the codes (B, H, T) int32 of tokens that open a page."""
        if k_new.dim() != 4 or v_new.shape != k_new.shape:
            raise ValueError("k_new / v_new must be (B, H_kv, T, D) of one shape")
        B, Hkv, T, D = k_new.shape
        if Hkv != self.kv_heads or D != self.head_dim or B > self.max_seqs:
            raise ValueError("k_new does not fit the cache")
        if k_new.dtype != self.k.dtype or v_new.dtype != self.k.dtype:
            raise ValueError("k_new / v_new must have the cache dtype")
        if token_codes is not None and (token_codes.shape != (B, self.heads, T) or token_codes.dtype != torch.int32):
            raise ValueError("token_codes must be (B, H, T) int32")
        if n_new is not None and (n_new.dtype != torch.int32 or n_new.shape != (B,) or not n_new.is_contiguous()):
            raise ValueError("n_new must be a contiguous (B,) int32 tensor")
        dev = nat.require_device(k_new, v_new, self.k)
        kc, vc, sc = self.k[layer], self.v[layer], self.seq_codes[layer]
        with torch.cuda.device(dev):
            rc = nat.lib().sa_paged_kv_write(
                nat.ptr(k_new), nat.ptr(v_new), nat.strides(k_new), nat.strides(v_new),
                nat.ptr(token_codes), None if token_codes is None else nat.strides(token_codes),
                nat.ptr(n_new), B, Hkv, T, D, self.heads, nat.ptr(kc), nat.ptr(vc), nat.strides(kc),
                nat.strides(vc), nat.ptr(self.block_tables), nat.strides(self.block_tables),
                nat.ptr(self.context_lens), self.max_pages, self.num_pages, self.page_size,
                nat.ptr(sc) if token_codes is not None else None, sc.element_size(), nat.strides(sc),
                nat.dtype_code(k_new.dtype, _KV_DTYPES), nat.ptr(self.status), nat.stream(dev))
        nat.check(rc)

    def decode(self, layer: int, q: torch.Tensor, q_codes: torch.Tensor, req_depth: int, *,
               local_blocks: int = 0, sink_block: bool = False) -> torch.Tensor:
        """Sparse paged decode of q (B, H, D) over rows 0 .. B-1 of layer ``layer``:
        a page is read iff its code matches q_codes (B, H) int32 on the first
        ``req_depth`` levels, or it is the sink page / one of the last ``local_blocks``."""
        B = q.shape[0]
        if self._ws is None:
            # split-KV scratch for any batch up to max_seqs, allocated once
            from .kernel_decode import decode_workspace_bytes
            need = max(decode_workspace_bytes(b, self.heads, self.head_dim, self.max_pages, self.kv_heads)
                       for b in range(1, self.max_seqs + 1))
            self._ws = torch.empty(max(need, 1), dtype=torch.uint8, device=self.device)
        return ultrametric_decode_seq_codes(q, self.k[layer], self.v[layer], self.block_tables[:B],
                                            self.context_lens[:B], self.seq_codes[layer, :B], q_codes,
                                            self.tree_depth, self.bits_per_level, req_depth,
                                            local_blocks=local_blocks, sink_block=sink_block, workspace=self._ws)

    def check_status(self):
        """Raises if a write met a page slot outside the reserved pages (one device read)."""
        if int(self.status.item()):
            self.status.zero_()
            raise RuntimeError("paged KV write outside the reserved pages (call reserve() first)")
