"""ultrametric — MI355X-native block-sparse attention hot path of sparse-ai.

Drop-in for the kernel API of the reference package ``src/ultrametric``
(__init__.py:24-36 and kernel_decode.py): the same function names and
signatures, backed by hand-written HIP kernels for gfx950 in libsparseattn.so.
``surgery`` adds the model-side caller (the route-block vote and causal
prefill of src/llama_surgery/surgery.py:521-601), ``paged_cache`` the serving
side of the decode (a paged K / V cache with per-sequence page routing codes
and its write / decode step), ``llama_model`` a Llama-3.1-8B-shaped decoder
that drives both. The reference's training
model, topology routers, layers and legacy kernels are outside this
package's scope.
"""

from .block_list import (
    HAS_HIP,
    HAS_TRITON,
    BlockLists,
    block_list_attention,
    block_lists_from_mask,
    build_block_lists,
    build_transposed_block_lists,
    routed_block_attention,
)
from .kernel import block_sparse_attention, routing_to_block_indices
from .kernel_decode import (pack_routing_codes, sequence_page_codes, ultrametric_decode,
                            ultrametric_decode_packed, ultrametric_decode_seq_codes)
from .paged_cache import PagedKVCache, token_routing_codes
from .surgery import RouteCache, block_list_prefill, route_block_vote
from .ternary import pack_ternary, ternary_quantize_pack, ternary_ultrametric_attention

__all__ = [
    "HAS_TRITON",
    "HAS_HIP",
    "BlockLists",
    "build_block_lists",
    "block_lists_from_mask",
    "build_transposed_block_lists",
    "block_list_attention",
    "routed_block_attention",
    "block_sparse_attention",
    "routing_to_block_indices",
    "ultrametric_decode",
    "pack_routing_codes",
    "ultrametric_decode_packed",
    "sequence_page_codes",
    "ultrametric_decode_seq_codes",
    "route_block_vote",
    "block_list_prefill",
    "RouteCache",
    "PagedKVCache",
    "token_routing_codes",
    "ternary_quantize_pack",
    "pack_ternary",
    "ternary_ultrametric_attention",
]
