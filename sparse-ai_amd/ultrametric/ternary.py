"""Ternary (2-bit) packed K / V on MI355X (src/llama_surgery/surgery.py:15-76
and src/llama_surgery/kernel.py:147-249, :348-420).

``ternary_quantize_pack`` (TernaryQuantize + pack_ternary in one HIP kernel)
turns K or V rows into 16 two-bit codes per int32 word plus one fp32 scale per
row; ``ternary_ultrametric_attention`` keeps the reference launcher's
signature and runs the causal block-sparse prefill over the packed rows: the
block choice (routing match on the first ``req_depth`` levels, sink, local
window) becomes block lists (route block 128), and the HIP kernel unpacks
64 bytes per key row instead of reading 512 (bf16, D = 128).
"""

from __future__ import annotations

import math

import torch

from . import _native as nat
from .block_list import build_block_lists

__all__ = ["ternary_quantize_pack", "pack_ternary", "unpack_ternary", "ternary_block_lists",
           "ternary_ultrametric_attention", "ternary_ultrametric_attention_triton"]


def _pack(x: torch.Tensor, mode: int):
    if x.shape[-1] % 16 != 0:
        raise ValueError("Last dimension must be multiple of 16 for packing")
    dev = nat.require_device(x)
    D = x.shape[-1]
    lead = tuple(x.shape[:-1])
    x2 = x.reshape(-1, D)
    if x2.dtype not in (torch.float32, torch.bfloat16, torch.float16):
        x2 = x2.float()
    rows = x2.shape[0]
    packed = torch.empty((rows, D // 16), dtype=torch.int32, device=dev)
    scale = torch.empty((rows,), dtype=torch.float32, device=dev)
    with torch.cuda.device(dev):
        rc = nat.lib().sa_ternary_pack(nat.ptr(x2), nat.DTYPE_CODES[x2.dtype], nat.strides(x2), rows, D, mode,
                                       nat.ptr(packed), nat.ptr(scale), nat.stream(dev))
    nat.check(rc)
    return packed.reshape(*lead, D // 16), scale.reshape(lead)


def ternary_quantize_pack(x: torch.Tensor):
    """TernaryQuantize (surgery.py:15-28) + pack_ternary (:35-55): returns
    (packed (..., D / 16) int32, scale (...) fp32) with x ~ unpack(packed) * scale."""
    return _pack(x, 0)


def pack_ternary(x_ternary: torch.Tensor) -> torch.Tensor:
    """surgery.py:35-55: values in {-1, 0, 1} -> (..., D / 16) int32."""
    return _pack(x_ternary, 1)[0]


def unpack_ternary(packed: torch.Tensor, original_shape: tuple) -> torch.Tensor:
    """surgery.py:57-76: (..., D / 16) int32 -> float tensor of original_shape in {-1, 0, 1}."""
    shifts = torch.arange(0, 32, 2, device=packed.device, dtype=torch.int32)
    codes = (packed.unsqueeze(-1) >> shifts) & 3
    vals = codes.reshape(original_shape).float()
    return torch.where(vals == 2, torch.full_like(vals, -1.0), torch.where(vals == 1, vals, torch.zeros_like(vals)))


# The reference kernel compares routing ids level by level (kernel.py:197-201),
# whatever `p` is. A sync-free build with this base never takes the mixed-radix
# code path for TD >= 2 (TD * 31 >= 62) and, for TD = 1, codes each id as
# itself: level-wise equality, with no aliasing of ids >= p and no host read.
_LEVELWISE_ARITY = 1 << 31


def ternary_block_lists(router: torch.Tensor, req_depth: int, local_window: int = 128):
    """The visited (query block, key block) pairs of the ternary prefill as
    sync-free BlockLists (route block 128): the first req_depth routing levels
    equal, or the sink block, or within ceil(local_window / 128) blocks, causal
    (kernel.py:193-208)."""
    return build_block_lists(router, req_depth, is_causal=True, sink_block=True,
                             local_blocks=math.ceil(local_window / 128), arity=_LEVELWISE_ARITY)


def ternary_ultrametric_attention(
    q: torch.Tensor,
    k_packed: torch.Tensor,
    v_packed: torch.Tensor,
    k_scale: torch.Tensor,
    v_scale: torch.Tensor,
    router_indices: torch.Tensor,
    local_window: int = 128,
    req_depth: int = 2,
    shift_size: int = 0,
    p: int = 2,
) -> torch.Tensor:
    """Causal block-sparse attention over ternary packed K / V (kernel.py:348-420).

    q: (Z, H, N, D) fp16; k_packed / v_packed: (Z, H_kv, N, D / 16) int32;
    k_scale / v_scale: (Z, H_kv, N); router_indices: (Z, H, NB', TD) branch ids
    (rows past NB' count as zeros, as the reference pads them). Blocks match
    when their first req_depth ids are equal, level by level, as in the
    reference; ``p`` is accepted for its signature and does not enter the
    match. Returns (Z, H, N, D) fp16.
    """
    if q.dtype != torch.float16:
        raise ValueError(f"ternary attention requires float16 Q, got {q.dtype}")
    if k_packed.dtype != torch.int32 or v_packed.dtype != torch.int32:
        raise ValueError("k_packed / v_packed must be int32")
    Z, H, N, D = q.shape
    if k_packed.shape[-1] * 16 != D or v_packed.shape != k_packed.shape or k_packed.shape[2] != N:
        raise ValueError(f"packed K / V must be (Z, H_kv, N, D/16); got {tuple(k_packed.shape)}, {tuple(v_packed.shape)}")
    Hkv = k_packed.shape[1]
    if H % Hkv != 0:
        raise ValueError("query heads must be a multiple of the packed K / V heads")
    dev = nat.require_device(q, k_packed, v_packed, k_scale, v_scale, router_indices)
    NB = math.ceil(N / 128)
    r = router_indices.to(torch.int32)
    TD = r.shape[-1]
    if r.shape[2] < NB:
        r = torch.cat([r, torch.zeros((Z, H, NB - r.shape[2], TD), dtype=torch.int32, device=dev)], dim=2)
    r = r[:, :, :NB]
    depth = min(max(int(req_depth), 0), TD)
    bl = ternary_block_lists(r, depth, local_window)
    ks = k_scale if k_scale.dtype in (torch.float32, torch.bfloat16, torch.float16) else k_scale.float()
    vs = v_scale if v_scale.dtype == ks.dtype else v_scale.to(ks.dtype)
    qc = q if q.stride(-1) == 1 else q.contiguous()
    kp = k_packed if k_packed.stride(-1) == 1 else k_packed.contiguous()
    vp = v_packed if v_packed.stride(-1) == 1 else v_packed.contiguous()
    out = torch.empty((Z, H, N, D), dtype=torch.float16, device=dev)
    with torch.cuda.device(dev):
        rc = nat.lib().sa_ternary_prefill_fwd(
            nat.ptr(qc), nat.ptr(kp), nat.ptr(vp), nat.ptr(ks), nat.ptr(vs), nat.DTYPE_CODES[ks.dtype],
            nat.ptr(bl.lists), nat.ptr(bl.counts), bl.max_count, nat.ptr(out), Z, H, Hkv, N, D, int(shift_size),
            nat.strides(qc), nat.strides(kp), nat.strides(vp), nat.strides(ks), nat.strides(vs), nat.strides(out),
            nat.stream(dev))
    nat.check(rc)
    return out


# the reference's name for the same launcher (kernel.py:348)
ternary_ultrametric_attention_triton = ternary_ultrametric_attention
