"""The HIP path against the committed golden fixtures (tests/golden/*.npz):
block lists and ternary packing bit-exact; prefill fp32 <= 1e-5 (generic
kernel) and bf16 <= 2e-2 (MFMA kernel, GQA 4/2, N not a multiple of 32);
decode bf16 <= 2e-2 (GQA 8/2, ragged and zero context lengths) through the
level-wise router, packed page codes and sequence codes; the bf16 backward
(GQA 4/2) <= 2e-2 of the gradient scale; the ternary prefill <= 5e-3 of the
output scale."""

import os

import numpy as np
import pytest
import torch

from ultrametric import BlockLists, block_list_attention, block_lists_from_mask, build_block_lists
from ultrametric import (pack_routing_codes, sequence_page_codes, ternary_quantize_pack,
                         ternary_ultrametric_attention, ultrametric_decode, ultrametric_decode_packed,
                         ultrametric_decode_seq_codes)

pytestmark = pytest.mark.gpu
DEV = "cuda"
GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bf16_tensor(bits):
    return torch.from_numpy(bits.astype(np.int16)).view(torch.bfloat16).to(DEV)


BL_CASES = {
    "tree_causal_sink": dict(is_causal=True, sink_block=True, arity=4),
    "tree_local_sync": dict(local_blocks=1),
    "random_depth_per_head": dict(is_causal=True, arity=2),
    "wide_ids_elementwise": dict(sink_block=True, local_blocks=2),
}


@pytest.mark.parametrize("name", sorted(BL_CASES))
def test_block_lists_golden(name):
    g = load("block_lists.npz")
    depth = g[f"{name}__depth"]
    depth = int(depth) if depth.ndim == 0 else [int(x) for x in depth]
    bl = build_block_lists(torch.from_numpy(g[f"{name}__router"]).to(DEV), depth, **BL_CASES[name])
    assert np.array_equal(bl.lists.cpu().numpy(), g[f"{name}__lists"])
    assert np.array_equal(bl.counts.cpu().numpy(), g[f"{name}__counts"])


def test_prefill_golden_fp32():
    g = load("prefill.npz")
    q, k, v = (torch.from_numpy(g[f"f32__{t}"]).to(DEV) for t in "qkv")
    bl = block_lists_from_mask(torch.from_numpy(g["f32__mask"]).to(DEV))
    out, lse = block_list_attention(q, k, v, bl, route_block=int(g["f32__route_block"]), is_causal=True,
                                    return_lse=True)
    assert np.abs(out.cpu().numpy() - g["f32__out"]).max() <= 1e-5
    assert np.abs(lse.cpu().numpy() - g["f32__lse"]).max() <= 1e-5


def test_prefill_golden_bf16_gqa():
    g = load("prefill.npz")
    q, k, v = (bf16_tensor(g[f"bf16__{t}_bits"]) for t in "qkv")
    lists = torch.from_numpy(g["bf16__lists"]).to(DEV)
    bl = BlockLists(lists, torch.from_numpy(g["bf16__counts"]).to(DEV), lists.shape[-1])
    out, lse = block_list_attention(q, k, v, bl, route_block=int(g["bf16__route_block"]), is_causal=True,
                                    return_lse=True)
    assert np.abs(out.float().cpu().numpy() - g["bf16__out"]).max() <= 2e-2
    assert np.abs(lse.cpu().numpy() - g["bf16__lse"]).max() <= 2e-2


@pytest.mark.parametrize("name,kw", [("r2_sink_local", dict(req_depth=2, local_blocks=2, sink_block=True)),
                                     ("r3", dict(req_depth=3)), ("dense", dict(req_depth=0))])
def test_decode_golden_bf16(name, kw):
    g = load("decode.npz")
    q, k, v = (bf16_tensor(g[f"{t}_bits"]) for t in "qkv")
    args = [torch.from_numpy(g[n]).to(DEV) for n in ("block_tables", "context_lens", "router", "q_router")]
    out = ultrametric_decode(q, k, v, *args, **kw)
    assert np.abs(out.float().cpu().numpy() - g[f"{name}__out"]).max() <= 2e-2
    assert torch.all(out[0] == 0)


@pytest.mark.parametrize("name,kw", [("r2_sink_local", dict(req_depth=2, local_blocks=2, sink_block=True)),
                                     ("r3", dict(req_depth=3)), ("dense", dict(req_depth=0))])
def test_decode_golden_codes(name, kw):
    # routing ids in {0, 1}: one bit per level
    g = load("decode.npz")
    q, k, v = (bf16_tensor(g[f"{t}_bits"]) for t in "qkv")
    bt, ctx, router, q_router = (torch.from_numpy(g[n]).to(DEV)
                                 for n in ("block_tables", "context_lens", "router", "q_router"))
    TD = router.shape[-1]
    pc, qc = pack_routing_codes(router, 1), pack_routing_codes(q_router, 1)
    out = ultrametric_decode_packed(q, k, v, bt, ctx, pc, qc, TD, 1, **kw)
    assert np.abs(out.float().cpu().numpy() - g[f"{name}__out"]).max() <= 2e-2
    sc = sequence_page_codes(pc, bt, bits=TD)
    sout = ultrametric_decode_seq_codes(q, k, v, bt, ctx, sc, qc, TD, 1, **kw)
    assert torch.equal(sout, out)


def test_backward_golden_bf16_gqa():
    g = load("backward.npz")
    q, k, v = (bf16_tensor(g[f"{t}_bits"]).requires_grad_(True) for t in "qkv")
    do = bf16_tensor(g["do_bits"])
    lists = torch.from_numpy(g["lists"]).to(DEV)
    bl = BlockLists(lists, torch.from_numpy(g["counts"]).to(DEV), lists.shape[-1])
    block_list_attention(q, k, v, bl, route_block=int(g["route_block"]), is_causal=True).backward(do)
    for t, name in ((q, "dq"), (k, "dk"), (v, "dv")):
        ref = g[name]
        assert np.abs(t.grad.float().cpu().numpy() - ref).max() <= 2e-2 * max(1.0, np.abs(ref).max()), name


def test_ternary_golden():
    g = load("ternary.npz")
    packed, scale = ternary_quantize_pack(torch.from_numpy(g["x"]).to(DEV))
    assert np.array_equal(packed.cpu().numpy(), g["packed"])
    assert np.allclose(scale.cpu().numpy(), g["scale"], rtol=1e-6)
    args = [torch.from_numpy(g[n]).to(DEV) for n in ("q", "k_packed", "v_packed", "k_scale", "v_scale", "router")]
    out = ternary_ultrametric_attention(*args, local_window=128, req_depth=2, shift_size=77)
    ref = g["out"]
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 5e-3 * max(1.0, np.abs(ref).max())
