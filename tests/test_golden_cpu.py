"""The CPU oracle against the committed golden fixtures (tests/golden/*.npz,
written by tests/golden/make_golden.py): block lists and ternary packing
bit-exact; attention, decode, backward gradients and the ternary prefill to
float32 storage precision. A change to the oracle that moves any of
these fails here."""

import os

import numpy as np
import pytest

from oracle import attention as oa
from oracle import blocks as ob
from oracle import decode as od
from oracle import ternary as ot

GOLD = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    return np.load(os.path.join(GOLD, name), allow_pickle=False)


def bits_to_f32(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


BL_CASES = {
    "tree_causal_sink": dict(is_causal=True, sink_block=True, arity=4),
    "tree_local_sync": dict(local_blocks=1),
    "random_depth_per_head": dict(is_causal=True, arity=2),
    "wide_ids_elementwise": dict(sink_block=True, local_blocks=2),
}


@pytest.mark.parametrize("name", sorted(BL_CASES))
def test_block_lists_fixture(name):
    g = load("block_lists.npz")
    depth = g[f"{name}__depth"]
    depth = int(depth) if depth.ndim == 0 else [int(x) for x in depth]
    bl = ob.build_block_lists(g[f"{name}__router"], depth, **BL_CASES[name])
    assert np.array_equal(bl.lists, g[f"{name}__lists"])
    assert np.array_equal(bl.counts, g[f"{name}__counts"])


def test_prefill_fixture_fp32():
    g = load("prefill.npz")
    o, lse = oa.block_sparse_attention_ref(g["f32__q"], g["f32__k"], g["f32__v"], g["f32__mask"],
                                           int(g["f32__route_block"]), is_causal=True)
    assert np.abs(o - g["f32__out"]).max() <= 1e-6
    assert np.abs(lse - g["f32__lse"]).max() <= 1e-5


def test_prefill_fixture_bf16_gqa():
    g = load("prefill.npz")
    q, k, v = (bits_to_f32(g[f"bf16__{t}_bits"]) for t in "qkv")
    mask = ob.lists_to_mask(g["bf16__lists"], g["bf16__counts"])
    o, lse = oa.block_sparse_attention_ref(q, k, v, mask, int(g["bf16__route_block"]), is_causal=True)
    assert np.abs(o - g["bf16__out"]).max() <= 1e-6
    assert np.abs(lse - g["bf16__lse"]).max() <= 1e-5


@pytest.mark.parametrize("name,kw", [("r2_sink_local", dict(req_depth=2, local_blocks=2, sink_block=True)),
                                     ("r3", dict(req_depth=3)), ("dense", dict(req_depth=0))])
def test_decode_fixture(name, kw):
    g = load("decode.npz")
    q, k, v = (bits_to_f32(g[f"{t}_bits"]) for t in "qkv")
    o = od.decode_reference(q, k, v, g["block_tables"], g["context_lens"], g["router"], g["q_router"], **kw)
    assert np.abs(o - g[f"{name}__out"]).max() <= 1e-6
    assert np.all(o[0] == 0)   # context length 0 -> zeros


def test_backward_fixture():
    g = load("backward.npz")
    q, k, v, do = (bits_to_f32(g[f"{t}_bits"]) for t in ("q", "k", "v", "do"))
    mask = ob.lists_to_mask(g["lists"], g["counts"])
    dq, dk, dv, _ = oa.block_sparse_attention_grad_ref(q, k, v, mask, int(g["route_block"]), do, is_causal=True)
    for got, name in ((dq, "dq"), (dk, "dk"), (dv, "dv")):
        assert np.abs(got - g[name]).max() <= 1e-5 * max(1.0, np.abs(g[name]).max()), name


def test_ternary_fixture():
    g = load("ternary.npz")
    t, gamma = ot.ternary_quantize(g["x"])
    assert np.array_equal(ot.pack_ternary(t), g["packed"])
    assert np.allclose(np.asarray(gamma).reshape(-1), g["scale"], rtol=1e-6)
    ref = ot.ternary_attention_ref(g["q"].astype(np.float32), g["k_packed"], g["v_packed"], g["k_scale"],
                                   g["v_scale"], g["router"], local_window=128, req_depth=2, shift_size=77)
    assert np.abs(ref - g["out"]).max() <= 1e-6
