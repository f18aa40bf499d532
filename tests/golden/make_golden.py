"""Writes the golden fixtures of tests/golden/*.npz from this repository's CPU
oracle (oracle/), on seeded inputs. Test infrastructure only.

The reference (sneed-and-feed/sparse-ai) ships no golden vectors for the
block-sparse attention path: its tests regenerate seeded inputs and compare
the Triton kernels with its own masked-dense PyTorch oracles
(tests/test_block_list.py:96-128,200-253,358-380; tests/test_llama_surgery.py:355-398).
These fixtures freeze this build's oracle outputs on small cases of the same
kinds, so that (a) the oracle is regression-pinned (tests/test_golden_cpu.py
recomputes them) and (b) the HIP path is checked against fixed vectors
(tests/test_golden_gpu.py). Inputs are stored exactly (bf16 values as their
uint16 bit patterns); expectations are the float64 oracle results stored as
float32.

Usage: python tests/golden/make_golden.py   (rewrites the .npz files)
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

from oracle import attention as oa  # noqa: E402
from oracle import blocks as ob  # noqa: E402
from oracle import decode as od  # noqa: E402
from oracle import ternary as ot  # noqa: E402


def bf16_round(x):
    """float32 array -> (bf16 bit patterns uint16, the float32 values they encode), RNE."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    return r, (r.astype(np.uint32) << 16).view(np.float32)


def tree_router(rng, Z, H, NB, p, depth):
    """Per head, a random leaf permutation; ids = base-p digits of the leaf (root first)."""
    leaves = np.stack([np.stack([rng.permutation(NB) for _ in range(H)]) for _ in range(Z)])
    return np.stack([(leaves // p ** (depth - 1 - d)) % p for d in range(depth)], -1).astype(np.int32)


def make_block_lists(path):
    rng = np.random.default_rng(1001)
    out = {}
    cases = [
        # name, router shape (Z,H,NB,TD), ids in [0,p), req_depth, kwargs
        ("tree_causal_sink", (1, 2, 16, 2), 4, 1, dict(is_causal=True, sink_block=True, arity=4)),
        ("tree_local_sync", (1, 2, 16, 2), 4, 2, dict(local_blocks=1)),
        ("random_depth_per_head", (2, 3, 12, 3), 2, [0, 2, 3], dict(is_causal=True, arity=2)),
        ("wide_ids_elementwise", (1, 2, 8, 8), 300, 5, dict(sink_block=True, local_blocks=2)),
    ]
    for name, shape, p, depth, kw in cases:
        if name.startswith("tree"):
            router = tree_router(rng, shape[0], shape[1], shape[2], p, shape[3])
        else:
            router = rng.integers(0, p, size=shape, dtype=np.int32)
        bl = ob.build_block_lists(router, depth, **kw)
        out[f"{name}__router"] = router
        out[f"{name}__depth"] = np.asarray(depth, dtype=np.int64)
        out[f"{name}__lists"] = bl.lists.astype(np.int32)
        out[f"{name}__counts"] = bl.counts.astype(np.int32)
    np.savez_compressed(path, **out)


def make_prefill(path):
    rng = np.random.default_rng(2002)
    out = {}
    # fp32, generic kernel shapes (config-1 style: Bernoulli lower-triangle + diag + sink, causal)
    Z, H, N, D, RB = 1, 2, 200, 32, 32
    NB = -(-N // RB)
    q, k, v = (rng.standard_normal((Z, H, N, D)).astype(np.float32) for _ in range(3))
    m = rng.random((Z, H, NB, NB)) < 0.3
    m &= np.tril(np.ones((NB, NB), dtype=bool))
    m[..., np.arange(NB), np.arange(NB)] = True
    m[..., 0] = True
    o, lse = oa.block_sparse_attention_ref(q, k, v, m, RB, is_causal=True)
    out.update({"f32__q": q, "f32__k": k, "f32__v": v, "f32__mask": m, "f32__out": o.astype(np.float32),
                "f32__lse": lse.astype(np.float32),
                "f32__route_block": np.int64(RB)})
    # bf16, MFMA kernel shapes, GQA 4/2, binary routing ids, causal, N not a multiple of 32
    Z, H, Hkv, N, D, RB = 1, 4, 2, 300, 64, 64
    NB = -(-N // RB)
    qb, qf = bf16_round(rng.standard_normal((Z, H, N, D)).astype(np.float32))
    kb, kf = bf16_round(rng.standard_normal((Z, Hkv, N, D)).astype(np.float32))
    vb, vf = bf16_round(rng.standard_normal((Z, Hkv, N, D)).astype(np.float32))
    router = rng.integers(0, 2, size=(Z, H, NB, 3), dtype=np.int32)
    bl = ob.build_block_lists(router, 2, is_causal=True, sink_block=True, arity=2)
    mask = ob.lists_to_mask(bl.lists, bl.counts)
    o, lse = oa.block_sparse_attention_ref(qf, kf, vf, mask, RB, is_causal=True)
    out.update({"bf16__q_bits": qb, "bf16__k_bits": kb, "bf16__v_bits": vb, "bf16__lists": bl.lists.astype(np.int32),
                "bf16__counts": bl.counts.astype(np.int32), "bf16__out": o.astype(np.float32),
                "bf16__lse": lse.astype(np.float32),
                "bf16__route_block": np.int64(RB)})
    np.savez_compressed(path, **out)


def make_decode(path):
    rng = np.random.default_rng(3003)
    B, H, Hkv, D, page, pages, TD = 4, 8, 2, 64, 8, 40, 3
    lens = np.array([0, 5, 70, 150], dtype=np.int32)
    mp = -(-int(lens.max()) // page)
    qb, qf = bf16_round(rng.standard_normal((B, H, D)).astype(np.float32))
    kb, kf = bf16_round(rng.standard_normal((pages, Hkv, page, D)).astype(np.float32))
    vb, vf = bf16_round(rng.standard_normal((pages, Hkv, page, D)).astype(np.float32))
    bt = np.stack([rng.permutation(pages)[:mp] for _ in range(B)]).astype(np.int32)
    router = rng.integers(0, 2, size=(pages, H, TD), dtype=np.int32)
    q_router = rng.integers(0, 2, size=(B, H, TD), dtype=np.int32)
    out = {"q_bits": qb, "k_bits": kb, "v_bits": vb, "block_tables": bt, "context_lens": lens,
           "router": router, "q_router": q_router}
    for name, kw in (("r2_sink_local", dict(req_depth=2, local_blocks=2, sink_block=True)),
                     ("r3", dict(req_depth=3)), ("dense", dict(req_depth=0))):
        out[f"{name}__out"] = od.decode_reference(qf, kf, vf, bt, lens, router, q_router, **kw).astype(np.float32)
    np.savez_compressed(path, **out)


def make_backward(path):
    # bf16 inputs on the MFMA backward's shapes: GQA 4/2, route block 64, causal with sink
    rng = np.random.default_rng(4004)
    Z, H, Hkv, N, D, RB = 1, 4, 2, 256, 64, 64
    NB = N // RB
    qb, qf = bf16_round(rng.standard_normal((Z, H, N, D)).astype(np.float32))
    kb, kf = bf16_round(rng.standard_normal((Z, Hkv, N, D)).astype(np.float32))
    vb, vf = bf16_round(rng.standard_normal((Z, Hkv, N, D)).astype(np.float32))
    gb, gf = bf16_round(rng.standard_normal((Z, H, N, D)).astype(np.float32))
    router = rng.integers(0, 2, size=(Z, H, NB, 2), dtype=np.int32)
    bl = ob.build_block_lists(router, 1, is_causal=True, sink_block=True, arity=2)
    mask = ob.lists_to_mask(bl.lists, bl.counts)
    dq, dk, dv, _ = oa.block_sparse_attention_grad_ref(qf, kf, vf, mask, RB, gf, is_causal=True)
    np.savez_compressed(path, q_bits=qb, k_bits=kb, v_bits=vb, do_bits=gb, lists=bl.lists.astype(np.int32),
                        counts=bl.counts.astype(np.int32), dq=dq.astype(np.float32), dk=dk.astype(np.float32),
                        dv=dv.astype(np.float32), route_block=np.int64(RB))


def make_ternary(path):
    rng = np.random.default_rng(5005)
    # quantize + pack of rows whose entries stay clear of the +-gamma/2 thresholds
    x = rng.standard_normal((6, 64)).astype(np.float32)
    gamma = np.abs(x).mean(-1, keepdims=True)
    x = np.where(np.abs(np.abs(x) - 0.5 * gamma) < 1e-3 * gamma, 0.0, x).astype(np.float32)
    t, g = ot.ternary_quantize(x)
    out = {"x": x, "packed": ot.pack_ternary(t), "scale": np.asarray(g, dtype=np.float32).reshape(-1)}
    # prefill over packed K / V: fp16 Q, ternary codes, fp32 row scales, routing + sink + local + shift
    Z, H, N, D = 1, 2, 384, 64
    q = rng.standard_normal((Z, H, N, D)).astype(np.float16)
    kt = rng.integers(-1, 2, size=(Z, H, N, D)).astype(np.float32)
    vt = rng.integers(-1, 2, size=(Z, H, N, D)).astype(np.float32)
    ks = (rng.random((Z, H, N)) * 0.6 + 0.1).astype(np.float32)
    vs = (rng.random((Z, H, N)) * 1.5 + 0.2).astype(np.float32)
    router = rng.integers(0, 2, size=(Z, H, N // 128, 3), dtype=np.int32)
    kp, vp = ot.pack_ternary(kt), ot.pack_ternary(vt)
    ref = ot.ternary_attention_ref(q.astype(np.float32), kp, vp, ks, vs, router, local_window=128, req_depth=2,
                                   shift_size=77)
    out.update({"q": q, "k_packed": kp, "v_packed": vp, "k_scale": ks, "v_scale": vs, "router": router,
                "out": ref.astype(np.float32)})
    np.savez_compressed(path, **out)


if __name__ == "__main__":
    make_block_lists(os.path.join(HERE, "block_lists.npz"))
    make_prefill(os.path.join(HERE, "prefill.npz"))
    make_decode(os.path.join(HERE, "decode.npz"))
    make_backward(os.path.join(HERE, "backward.npz"))
    make_ternary(os.path.join(HERE, "ternary.npz"))
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")
