"""CPU checks of the package functions that keep the reference's torch
formulations for callers: ``routing_to_block_indices``
(src/ultrametric/kernel.py:152-191), ``block_mask_reference``,
``token_mask_from_blocks``, ``masked_reference_attention``
(src/ultrametric/block_list.py:334-378) and ``_ultrametric_decode_reference``
(src/ultrametric/kernel_decode.py:129-185).

``routing_to_block_indices`` is pinned by a brute-force loop of its rule (each
block takes its first token's argmax branch per level; a sequence shorter than
num_blocks * block_size is padded with branch 0), with and without padding.
The other four are compared with the float64 / exact-integer oracle
(oracle/blocks.py, oracle/attention.py, oracle/decode.py) on seeded inputs.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import blocks as ob
from oracle import decode as od
from ultrametric import routing_to_block_indices
from ultrametric.block_list import block_mask_reference, masked_reference_attention, token_mask_from_blocks
from ultrametric.kernel_decode import _ultrametric_decode_reference


def _onehot_assignments(B, H, S, L, P, seed):
    g = torch.Generator().manual_seed(seed)
    logits = torch.randn(B, H, S, L, P, generator=g)
    return torch.nn.functional.one_hot(logits.argmax(-1), P).to(torch.float32)


def _first_token_loop(a, seq_len, block_size):
    B, H, S, L, P = a.shape
    nb = math.ceil(seq_len / block_size)
    out = np.zeros((B, H, nb, L), dtype=np.int32)
    for b in range(B):
        for h in range(H):
            for blk in range(nb):
                t = blk * block_size
                for l in range(L):
                    out[b, h, blk, l] = int(a[b, h, t, l].argmax()) if t < S else 0
    return out


@pytest.mark.parametrize("S,block_size", [(256, 64), (200, 64), (128, 128), (1, 16), (97, 32)])
def test_routing_to_block_indices_first_token_rule(S, block_size):
    a = _onehot_assignments(2, 3, S, 4, 4, seed=S + block_size)
    got = routing_to_block_indices(a, S, block_size)
    assert got.dtype == torch.int32
    assert got.shape == (2, 3, math.ceil(S / block_size), 4)
    assert np.array_equal(got.numpy(), _first_token_loop(a, S, block_size))


def test_routing_to_block_indices_pads_with_branch_zero():
    # seq_len beyond the tokens given: the extra blocks read padded tokens (branch 0)
    a = _onehot_assignments(1, 2, 64, 3, 4, seed=1)
    got = routing_to_block_indices(a, 64, 16)
    assert np.array_equal(got.numpy(), _first_token_loop(a, 64, 16))
    a_short = a[:, :, :40]
    got = routing_to_block_indices(a_short, 64, 16).numpy()
    assert np.array_equal(got[:, :, :3], _first_token_loop(a, 64, 16)[:, :, :3])
    assert (got[:, :, 3] == 0).all()


@pytest.mark.parametrize("depth", [0, 1, 2, [0, 3, 1]])
@pytest.mark.parametrize("causal,sink,local", [(False, False, 0), (True, True, 0), (True, False, 2),
                                               (False, True, 1)])
def test_block_mask_reference_matches_oracle(depth, causal, sink, local):
    rng = np.random.default_rng(7)
    router = rng.integers(0, 3, size=(2, 3, 10, 3)).astype(np.int64)
    got = block_mask_reference(torch.from_numpy(router), depth, is_causal=causal, sink_block=sink,
                               local_blocks=local)
    ref = ob.block_mask_reference(router, depth, is_causal=causal, sink_block=sink, local_blocks=local)
    assert np.array_equal(got.numpy(), ref)


@pytest.mark.parametrize("N,rb,causal", [(100, 16, True), (128, 32, False), (33, 8, True)])
def test_token_mask_from_blocks_matches_oracle(N, rb, causal):
    rng = np.random.default_rng(N)
    nb = -(-N // rb)
    bm = rng.random((1, 2, nb, nb)) < 0.4
    got = token_mask_from_blocks(torch.from_numpy(bm), rb, N, is_causal=causal)
    assert np.array_equal(got.numpy(), oa.token_mask_from_blocks(bm, rb, N, is_causal=causal))


@pytest.mark.parametrize("scale", [None, 0.3])
def test_masked_reference_attention_matches_oracle(scale):
    rng = np.random.default_rng(3)
    Z, H, N, D, rb = 1, 2, 48, 16, 16
    q, k, v = (rng.standard_normal((Z, H, N, D)).astype(np.float32) for _ in range(3))
    bm = ob.apply_structural_masks(rng.random((Z, H, 3, 3)) < 0.5, is_causal=True, sink_block=True,
                                   local_blocks=0)
    tm = oa.token_mask_from_blocks(bm, rb, N, is_causal=True)
    got = masked_reference_attention(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                     torch.from_numpy(tm), sm_scale=scale)
    ref, _ = oa.masked_attention(q, k, v, tm, sm_scale=scale)
    assert got.dtype == torch.float32
    assert np.abs(got.numpy() - ref).max() <= 1e-5   # fp32 against float64


@pytest.mark.parametrize("req_depth,local,sink,group", [(0, 0, False, 1), (2, 1, True, 2), (3, 2, False, 4),
                                                        (1, 0, True, 1)])
def test_decode_reference_matches_oracle(req_depth, local, sink, group):
    rng = np.random.default_rng(11 + req_depth)
    B, Hkv, D, page, pages, TD = 3, 2, 8, 4, 12, 3
    H = Hkv * group
    lens = (13, 0, 5)
    q = rng.standard_normal((B, H, D)).astype(np.float32)
    kc = rng.standard_normal((pages, Hkv, page, D)).astype(np.float32)
    vc = rng.standard_normal((pages, Hkv, page, D)).astype(np.float32)
    tables = np.stack([rng.permutation(pages)[:4] for _ in range(B)]).astype(np.int32)
    ctx = np.array(lens, dtype=np.int32)
    router = rng.integers(0, 2, size=(pages, H, TD)).astype(np.int32)
    qr = rng.integers(0, 2, size=(B, H, TD)).astype(np.int32)
    t = torch.from_numpy
    got = _ultrametric_decode_reference(t(q), t(kc), t(vc), t(tables), t(ctx), t(router), t(qr), req_depth,
                                        local_blocks=local, sink_block=sink)
    ref = od.decode_reference(q, kc, vc, tables, ctx, router, qr, req_depth, local_blocks=local,
                              sink_block=sink)
    assert np.abs(got.numpy() - ref).max() <= 1e-5
    assert (got[1] == 0).all()   # ctx = 0 -> zeros
