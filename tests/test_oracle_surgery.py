"""Pins oracle/surgery.py (the route-block majority vote and allowed-key
statistics of src/llama_surgery/surgery.py:536-551,589-595) against
independent constructions: the reference test's own Python loop of bincount +
argmax per block and level (tests/test_surgery_block_list.py:42-55) on its
parameter grid, hand-made blocks with forced winners, and the row sums of the
token mask built from the same lists (tests/test_surgery_block_list.py:93-95)."""

import math

import numpy as np
import pytest

from oracle import attention as oa
from oracle import blocks as ob
from oracle import surgery as osg


def loop_route(assign, r, rb):
    """The reference test's construction (tests/test_surgery_block_list.py:42-55)."""
    B, H, S, _, p = assign.shape
    nb = math.ceil(S / rb)
    idx = assign[..., :r, :].argmax(-1)
    out = np.zeros((B, H, nb, r), dtype=np.int32)
    for b in range(B):
        for h in range(H):
            for i in range(nb):
                seg = idx[b, h, i * rb:(i + 1) * rb]
                for lvl in range(r):
                    cnt = np.bincount(seg[:, lvl], minlength=p)
                    out[b, h, i, lvl] = int(np.argmax(cnt))   # first max = lowest id
    return out


@pytest.mark.parametrize("S,rb,r,p,L", [(200, 32, 2, 2, 4), (256, 64, 3, 2, 4), (96, 32, 1, 2, 3),
                                        (333, 16, 4, 4, 4), (50, 128, 2, 3, 2)])
def test_majority_matches_loop(S, rb, r, p, L):
    rng = np.random.default_rng(S + rb)
    assign = rng.random((2, 3, S, L, p))
    assert np.array_equal(osg.majority_route(assign, r, rb), loop_route(assign, r, rb))


def test_forced_winners():
    p, rb = 3, 4
    a = np.zeros((1, 1, 10, 1, p))
    a[0, 0, 0:4, 0, 2] = 1.0                   # block 0 unanimous for branch 2
    a[0, 0, 4:6, 0, 1] = 1.0                   # block 1: two votes for 1,
    a[0, 0, 6:8, 0, 2] = 1.0                   #          two for 2 -> tie -> 1
    a[0, 0, 8:10, 0, :] = 0.5                  # tail block (2 tokens): all-equal scores -> argmax 0
    got = osg.majority_route(a, 1, rb)[0, 0, :, 0]
    assert got.tolist() == [2, 1, 0]
    # direct block routing: per-row argmax, first max on ties
    d = np.array([[[[[0.1, 0.9, 0.9]], [[0.5, 0.2, 0.1]]]]])
    assert osg.direct_route(d, 1)[0, 0, :, 0].tolist() == [1, 0]


def test_local_blocks_of():
    assert osg.local_blocks_of(16, 128) == 1
    assert osg.local_blocks_of(40, 32) == 2
    assert osg.local_blocks_of(0, 32) == 0


@pytest.mark.parametrize("S,rb,lw,r", [(200, 32, 16, 2), (256, 64, 0, 3), (96, 32, 40, 1)])
def test_allowed_key_stats_match_token_mask(S, rb, lw, r):
    rng = np.random.default_rng(7 * S)
    assign = rng.random((1, 2, S, 4, 2))
    route = osg.majority_route(assign, r, rb)
    bl = ob.build_block_lists(route, r, is_causal=True, sink_block=True,
                              local_blocks=osg.local_blocks_of(lw, rb), arity=2)
    mask = ob.lists_to_mask(bl.lists, bl.counts)
    tm = oa.token_mask_from_blocks(mask, rb, S, is_causal=True)
    st = osg.allowed_key_stats(bl.counts, S, rb)
    assert abs(st["mean_allowed_keys"] - tm.sum(-1).mean()) < 1e-9
    assert st["mean_causal_keys"] == (S + 1) / 2
    NB = -(-S // rb)
    assert abs(st["block_density"] - mask.sum() / (2 * NB * (NB + 1) / 2)) < 1e-12


def test_majority_route_nan_scores_match_torch_chain():
    # the reference's chain: argmax (first NaN wins) -> one-hot -> sum over the block -> argmax
    import torch
    g = torch.Generator().manual_seed(4)
    a = torch.randn(1, 2, 40, 2, 3, generator=g)
    a = a.masked_fill(torch.rand(a.shape, generator=g) < 0.2, float("nan"))
    rb = 8
    idx = a.argmax(-1)
    votes = torch.nn.functional.one_hot(idx, 3).float().view(1, 2, 5, rb, 2, 3).sum(3)
    ref = votes.argmax(-1).to(torch.int32).numpy()
    assert np.array_equal(osg.majority_route(a.numpy(), 2, rb), ref)
