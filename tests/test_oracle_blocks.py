"""Pins the block-list oracle (oracle/blocks.py) on the CPU.

Checks, each chosen so that a plausible mistake fails one of them:
  * a pure-Python brute force over (i, j) pairs (no codes, no numpy masks)
    on the parameter grids of the reference tests
    (tests/test_block_list.py:50-70, :96-128, :170-183);
  * known answers from the reference tests: depth 0 is dense and causal counts
    are 1..NB (:141-146); a binary tree router at depth r keeps NB/2^r blocks
    per row and is block-diagonal at full depth (:149-157); the diagonal is
    always listed (:131-138); sync-free lists equal syncing lists on the valid
    prefix and are padded to NB (:170-183); bad depths raise (:160-167);
  * the sync-free code alias (ids >= arity) read from block_list.py:212-229;
  * transposed lists against the transposed pairwise mask (:73-93).
"""

import itertools
import math

import numpy as np
import pytest

from oracle import blocks as ob


def random_router(Z, H, NB, TD, p, seed=0):
    return np.random.default_rng(seed).integers(0, p, size=(Z, H, NB, TD), dtype=np.int32)


def tree_router(Z, H, NB, TD):
    depth = max(1, math.ceil(math.log2(max(NB, 2))))
    r = np.zeros((Z, H, NB, TD), dtype=np.int32)
    for d in range(depth):
        r[:, :, :, d] = (np.arange(NB) >> (depth - 1 - d)) % 2
    return r


def brute_lists(router, depths, is_causal, sink, local):
    """Pure-Python pairwise rule, in the reference's order."""
    Z, H, NB, TD = router.shape
    out = {}
    for z, h, i in itertools.product(range(Z), range(H), range(NB)):
        d = depths[h]
        row = []
        for j in range(NB):
            m = all(int(router[z, h, i, l]) == int(router[z, h, j, l]) for l in range(d))
            if local > 0 and abs(i - j) <= local:
                m = True
            if sink and j == 0:
                m = True
            if is_causal and j > i:
                m = False
            if m:
                row.append(j)
        out[(z, h, i)] = row
    return out


def assert_lists(bl, expected, max_count=None):
    for (z, h, i), row in expected.items():
        assert int(bl.counts[z, h, i]) == len(row)
        assert bl.lists[z, h, i, :len(row)].tolist() == row
        assert (bl.lists[z, h, i, len(row):] == 0).all()
    if max_count is not None:
        assert bl.max_count == max_count == bl.lists.shape[-1]


@pytest.mark.parametrize("p", [2, 3])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("sink,local", [(False, 0), (True, 0), (False, 1), (True, 2)])
def test_builder_matches_brute_force(p, is_causal, sink, local):
    router = random_router(2, 3, 7, 4, p, seed=p)
    depth = [0, 2, 4]
    bl = ob.build_block_lists(router, np.array(depth), is_causal=is_causal, sink_block=sink,
                              local_blocks=local)
    exp = brute_lists(router, depth, is_causal, sink, local)
    assert_lists(bl, exp, max(len(r) for r in exp.values()))
    ref = ob.block_mask_reference(router, np.array(depth), is_causal=is_causal, sink_block=sink,
                                  local_blocks=local)
    assert (ref.sum(-1) == bl.counts).all()


@pytest.mark.parametrize("p", [2, 3])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("depth", [0, 1, 3, [0, 2]])
def test_sync_free_matches_syncing(p, is_causal, depth):
    router = random_router(2, 2, 9, 3, p, seed=7)
    a = ob.build_block_lists(router, depth, is_causal=is_causal, sink_block=True)
    b = ob.build_block_lists(router, depth, is_causal=is_causal, sink_block=True, arity=p)
    assert b.max_count == 9 and b.lists.shape[-1] == 9
    assert (a.counts == b.counts).all()
    for z, h, i in itertools.product(range(2), range(2), range(9)):
        c = int(a.counts[z, h, i])
        assert (a.lists[z, h, i, :c] == b.lists[z, h, i, :c]).all()
        assert (b.lists[z, h, i, c:] == 0).all()


def test_diagonal_always_present():
    router = random_router(1, 2, 9, 3, 2, seed=1)
    for causal in (False, True):
        bl = ob.build_block_lists(router, 3, is_causal=causal)
        for h, i in itertools.product(range(2), range(9)):
            assert i in bl.lists[0, h, i, :int(bl.counts[0, h, i])].tolist()


def test_depth_zero_is_dense():
    router = random_router(1, 2, 5, 3, 2)
    assert (ob.build_block_lists(router, 0).counts == 5).all()
    blc = ob.build_block_lists(router, 0, is_causal=True)
    assert blc.counts[0, 0].tolist() == [1, 2, 3, 4, 5]


def test_tree_router_closed_form():
    NB = 16
    router = tree_router(1, 1, NB, 4)
    bl = ob.build_block_lists(router, 4)
    assert (bl.counts == 1).all()
    assert bl.lists[0, 0, :, 0].tolist() == list(range(NB))
    for r in range(5):
        assert (ob.build_block_lists(router, r).counts == NB // 2 ** r).all()


def test_invalid_depth_raises():
    router = random_router(1, 2, 4, 3, 2)
    with pytest.raises(ValueError):
        ob.build_block_lists(router, 4)
    with pytest.raises(ValueError):
        ob.build_block_lists(router, [1, 2, 3])
    with pytest.raises(ValueError):
        ob.build_block_lists(router, 4, arity=2)
    with pytest.raises(ValueError):
        ob.build_block_lists(-random_router(1, 1, 4, 2, 2) - 1, 1)


def test_sync_free_code_alias():
    # base = arity = 2; ids (2, 0) and (0, 1) both encode to 2*1 + 0*2 = 0*1 + 1*2 = 2,
    # so the codes match although the vectors differ (block_list.py:212-229).
    router = np.array([[[[2, 0], [0, 1], [1, 1]]]], dtype=np.int32)  # (1, 1, 3, 2)
    bl = ob.build_block_lists(router, 2, arity=2)
    assert bl.lists[0, 0, 0, :int(bl.counts[0, 0, 0])].tolist() == [0, 1]
    # the syncing builder uses base = max(id) + 1 = 3: no alias.
    bs = ob.build_block_lists(router, 2)
    assert bs.lists[0, 0, 0, :int(bs.counts[0, 0, 0])].tolist() == [0]


def test_elementwise_path_matches_codes_path():
    # TD * log2(base) >= 62 switches to element-wise equality (block_list.py:225-258).
    router = random_router(1, 2, 12, 40, 3, seed=5)
    router[..., 2:] = 0
    bl = ob.build_block_lists(router, [2, 40], sink_block=True)
    exp = brute_lists(router, [2, 40], False, True, 0)
    assert_lists(bl, exp)


@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("sink,local", [(False, 0), (True, 0), (False, 1), (True, 2)])
def test_transposed_lists(is_causal, sink, local):
    router = random_router(2, 3, 7, 4, 2, seed=42)
    depth = np.array([0, 2, 4])
    bl = ob.build_block_lists(router, depth, is_causal=is_causal, sink_block=sink, local_blocks=local)
    t = ob.build_transposed_block_lists(bl.lists, bl.counts, 7)
    exp = brute_lists(router, [0, 2, 4], is_causal, sink, local)
    for z, h, kb in itertools.product(range(2), range(3), range(7)):
        col = [i for i in range(7) if kb in exp[(z, h, i)]]
        assert int(t.counts[z, h, kb]) == len(col)
        assert t.lists[z, h, kb, :len(col)].tolist() == col


def test_mask_compaction_matches_brute_force():
    rng = np.random.default_rng(3)
    mask = rng.random((1, 2, 10, 10)) < 0.3
    bl = ob.block_lists_from_mask(mask, is_causal=True, sink_block=True, local_blocks=1)
    for h, i in itertools.product(range(2), range(10)):
        row = [j for j in range(10) if (mask[0, h, i, j] or abs(i - j) <= 1 or j == 0) and j <= i]
        assert bl.lists[0, h, i, :int(bl.counts[0, h, i])].tolist() == row
    assert bl.max_count == 10
