"""GPU parity: the HIP block-list compaction is bit-exact with the CPU oracle
(oracle/blocks.py), including zero padding, for the parameter grids of the
reference tests (tests/test_block_list.py:50-183) and the BASELINE shapes."""

import itertools

import numpy as np
import pytest
import torch

import sparse_workloads as wl
from oracle import blocks as ob
from ultrametric import (block_lists_from_mask, build_block_lists, build_transposed_block_lists)

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rand_router(Z, H, NB, TD, p, seed, dtype=np.int32):
    return np.random.default_rng(seed).integers(0, p, size=(Z, H, NB, TD)).astype(dtype)


def assert_same(bl, ref, check_padding=True):
    assert bl.max_count == ref.max_count
    assert tuple(bl.lists.shape) == ref.lists.shape
    assert np.array_equal(bl.counts.cpu().numpy(), ref.counts)
    got = bl.lists.cpu().numpy()
    if check_padding:
        assert np.array_equal(got, ref.lists)
    else:
        for idx in np.ndindex(ref.counts.shape):
            c = ref.counts[idx]
            assert np.array_equal(got[idx][:c], ref.lists[idx][:c])


@pytest.mark.parametrize("p", [2, 3])
@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("sink,local", [(False, 0), (True, 0), (False, 1), (True, 2)])
@pytest.mark.parametrize("sync_free", [False, True])
def test_builder_grid(p, is_causal, sink, local, sync_free):
    router = rand_router(2, 3, 7, 4, p, seed=p)
    depth = [0, 2, 4]
    kw = dict(is_causal=is_causal, sink_block=sink, local_blocks=local)
    ar = p if sync_free else None
    ref = ob.build_block_lists(router, np.array(depth), arity=ar, **kw)
    bl = build_block_lists(torch.from_numpy(router).to(DEV), torch.tensor(depth), arity=ar, **kw)
    assert bl.lists.dtype == torch.int32 and bl.counts.dtype == torch.int32
    assert_same(bl, ref)


@pytest.mark.parametrize("depth", [0, 1, 3])
@pytest.mark.parametrize("id_dtype", [np.int32, np.int64])
def test_uniform_depth_sync_free_int_types(depth, id_dtype):
    router = rand_router(2, 2, 9, 3, 3, seed=7, dtype=id_dtype)
    ref = ob.build_block_lists(router, depth, is_causal=True, sink_block=True, arity=3)
    bl = build_block_lists(torch.from_numpy(router).to(DEV), depth, is_causal=True, sink_block=True, arity=3)
    assert_same(bl, ref)


def test_non_contiguous_router_and_alias():
    base = rand_router(1, 4, 33, 6, 2, seed=9)
    r = torch.from_numpy(base).to(DEV).transpose(1, 2).contiguous().transpose(1, 2)[..., ::2]
    assert not r.is_contiguous()
    ref = ob.build_block_lists(r.cpu().numpy(), 2, local_blocks=1, arity=2)
    assert_same(build_block_lists(r, 2, local_blocks=1, arity=2), ref)
    # ids >= arity alias through the mixed-radix code in sync-free mode
    router = np.array([[[[2, 0], [0, 1], [1, 1]]]], dtype=np.int32)
    bl = build_block_lists(torch.from_numpy(router).to(DEV), 2, arity=2)
    assert bl.lists[0, 0, 0, :int(bl.counts[0, 0, 0])].tolist() == [0, 1]
    assert_same(bl, ob.build_block_lists(router, 2, arity=2))


def test_elementwise_path():
    router = rand_router(1, 2, 12, 40, 3, seed=5)
    router[..., 2:] = 0
    ref = ob.build_block_lists(router, [2, 40], sink_block=True)
    assert_same(build_block_lists(torch.from_numpy(router).to(DEV), [2, 40], sink_block=True), ref)


@pytest.mark.parametrize("NB", [1, 63, 64, 65, 200, 1000, 4100])
def test_large_nb(NB):
    router = rand_router(1, 2, NB, 5, 2, seed=NB)
    for causal in (False, True):
        ref = ob.build_block_lists(router, [3, 5], is_causal=causal, sink_block=True, local_blocks=2)
        bl = build_block_lists(torch.from_numpy(router).to(DEV), [3, 5], is_causal=causal,
                               sink_block=True, local_blocks=2)
        assert_same(bl, ref)


def test_config2_and_config5_shapes():
    c2 = wl.config2(device="cpu", N=8192)
    r = c2["router"].numpy()
    ref = ob.build_block_lists(r, 2, is_causal=True, sink_block=True, arity=4)
    bl = build_block_lists(c2["router"].to(DEV), 2, is_causal=True, sink_block=True, arity=4)
    assert_same(bl, ref)
    # config 5: (1, 32, 128, 4) routes from argmax of N(0,1) logits, r = 2, local 1
    g = torch.Generator().manual_seed(5)
    route = torch.randn(1, 32, 128, 4, 4, generator=g).argmax(-1).to(torch.int32)
    ref = ob.build_block_lists(route.numpy(), 2, is_causal=True, sink_block=True, local_blocks=1, arity=4)
    bl = build_block_lists(route.to(DEV), 2, is_causal=True, sink_block=True, local_blocks=1, arity=4)
    assert_same(bl, ref)


@pytest.mark.parametrize("NB,density", [(16, 0.25), (64, 0.05), (300, 0.5)])
@pytest.mark.parametrize("sync_free", [True, False])
def test_mask_compaction(NB, density, sync_free):
    rng = np.random.default_rng(NB)
    mask = rng.random((2, 3, NB, NB)) < density
    for kw in (dict(), dict(is_causal=True, sink_block=True, local_blocks=1)):
        ref = ob.block_lists_from_mask(mask, sync_free=sync_free, **kw)
        bl = block_lists_from_mask(torch.from_numpy(mask).to(DEV), sync_free=sync_free, **kw)
        assert_same(bl, ref)


@pytest.mark.parametrize("is_causal", [False, True])
@pytest.mark.parametrize("sink,local", [(False, 0), (True, 0), (False, 1), (True, 2)])
def test_transposed_lists(is_causal, sink, local):
    router = rand_router(2, 3, 7, 4, 2, seed=42)
    depth = [0, 2, 4]
    kw = dict(is_causal=is_causal, sink_block=sink, local_blocks=local)
    bl = build_block_lists(torch.from_numpy(router).to(DEV), depth, **kw)
    ref_bl = ob.build_block_lists(router, np.array(depth), **kw)
    ref = ob.build_transposed_block_lists(ref_bl.lists, ref_bl.counts, 7)
    assert_same(build_transposed_block_lists(bl, num_key_blocks=7), ref)


def test_empty_and_dense_edges():
    r = torch.zeros(1, 2, 0, 3, dtype=torch.int32, device=DEV)
    bl = build_block_lists(r, 1)
    assert bl.max_count == 0 and bl.lists.shape == (1, 2, 0, 0)
    bl = build_block_lists(r, 1, arity=2)
    assert bl.max_count == 0
    r = torch.from_numpy(rand_router(1, 2, 5, 3, 2, seed=0)).to(DEV)
    assert torch.all(build_block_lists(r, 0).counts == 5)
    assert build_block_lists(r, 0, is_causal=True).counts[0, 0].tolist() == [1, 2, 3, 4, 5]


@pytest.mark.parametrize("NB,density", [(33, 0.3), (300, 0.05), (512, 0.02), (600, 0.01), (1200, 0.004),
                                        (2100, 0.002)])
def test_transposed_lists_large(NB, density):
    # the HIP transpose kernel: one key-block chunk per head up to NB = 512,
    # several chunks above (431 key blocks per chunk at NB = 1200, 244 at 2100)
    rng = np.random.default_rng(NB + 1)
    mask = rng.random((1, 2, NB, NB)) < density
    mask[..., 0] = True                       # a full sink column
    bl = block_lists_from_mask(torch.from_numpy(mask).to(DEV), sync_free=False)
    ref_bl = ob.block_lists_from_mask(mask, sync_free=False)
    ref = ob.build_transposed_block_lists(ref_bl.lists, ref_bl.counts, NB)
    assert_same(build_transposed_block_lists(bl, num_key_blocks=NB), ref)
