"""GPU parity of the block-list backward (dQ, dK, dV and the straight-through
soft-bias gradient) against the float64 gradient oracle
(oracle/attention.py:block_sparse_attention_grad_ref), on the reference's own
grid and tolerances (tests/test_block_list.py:260-351: fp16 <= 5e-3, fp32 <= 1e-4)
plus GQA and bf16 at the MFMA shapes (<= 2e-2 relative to the gradient scale)."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import blocks as ob
from ultrametric import block_list_attention, build_block_lists

pytestmark = pytest.mark.gpu
DEV = "cuda"


def random_router(Z, H, NB, TD, p, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, p, (Z, H, NB, TD), generator=g, dtype=torch.int32)


def run(q0, k0, v0, do, bl, rb, causal, bias=None):
    q, k, v = (t.to(DEV).clone().requires_grad_(True) for t in (q0, k0, v0))
    out = block_list_attention(q, k, v, bl, route_block=rb, is_causal=causal, soft_block_bias=bias)
    out.backward(do.to(DEV))
    return q.grad.float().cpu().numpy(), k.grad.float().cpu().numpy(), v.grad.float().cpu().numpy()


def oracle(q0, k0, v0, do, bl, rb, causal, pair_bias=None):
    bm = ob.lists_to_mask(bl.lists.cpu().numpy(), bl.counts.cpu().numpy())
    f = lambda t: t.float().numpy()  # noqa: E731
    return oa.block_sparse_attention_grad_ref(f(q0), f(k0), f(v0), bm, rb, f(do), is_causal=causal,
                                              pair_bias=pair_bias)


@pytest.mark.parametrize("dtype,tol", [(torch.float16, 5e-3), (torch.float32, 1e-4)])
@pytest.mark.parametrize("N,rb,depth,causal,sink,local", [(128, 64, 1, False, False, 0),
                                                           (100, 32, 2, True, True, 0),
                                                           (96, 32, 1, False, False, 1)])
def test_backward_reference_grid(dtype, tol, N, rb, depth, causal, sink, local):
    torch.manual_seed(42)
    Z, H, D = 1, 2, 16
    q0, k0, v0, do = (torch.randn(Z, H, N, D).to(dtype) for _ in range(4))
    NB = math.ceil(N / rb)
    router = random_router(Z, H, NB, 3, 2, seed=N).to(DEV)
    bl = build_block_lists(router, depth, is_causal=causal, sink_block=sink, local_blocks=local)
    got = run(q0, k0, v0, do, bl, rb, causal)
    ref = oracle(q0, k0, v0, do, bl, rb, causal)
    for g_, r_, name in zip(got, ref[:3], "qkv"):
        assert np.abs(g_ - r_).max() < tol, name


@pytest.mark.parametrize("causal", [False, True])
def test_backward_soft_bias_ste(causal):
    torch.manual_seed(99)
    Z, H, N, D, rb = 1, 2, 96, 16, 32
    q0, k0, v0, do = (torch.randn(Z, H, N, D) for _ in range(4))
    NB = math.ceil(N / rb)
    router = random_router(Z, H, NB, 3, 2, seed=17).to(DEV)
    bl = build_block_lists(router, 1, is_causal=causal, sink_block=True)
    raw = torch.randn(Z, H, NB, bl.max_count, device=DEV, requires_grad=True)
    ste = raw - raw.detach()            # zero-valued: forward unchanged, d/draw = d/dbias
    q, k, v = (t.to(DEV).clone().requires_grad_(True) for t in (q0, k0, v0))
    out = block_list_attention(q, k, v, bl, route_block=rb, is_causal=causal, soft_block_bias=ste)
    out.backward(do.to(DEV))
    lists, counts = bl.lists.cpu().numpy(), bl.counts.cpu().numpy()
    bm = ob.lists_to_mask(lists, counts)
    _, _, _, dpb = oa.block_sparse_attention_grad_ref(q0.numpy(), k0.numpy(), v0.numpy(), bm, rb, do.numpy(),
                                                      is_causal=causal, pair_bias=np.zeros((Z, H, NB, NB)))
    want = np.zeros((Z, H, NB, bl.max_count))
    for h in range(H):
        for qb in range(NB):
            for t in range(counts[0, h, qb]):
                want[0, h, qb, t] = dpb[0, h, qb, lists[0, h, qb, t]]
    assert np.abs(raw.grad.cpu().numpy() - want).max() < 1e-4


def test_backward_nonzero_bias_gqa_fp32():
    torch.manual_seed(3)
    Z, H, Hkv, N, D, rb = 1, 4, 2, 160, 32, 32
    q0, do = (torch.randn(Z, H, N, D) for _ in range(2))
    k0, v0 = (torch.randn(Z, Hkv, N, D) for _ in range(2))
    NB = N // rb
    router = random_router(Z, H, NB, 2, 2, seed=4).to(DEV)
    bl = build_block_lists(router, 1, is_causal=True, sink_block=True, local_blocks=1)
    bias = torch.randn(Z, H, NB, bl.max_count) * 0.5
    got = run(q0, k0, v0, do, bl, rb, True, bias=bias.to(DEV))
    lists, counts = bl.lists.cpu().numpy(), bl.counts.cpu().numpy()
    pb = np.zeros((Z, H, NB, NB))
    for h in range(H):
        for qb in range(NB):
            for t in range(counts[0, h, qb]):
                pb[0, h, qb, lists[0, h, qb, t]] = bias[0, h, qb, t]
    ref = oracle(q0, k0, v0, do, bl, rb, True, pair_bias=pb)
    for g_, r_, name in zip(got, ref[:3], "qkv"):
        assert np.abs(g_ - r_).max() < 1e-4, name


@pytest.mark.parametrize("H,Hkv,N,D,rb", [(4, 4, 512, 64, 64), (8, 2, 640, 128, 128)])
def test_backward_bf16_gqa(H, Hkv, N, D, rb):
    torch.manual_seed(H + N)
    Z = 1
    q0, do = (torch.randn(Z, H, N, D).to(torch.bfloat16) for _ in range(2))
    k0, v0 = (torch.randn(Z, Hkv, N, D).to(torch.bfloat16) for _ in range(2))
    NB = N // rb
    router = random_router(Z, H, NB, 3, 2, seed=N).to(DEV)
    bl = build_block_lists(router, 2, is_causal=True, sink_block=True, arity=2)
    got = run(q0, k0, v0, do, bl, rb, True)
    ref = oracle(q0, k0, v0, do, bl, rb, True)
    for g_, r_, name in zip(got, ref[:3], "qkv"):
        scale = max(1.0, np.abs(r_).max())
        assert np.abs(g_ - r_).max() <= 2e-2 * scale, name


def pair_bias_of(bias, bl):
    lists, counts = bl.lists.cpu().numpy(), bl.counts.cpu().numpy()
    Z, H, NB, _ = bias.shape
    pb = np.zeros((Z, H, NB, NB))
    for z in range(Z):
        for h in range(H):
            for qb in range(NB):
                for t in range(counts[z, h, qb]):
                    pb[z, h, qb, lists[z, h, qb, t]] = bias[z, h, qb, t]
    return pb


def check_grads(got, ref, rel=2e-2):
    for g_, r_, name in zip(got, ref, "qkv"):
        scale = max(1.0, np.abs(r_).max())
        err = np.abs(g_ - r_).max()
        assert err <= rel * scale, (name, err, scale)


# MFMA path: bf16 / fp16, D in {32, 64, 128}, route blocks 32 .. 256 (one to
# four waves per workgroup, two key tiles per route block at 256), ragged N,
# soft bias, and sink columns long enough to split a key tile into several
# work items (fp32 partials summed by the finalize kernel).
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("H,Hkv,N,D,rb,causal,bias", [
    (2, 2, 1000, 128, 128, True, False),    # ragged tail
    (4, 1, 2048, 128, 128, True, True),     # sink tile of 4 x 16 entries: 4 items of 16
    (2, 2, 2176, 128, 128, True, False),    # 17 sink entries: items of 16 and 1
    (2, 2, 1536, 64, 64, False, True),      # two waves per workgroup
    (4, 2, 2048, 64, 64, True, True),       # route block 64: sink tile of 2 x 32 entries, 2 items of 32
    (2, 1, 640, 32, 32, True, False),       # one wave per workgroup
    (4, 1, 1024, 64, 32, True, False),      # route block 32: sink tile of 4 x 32 entries, 2 items of 64
    (2, 2, 2048, 128, 256, True, True),     # two key tiles per route block
    (3, 3, 777, 64, 128, False, False),
])
def test_backward_mfma(dtype, H, Hkv, N, D, rb, causal, bias):
    torch.manual_seed(N + D + rb)
    Z = 1
    q0, do = (torch.randn(Z, H, N, D).to(dtype) for _ in range(2))
    k0, v0 = (torch.randn(Z, Hkv, N, D).to(dtype) for _ in range(2))
    NB = -(-N // rb)
    router = random_router(Z, H, NB, 3, 2, seed=N + 1).to(DEV)
    bl = build_block_lists(router, 2, is_causal=causal, sink_block=True, local_blocks=1, arity=2)
    sb = (torch.randn(Z, H, NB, bl.max_count) * 0.5) if bias else None
    got = run(q0, k0, v0, do, bl, rb, causal, bias=None if sb is None else sb.to(DEV))
    ref = oracle(q0, k0, v0, do, bl, rb, causal, pair_bias=None if sb is None else pair_bias_of(sb.numpy(), bl))
    check_grads(got, ref[:3])


@pytest.mark.parametrize("causal", [False, True])
def test_backward_mfma_soft_bias_ste(causal):
    # straight-through bias gradient on the MFMA path, with split sink tiles
    torch.manual_seed(7)
    Z, H, Hkv, N, D, rb = 1, 4, 2, 1280, 64, 64
    q0, do = (torch.randn(Z, H, N, D).to(torch.bfloat16) for _ in range(2))
    k0, v0 = (torch.randn(Z, Hkv, N, D).to(torch.bfloat16) for _ in range(2))
    NB = N // rb
    router = random_router(Z, H, NB, 3, 2, seed=23).to(DEV)
    bl = build_block_lists(router, 1, is_causal=causal, sink_block=True, arity=2)
    raw = torch.randn(Z, H, NB, bl.max_count, device=DEV, requires_grad=True)
    ste = raw - raw.detach()
    q, k, v = (t.to(DEV).clone().requires_grad_(True) for t in (q0, k0, v0))
    out = block_list_attention(q, k, v, bl, route_block=rb, is_causal=causal, soft_block_bias=ste)
    out.backward(do.to(DEV))
    lists, counts = bl.lists.cpu().numpy(), bl.counts.cpu().numpy()
    bm = ob.lists_to_mask(lists, counts)
    f = lambda t: t.float().numpy()  # noqa: E731
    ref = oa.block_sparse_attention_grad_ref(f(q0), f(k0), f(v0), bm, rb, f(do), is_causal=causal,
                                             pair_bias=np.zeros((Z, H, NB, NB)))
    want = np.zeros((Z, H, NB, bl.max_count))
    for h in range(H):
        for qb in range(NB):
            for t in range(counts[0, h, qb]):
                want[0, h, qb, t] = ref[3][0, h, qb, lists[0, h, qb, t]]
    got = raw.grad.cpu().numpy()
    assert np.abs(got - want).max() <= 2e-2 * max(1.0, np.abs(want).max())
    check_grads((q.grad.float().cpu().numpy(), k.grad.float().cpu().numpy(), v.grad.float().cpu().numpy()),
                ref[:3])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_backward_expanded_output_gradient(dtype):
    # out.sum() hands the backward an expanded gradient (every stride 0): the
    # same gradients as an explicit, contiguous all-ones gradient
    torch.manual_seed(11)
    Z, H, N, D, rb = 1, 2, 320, 64, 64
    q0, k0, v0 = (torch.randn(Z, H, N, D).to(dtype) for _ in range(3))
    router = random_router(Z, H, N // rb, 3, 2, seed=5).to(DEV)
    bl = build_block_lists(router, 1, is_causal=True, sink_block=True, arity=2)
    q, k, v = (t.to(DEV).clone().requires_grad_(True) for t in (q0, k0, v0))
    block_list_attention(q, k, v, bl, route_block=rb, is_causal=True).sum().backward()
    got = (q.grad.float().cpu().numpy(), k.grad.float().cpu().numpy(), v.grad.float().cpu().numpy())
    ones = torch.ones(Z, H, N, D).to(dtype)
    ref = oracle(q0, k0, v0, ones, bl, rb, True)
    check_grads(got, ref[:3], rel=2e-2 if dtype == torch.bfloat16 else 1e-4)
