"""GPU parity of the surgery caller (src/llama_surgery/surgery.py:521-601):
the HIP route-block vote bit-exact against the oracle (fp32 / bf16 / fp16
scores, strided inputs, direct block routing, config-5 shape), and
block_list_prefill against the masked-dense oracle on the reference test's
grid (tests/test_surgery_block_list.py:61-95: fp16 <= 2e-3, statistics equal
to the token-mask counts), plus GQA."""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import blocks as ob
from oracle import surgery as osg
from ultrametric import block_list_prefill, route_block_vote

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("S,rb,r,p,L", [(200, 32, 2, 2, 4), (333, 16, 4, 4, 4), (1000, 128, 3, 5, 3),
                                        (7, 128, 2, 2, 2)])
def test_vote_matches_oracle(dtype, S, rb, r, p, L):
    g = torch.Generator().manual_seed(S * p + r)
    a = torch.randn(2, 3, S, L, p, generator=g).to(dtype)
    ref = osg.majority_route(a.float().numpy(), r, rb)
    got = route_block_vote(a.to(DEV), r, rb)
    assert np.array_equal(got.cpu().numpy(), ref)


def test_vote_ties_and_strided():
    # quantised scores: many exact ties between branches and between vote counts
    g = torch.Generator().manual_seed(3)
    a = torch.randint(0, 2, (1, 4, 300, 2, 3), generator=g).float()
    ref = osg.majority_route(a.numpy(), 2, 8)
    assert np.array_equal(route_block_vote(a.to(DEV), 2, 8).cpu().numpy(), ref)
    # non-contiguous view: levels and branches permuted in memory
    base = torch.randn(1, 4, 300, 3, 2, generator=g)
    view = base.transpose(-1, -2)            # (1, 4, 300, 2, 3), strided
    ref = osg.majority_route(view.contiguous().numpy(), 2, 32)
    assert np.array_equal(route_block_vote(view.to(DEV), 2, 32).cpu().numpy(), ref)
    # direct block routing (route_block = 1)
    ref = osg.direct_route(view.contiguous().numpy(), 2)
    assert np.array_equal(route_block_vote(view.to(DEV), 2, 1).cpu().numpy(), ref)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_vote_nan_scores_follow_torch_argmax(dtype):
    # torch.argmax (surgery.py:543) treats the first NaN of a token's scores as
    # the maximum; the vote counts that branch.
    g = torch.Generator().manual_seed(9)
    a = torch.randn(1, 2, 96, 3, 4, generator=g)
    nan = torch.rand(1, 2, 96, 3, 4, generator=g) < 0.15
    a = a.masked_fill(nan, float("nan")).to(dtype)
    ref = osg.majority_route(a.float().numpy(), 3, 16)
    assert np.array_equal(route_block_vote(a.to(DEV), 3, 16).cpu().numpy(), ref)
    # the strided (non-vector) path too
    view = a.float().transpose(-1, -2).contiguous().transpose(-1, -2).to(dtype)
    assert np.array_equal(route_block_vote(view.to(DEV), 3, 16).cpu().numpy(), ref)


def test_vote_config5_shape():
    # config 5: 32 heads, N = 16384, route block 128, p = 4, 4 levels, r = 2
    g = torch.Generator().manual_seed(5)
    a = torch.randn(1, 32, 16384, 4, 4, generator=g)
    ref = osg.majority_route(a.numpy(), 2, 128)
    assert np.array_equal(route_block_vote(a.to(DEV), 2, 128).cpu().numpy(), ref)


@pytest.mark.parametrize("S,rb,lw,r", [(200, 32, 16, 2), (256, 64, 0, 3), (96, 32, 40, 1)])
def test_block_list_prefill_matches_oracle(S, rb, lw, r):
    torch.manual_seed(S + r)
    B, H, D, L, p = 1, 2, 32, 4, 2
    q, k, v = (torch.randn(B, H, S, D).to(torch.float16) for _ in range(3))
    assign = torch.softmax(torch.randn(B, H, S, L, p), dim=-1)
    scale = 1.0 / math.sqrt(D)
    out, st = block_list_prefill(q.to(DEV), k.to(DEV), v.to(DEV), assign.to(DEV), r, p=p, route_block=rb,
                                 local_window=lw, sm_scale=scale, return_stats=True)
    route = osg.majority_route(assign.numpy(), r, rb)
    bl = ob.build_block_lists(route, r, is_causal=True, sink_block=True,
                              local_blocks=osg.local_blocks_of(lw, rb), arity=p)
    mask = ob.lists_to_mask(bl.lists, bl.counts)
    ref, _ = oa.block_sparse_attention_ref(q.float().numpy(), k.float().numpy(), v.float().numpy(), mask, rb,
                                           is_causal=True, sm_scale=scale)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-3
    tm = oa.token_mask_from_blocks(mask, rb, S, is_causal=True)
    assert abs(st["mean_allowed_keys"] - tm.sum(-1).mean()) < 1e-3
    assert abs(st["mean_causal_keys"] - (S + 1) / 2) < 1e-9


def test_block_list_prefill_gqa_bf16_direct_blocks():
    torch.manual_seed(9)
    B, H, Hkv, S, D, L, p, rb, r = 1, 8, 2, 640, 64, 3, 4, 128, 2
    q = torch.randn(B, H, S, D).to(torch.bfloat16)
    k, v = (torch.randn(B, Hkv, S, D).to(torch.bfloat16) for _ in range(2))
    NB = S // rb
    blk = torch.randn(B, H, NB, L, p)            # per-block scores: direct routing
    out = block_list_prefill(q.to(DEV), k.to(DEV), v.to(DEV), blk.to(DEV), r, p=p, route_block=rb,
                             local_window=16)
    route = osg.direct_route(blk.numpy(), r)
    bl = ob.build_block_lists(route, r, is_causal=True, sink_block=True, local_blocks=1, arity=p)
    mask = ob.lists_to_mask(bl.lists, bl.counts)
    ref, _ = oa.block_sparse_attention_ref(q.float().numpy(), k.float().numpy(), v.float().numpy(), mask, rb,
                                           is_causal=True)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 2e-2


def test_route_cache_reuses_anchor_lists():
    # stride 2: layers 1 and 3 reuse the lists of anchors 0 and 2 and never read their own scores
    from ultrametric import RouteCache
    torch.manual_seed(21)
    B, H, S, D, L, p, rb, r = 1, 4, 2048, 64, 3, 2, 128, 2
    q, k, v = (torch.randn(B, H, S, D).to(torch.bfloat16).to(DEV) for _ in range(3))
    a0, a1 = (torch.randn(B, H, S, L, p).to(DEV) for _ in range(2))
    cache = RouteCache(stride=2)
    kw = dict(p=p, route_block=rb, local_window=16)
    fresh0 = block_list_prefill(q, k, v, a0, r, **kw)
    fresh1 = block_list_prefill(q, k, v, a1, r, **kw)
    assert not torch.equal(fresh0, fresh1)
    assert torch.equal(block_list_prefill(q, k, v, a0, r, route_cache=cache, layer_idx=0, **kw), fresh0)
    assert torch.equal(block_list_prefill(q, k, v, a1, r, route_cache=cache, layer_idx=1, **kw), fresh0)
    assert torch.equal(block_list_prefill(q, k, v, a1, r, route_cache=cache, layer_idx=2, **kw), fresh1)
    assert torch.equal(block_list_prefill(q, k, v, a0, r, route_cache=cache, layer_idx=3, **kw), fresh1)
    # a different routing depth is a different key: layer 3 routes by itself
    got = block_list_prefill(q, k, v, a0, 1, route_cache=cache, layer_idx=3, **kw)
    assert torch.equal(got, block_list_prefill(q, k, v, a0, 1, **kw))


def test_block_list_prefill_config5_layer():
    # config 5: one Llama-3.1-8B layer at N = 16384 (32 query / 8 kv heads, D 128,
    # route block 128, p = 4, 4 levels, r = 2, local window 16 -> 1 block, sink)
    g = torch.Generator().manual_seed(55)
    B, H, Hkv, S, D, L, p, rb, r = 1, 32, 8, 16384, 128, 4, 4, 128, 2
    q = torch.randn(B, H, S, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    v = torch.randn(B, Hkv, S, D, generator=g).to(torch.bfloat16)
    a = torch.randn(B, H, S, L, p, generator=g)
    out, st = block_list_prefill(q.to(DEV), k.to(DEV), v.to(DEV), a.to(DEV), r, p=p, route_block=rb,
                                 local_window=16, return_stats=True)
    route = osg.majority_route(a.numpy(), r, rb)
    bl = ob.build_block_lists(route, r, is_causal=True, sink_block=True, local_blocks=1, arity=p)
    mask = ob.lists_to_mask(bl.lists, bl.counts)
    heads = [(0, 0), (0, 13), (0, 31)]
    kk = np.repeat(k.float().numpy(), H // Hkv, axis=1)
    vv = np.repeat(v.float().numpy(), H // Hkv, axis=1)
    ref, _ = oa.block_sparse_attention_ref(q.float().numpy(), kk, vv, mask, rb, is_causal=True, heads=heads)
    got = out.float().cpu().numpy()
    for z, h in heads:
        assert np.abs(got[z, h] - ref[z, h]).max() <= 2e-2, h
    assert torch.isfinite(out).all()
    # r = 2 of 4 levels with 4 branches: a block matches about 1/16 of the
    # earlier blocks; with the diagonal, sink and one local block that is
    # about 10% of the 8256 causal blocks per head
    assert 0.05 < st["block_density"] < 0.15


def _dense_with_block_bias(q, k, v, lists, counts, bias, rb, scale):
    """Token-level masked attention in float32 (torch on the GPU) with the
    per-(query block, list slot) bias added to that pair's scores."""
    Z, H, S, D = q.shape
    NB = counts.shape[-1]
    slot = torch.arange(lists.shape[-1], device=q.device).view(1, 1, 1, -1) < counts.unsqueeze(-1)
    kb = lists.clamp(0, NB - 1).long()
    # padding entries (kb 0, slot False) share index 0 with the sink: add, do not overwrite
    allowed = torch.zeros(Z, H, NB, NB, dtype=torch.int32, device=q.device).scatter_add(-1, kb, slot.int()) > 0
    bfull = torch.zeros(Z, H, NB, NB, dtype=torch.float32, device=q.device).scatter_add(
        -1, kb, torch.where(slot, bias, torch.zeros_like(bias)))
    tok = torch.arange(S, device=q.device) // rb
    m = allowed[:, :, tok][:, :, :, tok] & (torch.arange(S, device=q.device).view(-1, 1)
                                           >= torch.arange(S, device=q.device).view(1, -1))
    s = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale + bfull[:, :, tok][:, :, :, tok]
    s = s.masked_fill(~m, float("-inf"))
    return torch.matmul(torch.softmax(s, dim=-1), v)


def test_router_gradient_through_the_straight_through_bias():
    # block_list_prefill with scores that require grad adds the zero-valued STE
    # bias (surgery.py:566-588); the scores' gradient through the kernel's
    # soft-bias backward equals the one through dense masked attention with the
    # same bias (float32 inputs: the fp32 kernels)
    from ultrametric import build_block_lists
    from ultrametric.surgery import _block_mean, ste_soft_block_bias, local_blocks_of
    B, H, S, D, rb, L, p, r = 1, 2, 300, 64, 64, 3, 4, 2
    g = torch.Generator().manual_seed(11)
    q, k, v = (torch.randn(B, H, S, D, generator=g).to(DEV) for _ in range(3))
    scores = torch.randn(B, H, S, L, p, generator=g).to(DEV)
    a1 = torch.softmax(scores, -1).detach().requires_grad_(True)
    a2 = a1.detach().clone().requires_grad_(True)
    dout = torch.randn(B, H, S, D, generator=g).to(DEV)
    scale = 1.0 / math.sqrt(D)
    out = block_list_prefill(q, k, v, a1, r, p=p, route_block=rb, local_window=16, sm_scale=scale)
    with torch.no_grad():
        out_ng = block_list_prefill(q, k, v, a1, r, p=p, route_block=rb, local_window=16, sm_scale=scale)
    assert torch.equal(out, out_ng)                    # the bias is zero in the forward pass
    out.backward(dout)
    route = route_block_vote(a2.detach(), r, rb)
    bl = build_block_lists(route, r, is_causal=True, sink_block=True, local_blocks=local_blocks_of(16, rb), arity=p)
    bias = ste_soft_block_bias(_block_mean(a2, S, rb), bl.lists, r, p)
    ref = _dense_with_block_bias(q, k, v, bl.lists, bl.counts, bias, rb, scale)
    assert torch.allclose(out, ref, atol=1e-4, rtol=0)
    ref.backward(dout)
    assert a1.grad.abs().max() > 0
    err = (a1.grad - a2.grad).abs().max() / a2.grad.abs().max()
    assert err <= 1e-4, err
