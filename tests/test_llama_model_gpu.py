"""GPU parity of the config-5 model harness (ultrametric.llama_model) on two
decoder layers at reduced N: the attention each layer computes through
block_list_prefill (route-block vote, sync-free lists, GQA prefill) is checked
against the oracle on the q / k / v / routing scores that layer actually
produced (oracle/surgery.py majority vote -> oracle/blocks.py lists ->
oracle/attention.py masked-dense float64, bf16 tolerance 2e-2), and the lists
against the oracle's bit for bit. With r = 0 (every causal block) the same
model must agree with its dense SDPA condition (the reference benchmark's
``dense_sdpa`` baseline, experiments/bench_surgery_prefill.py:146-178)."""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import blocks as ob
from oracle import surgery as osg
from ultrametric.llama_model import LlamaShape, SurgeryLlama

pytestmark = pytest.mark.gpu
DEV = "cuda"
SHAPE = LlamaShape(layers=2, vocab=4096)   # Llama-3.1-8B layer shape, two layers, small vocabulary


def _capture(model):
    """Wrap core_attention to keep each layer's inputs and output on the host."""
    seen = []
    inner = model.core_attention

    def wrapped(layer, q, k, v, collect_stats=False):
        o = inner(layer, q, k, v, collect_stats)
        seen.append((layer, q.float().cpu().numpy(), k.float().cpu().numpy(), v.float().cpu().numpy(),
                     o.float().cpu().numpy()))
        return o

    model.core_attention = wrapped
    return seen


@pytest.fixture(scope="module")
def model():
    return SurgeryLlama(SHAPE, device=DEV, seed=3, r=2)


@pytest.mark.parametrize("S,r", [(2048, 2), (1000, 3)])
def test_two_layers_block_list_matches_oracle(model, S, r):
    model.r = r
    g = torch.Generator().manual_seed(S)
    ids = torch.randint(0, SHAPE.vocab, (1, S), generator=g).to(DEV)
    seen = _capture(model)
    try:
        out = model(ids, collect_stats=True)
    finally:
        del model.core_attention
    assert out.shape == (1, S, SHAPE.hidden) and torch.isfinite(out).all()
    assert [s[0] for s in seen] == [0, 1]
    rb, H = model.route_block, SHAPE.heads
    heads = [(0, h) for h in (0, 5, 17, 31)]
    for layer, q, k, v, o in seen:
        scores = model.routing_scores(layer, 1, S).float().cpu().numpy()
        route = osg.majority_route(scores, r, rb)
        bl = ob.build_block_lists(route, r, is_causal=True, sink_block=True,
                                  local_blocks=osg.local_blocks_of(model.local_window, rb), arity=model.p)
        mask = ob.lists_to_mask(bl.lists, bl.counts)
        ref, _ = oa.block_sparse_attention_ref(q, k, v, mask, rb, is_causal=True,
                                               sm_scale=SHAPE.head_dim ** -0.5, heads=heads)
        for z, h in heads:
            assert np.abs(o[z, h] - ref[z, h]).max() <= 2e-2, (layer, h)
        st = model.last_stats[layer]
        nb = -(-S // rb)
        assert abs(st["block_density"] - bl.counts.sum() / (H * nb * (nb + 1) / 2)) < 1e-6


def test_r0_matches_dense_sdpa(model):
    # every causal block routed: the block-list model is the dense causal model
    S = 1536
    g = torch.Generator().manual_seed(7)
    ids = torch.randint(0, SHAPE.vocab, (1, S), generator=g).to(DEV)
    model.r = 0
    seen = _capture(model)
    try:
        sparse = model(ids, collect_stats=True)
        model.attention = "sdpa"
        dense = model(ids)
    finally:
        model.attention = "block_list"
        del model.core_attention
    assert all(st["block_density"] == 1.0 for st in model.last_stats)
    # per layer: the block-list output on that layer's q / k / v against the
    # float64 oracle (GQA) and against SDPA with repeated key / value heads
    for layer, q, k, v, o in seen[:2]:
        tq, tk, tv = (torch.from_numpy(x).to(DEV).to(torch.bfloat16) for x in (q, k, v))
        model.attention = "sdpa"
        try:
            d = model.core_attention(layer, tq, tk, tv).float().cpu().numpy()
        finally:
            model.attention = "block_list"
        assert np.abs(o - d).max() <= 2e-2, layer
        ref = oa.masked_attention(q[:, :4], np.repeat(k, 4, axis=1)[:, :4], np.repeat(v, 4, axis=1)[:, :4],
                                  np.tril(np.ones((1, 4, S, S), dtype=bool)))[0]
        assert np.abs(o[:, :4] - ref).max() <= 2e-2, layer
    # and end to end: two layers' hidden states agree to bf16 rounding
    err = (sparse.float() - dense.float()).abs().max().item()
    assert err <= 5e-2 * max(1.0, dense.float().abs().max().item()), err
