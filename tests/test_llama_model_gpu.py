"""GPU parity of the config-5 model harness (ultrametric.llama_model) on two
decoder layers at reduced N: the attention each layer computes through
block_list_prefill (route-block vote, sync-free lists, GQA prefill) is checked
against the oracle on the q / k / v / routing scores that layer actually
produced (oracle/surgery.py majority vote -> oracle/blocks.py lists ->
oracle/attention.py masked-dense float64, bf16 tolerance 2e-2), and the lists
against the oracle's bit for bit. With r = 0 (every causal block) the same
model must agree with its dense SDPA condition (the reference benchmark's
``dense_sdpa`` baseline, experiments/bench_surgery_prefill.py:146-178).

The serving path: a prompt prefilled into a paged cache, then single-token
decode steps (the paged replacement of the eager decode masks of
src/llama_surgery/surgery.py:880-955), each layer's decode output against the
float64 decode oracle (oracle/decode.py) on that layer's own history; with
every page selected (r = 0) the decode step's hidden state equals the last
position of a dense forward over prompt + token."""

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


def test_paged_prefill_and_decode_steps_match_oracle(model):
    # prompt through the model into a paged cache, then single-token decode steps:
    # per layer and step, the decode output against the float64 oracle on that
    # layer's history (prefill K / V as the layer produced them, then each step's)
    from oracle import decode as od
    from paged_host import HostModel, oracle_inputs

    model.r = 2
    B, S, steps = 2, 200, 4
    H, Hkv, D, lv_n = SHAPE.heads, SHAPE.kv_heads, SHAPE.head_dim, model.levels
    g = torch.Generator().manual_seed(12)
    ids = torch.randint(0, SHAPE.vocab, (B, S), generator=g).to(DEV)
    cache = model.new_cache(max_seqs=B, max_tokens=S + steps, layers=SHAPE.layers)
    seen = _capture(model)
    try:
        model.prefill(cache, ids)
    finally:
        del model.core_attention
    hosts = [HostModel(B, Hkv, H, D) for _ in range(SHAPE.layers)]
    for layer, q, k, v, o in seen:
        lv = model.routing_scores(layer, B, S)[..., :lv_n, :].float().argmax(-1).cpu().numpy()
        for b in range(B):
            hosts[layer].add(b, k[b], v[b], lv[b])
    assert cache.lengths == [S] * B
    recorded = []
    dec, wr = cache.decode, cache.write

    def rec_write(layer, k_new, v_new, token_codes=None, n_new=None):
        recorded.append(("w", layer, k_new.float().cpu().numpy()[:, :, 0], v_new.float().cpu().numpy()[:, :, 0]))
        return wr(layer, k_new, v_new, token_codes, n_new)

    def rec_decode(layer, q, q_codes, req_depth, **kw):
        out = dec(layer, q, q_codes, req_depth, **kw)
        recorded.append(("d", layer, q.float().cpu().numpy(), out.float().cpu().numpy(), req_depth, kw))
        return out

    cache.write, cache.decode = rec_write, rec_decode
    try:
        for step in range(steps):
            recorded.clear()
            cache.reserve(1, rows=range(B))
            sc = torch.randn(SHAPE.layers, B, H, lv_n, model.p, generator=g).to(torch.bfloat16)
            hid = model.decode_step(cache, torch.randint(0, SHAPE.vocab, (B,), generator=g).to(DEV), sc.to(DEV))
            assert hid.shape == (B, SHAPE.hidden) and torch.isfinite(hid).all()
            lvs = sc.float().argmax(-1).numpy()                      # (layers, B, H, levels)
            for i in range(0, len(recorded), 2):
                _, layer, kn, vn = recorded[i]
                _, layer2, q, out, r, kw = recorded[i + 1]
                assert layer == layer2
                for b in range(B):
                    hosts[layer].add(b, kn[b][:, None], vn[b][:, None], lvs[layer, b][:, None])
                kc, vc, bt, router = oracle_inputs(cache, hosts[layer], cache._pages, H)
                ref = od.decode_reference(q, kc, vc, bt, np.array(hosts[layer].lens()), router,
                                          lvs[layer].astype(np.int32), r, local_blocks=kw["local_blocks"],
                                          sink_block=kw["sink_block"])
                assert np.abs(out - ref).max() <= 2e-2, (step, layer)
    finally:
        del cache.write, cache.decode
    assert cache.lengths == [S + steps] * B
    assert cache.context_lens[:B].cpu().tolist() == [S + steps] * B


def test_decode_step_all_pages_matches_full_forward(model):
    # r = 0 selects every page: the decode step's hidden state for the new
    # token equals the last position of a full dense (SDPA) forward over the
    # prompt plus that token (RoPE position, cache contents, GQA all agree)
    model.r = 0
    B, S = 2, 130
    g = torch.Generator().manual_seed(13)
    ids = torch.randint(0, SHAPE.vocab, (B, S + 1), generator=g).to(DEV)
    cache = model.new_cache(max_seqs=B, max_tokens=S + 1, layers=SHAPE.layers)
    model.prefill(cache, ids[:, :S])
    cache.reserve(1, rows=range(B))
    sc = torch.randn(SHAPE.layers, B, SHAPE.heads, model.levels, model.p, generator=g).to(torch.bfloat16).to(DEV)
    hid = model.decode_step(cache, ids[:, S], sc).float()
    model.attention = "sdpa"
    try:
        full = model(ids)[:, -1].float()
    finally:
        model.attention = "block_list"
    err = (hid - full).abs().max().item()
    assert err <= 5e-2 * max(1.0, full.abs().max().item()), err
