"""Empty problems on every public entry point: zero batch or zero sequence
length return correctly shaped empty (or untouched) outputs without a
launch, as the reference's host code does where it guards empty counts
(src/ultrametric/block_list.py:251, :267, :318)."""

import pytest
import torch

from ultrametric import (block_list_attention, build_block_lists, build_transposed_block_lists,
                         pack_routing_codes, route_block_vote, sequence_page_codes, ternary_quantize_pack,
                         ternary_ultrametric_attention, ultrametric_decode, ultrametric_decode_packed,
                         ultrametric_decode_seq_codes)

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("Z,H,N", [(0, 2, 256), (1, 2, 0)])
def test_prefill_and_backward_empty(Z, H, N):
    rb, D = 64, 64
    NB = -(-N // rb)
    for sync_free in (True, False):
        r = torch.zeros(Z, H, NB, 2, dtype=torch.int32, device=DEV)
        bl = build_block_lists(r, 1, is_causal=True, arity=2 if sync_free else None)
        assert bl.counts.shape == (Z, H, NB)
        q = torch.randn(Z, H, N, D, device=DEV, dtype=torch.bfloat16, requires_grad=True)
        k = torch.randn(Z, H, N, D, device=DEV, dtype=torch.bfloat16, requires_grad=True)
        v = torch.randn(Z, H, N, D, device=DEV, dtype=torch.bfloat16, requires_grad=True)
        out = block_list_attention(q, k, v, bl, route_block=rb, is_causal=True)
        assert out.shape == (Z, H, N, D)
        out.float().sum().backward()
        assert q.grad.shape == q.shape and k.grad.shape == k.shape and v.grad.shape == v.shape
    t = build_transposed_block_lists(bl)
    assert t.counts.numel() == Z * H * NB


def test_zero_heads_is_an_error():
    # k, v need at least one head to group the query heads over
    q = torch.randn(1, 0, 128, 64, device=DEV, dtype=torch.bfloat16)
    bl = build_block_lists(torch.zeros(1, 0, 2, 1, dtype=torch.int32, device=DEV), 1, arity=2)
    with pytest.raises(ValueError, match="share shape"):
        block_list_attention(q, q, q, bl, route_block=64)


def test_route_vote_empty():
    a = torch.randn(0, 2, 256, 3, 2, device=DEV)
    assert route_block_vote(a, 2, 64).shape == (0, 2, 4, 2)


@pytest.mark.parametrize("B", [0])
def test_decode_empty_batch(B):
    H, Hkv, D, page, pages, TD = 8, 2, 64, 16, 4, 3
    q = torch.randn(B, H, D, device=DEV, dtype=torch.bfloat16)
    kc = torch.randn(pages, Hkv, page, D, device=DEV, dtype=torch.bfloat16)
    vc = torch.randn_like(kc)
    bt = torch.zeros(B, 2, dtype=torch.int32, device=DEV)
    ctx = torch.zeros(B, dtype=torch.int32, device=DEV)
    r = torch.zeros(pages, H, TD, dtype=torch.int32, device=DEV)
    qr = torch.zeros(B, H, TD, dtype=torch.int32, device=DEV)
    assert ultrametric_decode(q, kc, vc, bt, ctx, r, qr, 2).shape == (B, H, D)
    pc, qc = pack_routing_codes(r, 2), pack_routing_codes(qr, 2)
    assert qc.shape == (B, H)
    assert ultrametric_decode_packed(q, kc, vc, bt, ctx, pc, qc, TD, 2, req_depth=2).shape == (B, H, D)
    sc = sequence_page_codes(pc, bt, bits=8)
    assert ultrametric_decode_seq_codes(q, kc, vc, bt, ctx, sc, qc, TD, 2, req_depth=2).shape == (B, H, D)


def test_ternary_empty():
    x = torch.randn(0, 3, 64, device=DEV)
    packed, scale = ternary_quantize_pack(x)
    assert packed.shape == (0, 3, 4) and scale.shape == (0, 3)
    q = torch.randn(0, 2, 256, 64, device=DEV, dtype=torch.float16)
    kp = torch.zeros(0, 2, 256, 4, dtype=torch.int32, device=DEV)
    ks = torch.ones(0, 2, 256, device=DEV)
    r = torch.zeros(0, 2, 2, 2, dtype=torch.int32, device=DEV)
    assert ternary_ultrametric_attention(q, kp, kp, ks, ks, r).shape == q.shape
