"""Rows with more listed blocks than one LDS list segment (256 entries) on the
MFMA paths: forward (route block 32 and 64), backward dQ / dK / dV, and the
ternary prefill. Dense causal lists make the block-sparse result equal dense
causal attention, so fp32 torch attention on the GPU is the reference
(floating-point kernels; tolerances as the other bf16 / fp16 tests)."""

import pytest
import torch
import torch.nn.functional as F

from oracle import ternary as ot
from ultrametric import block_list_attention, build_block_lists, ternary_ultrametric_attention

pytestmark = pytest.mark.gpu
DEV = "cuda"


def dense_lists(Z, H, N, rb):
    r = torch.zeros(Z, H, -(-N // rb), 1, dtype=torch.int32, device=DEV)
    return build_block_lists(r, 0, is_causal=True, arity=2)


def ref_attention(q, k, v):
    group = q.shape[1] // k.shape[1]
    kk = k.float().repeat_interleave(group, 1)
    vv = v.float().repeat_interleave(group, 1)
    return F.scaled_dot_product_attention(q.float(), kk, vv, is_causal=True)


@pytest.mark.parametrize("N,rb,D,dtype", [(16384, 32, 64, torch.float16), (20000, 64, 128, torch.bfloat16)])
def test_forward_rows_longer_than_a_segment(N, rb, D, dtype):
    g = torch.Generator(device=DEV).manual_seed(N)
    Z, H, Hkv = 1, 2, 1
    q = torch.randn(Z, H, N, D, generator=g, device=DEV).to(dtype)
    k, v = (torch.randn(Z, Hkv, N, D, generator=g, device=DEV).to(dtype) for _ in range(2))
    bl = dense_lists(Z, H, N, rb)
    assert bl.counts.max().item() > 256
    out = block_list_attention(q, k, v, bl, route_block=rb, is_causal=True)
    ref = ref_attention(q, k, v)
    assert (out.float() - ref).abs().max().item() <= 2e-2


def test_backward_rows_longer_than_a_segment():
    g = torch.Generator(device=DEV).manual_seed(7)
    Z, H, Hkv, N, D, rb = 1, 2, 1, 9600, 64, 32
    q0 = torch.randn(Z, H, N, D, generator=g, device=DEV).half()
    k0, v0 = (torch.randn(Z, Hkv, N, D, generator=g, device=DEV).half() for _ in range(2))
    do = torch.randn(Z, H, N, D, generator=g, device=DEV).half()
    bl = dense_lists(Z, H, N, rb)
    assert bl.counts.max().item() > 256
    q, k, v = (t.clone().requires_grad_(True) for t in (q0, k0, v0))
    block_list_attention(q, k, v, bl, route_block=rb, is_causal=True).backward(do)
    qf, kf, vf = (t.float().clone().requires_grad_(True) for t in (q0, k0, v0))
    ref_attention(qf, kf, vf).backward(do.float())
    for got, want, name in ((q.grad, qf.grad, "q"), (k.grad, kf.grad, "k"), (v.grad, vf.grad, "v")):
        scale = max(1.0, want.abs().max().item())
        assert (got.float() - want).abs().max().item() <= 2e-2 * scale, name


def test_ternary_rows_longer_than_a_segment():
    # req_depth 0: every causal block is visited (NB = 258 > 256 entries on the last rows)
    g = torch.Generator().manual_seed(3)
    Z, H, N, D = 1, 1, 33024, 64
    q = torch.randn(Z, H, N, D, generator=g).half()
    kt = torch.randint(-1, 2, (Z, H, N, D), generator=g).float()
    vt = torch.randint(-1, 2, (Z, H, N, D), generator=g).float()
    ks = torch.rand(Z, H, N, generator=g) * 0.5 + 0.1
    vs = torch.rand(Z, H, N, generator=g) + 0.2
    router = torch.zeros(Z, H, N // 128, 3, dtype=torch.int32)
    kp, vp = torch.from_numpy(ot.pack_ternary(kt.numpy())), torch.from_numpy(ot.pack_ternary(vt.numpy()))
    out = ternary_ultrametric_attention(q.to(DEV), kp.to(DEV), vp.to(DEV), ks.to(DEV), vs.to(DEV), router.to(DEV),
                                        req_depth=0)
    ref = ref_attention(q.to(DEV), (kt * ks[..., None]).to(DEV), (vt * vs[..., None]).to(DEV))
    assert (out.float() - ref).abs().max().item() <= 5e-3 * max(1.0, ref.abs().max().item())
