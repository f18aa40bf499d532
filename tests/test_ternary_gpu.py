"""GPU parity of the ternary packed-K/V path against oracle/ternary.py:
quantize + pack bit-exact (codes, words, scales), and the causal block-sparse
prefill over packed K / V (fp16; <= 5e-3 of the output scale) across head
dims, ragged N, local windows, routing depths, GQA and the shift regions."""

import math

import numpy as np
import pytest
import torch

from oracle import ternary as ot
from ultrametric import pack_ternary, ternary_quantize_pack, ternary_ultrametric_attention
from ultrametric.ternary import unpack_ternary

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("D", [16, 64, 128, 96])
def test_quantize_pack_matches_oracle(dtype, D):
    g = torch.Generator().manual_seed(D)
    x = torch.randn(3, 7, D, generator=g).to(dtype)
    packed, scale = ternary_quantize_pack(x.to(DEV))
    xf = x.double().numpy()
    t, gamma = ot.ternary_quantize(xf)
    assert np.allclose(scale.cpu().numpy(), gamma[..., 0], rtol=1e-6)
    # codes agree except at values within rounding of the threshold
    near = np.abs(np.abs(xf) - 0.5 * gamma) < 1e-5 * gamma
    got = ot.unpack_ternary(packed.cpu().numpy(), D)
    assert np.array_equal(got[~near], t[~near])
    if not near.any():
        assert np.array_equal(packed.cpu().numpy(), ot.pack_ternary(t))


def test_exact_pack_and_unpack():
    rng = np.random.default_rng(1)
    t = rng.integers(-1, 2, (5, 4, 128)).astype(np.float32)
    packed = pack_ternary(torch.from_numpy(t).to(DEV))
    assert np.array_equal(packed.cpu().numpy(), ot.pack_ternary(t))
    back = unpack_ternary(packed, t.shape)
    assert np.array_equal(back.cpu().numpy(), t)


def make(Z, H, Hkv, N, D, seed, TD=3, p=2, scale_dtype=torch.float32):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(Z, H, N, D, generator=g).half()
    kt = torch.randint(-1, 2, (Z, Hkv, N, D), generator=g).float()
    vt = torch.randint(-1, 2, (Z, Hkv, N, D), generator=g).float()
    ks = (torch.rand(Z, Hkv, N, generator=g) * 0.6 + 0.1).to(scale_dtype)
    vs = (torch.rand(Z, Hkv, N, generator=g) * 1.5 + 0.2).to(scale_dtype)
    router = torch.randint(0, p, (Z, H, math.ceil(N / 128), TD), generator=g, dtype=torch.int32)
    return q, ot.pack_ternary(kt.numpy()), ot.pack_ternary(vt.numpy()), ks, vs, router


def oracle(q, kp, vp, ks, vs, router, group, **kw):
    rep = lambda a: np.repeat(a, group, axis=1)  # noqa: E731
    return ot.ternary_attention_ref(q.float().numpy(), rep(kp), rep(vp), rep(ks.float().numpy()),
                                    rep(vs.float().numpy()), router.numpy(), **kw)


@pytest.mark.parametrize("Z,H,Hkv,N,D", [(1, 2, 2, 300, 64), (2, 4, 2, 1000, 128), (1, 2, 1, 640, 32),
                                         (1, 3, 3, 129, 128)])
@pytest.mark.parametrize("kw", [dict(local_window=128, req_depth=2), dict(local_window=256, req_depth=1),
                                dict(local_window=0, req_depth=3), dict(local_window=128, req_depth=0),
                                dict(local_window=128, req_depth=2, shift_size=77)])
def test_ternary_attention_matches_oracle(Z, H, Hkv, N, D, kw):
    q, kp, vp, ks, vs, router = make(Z, H, Hkv, N, D, seed=N + D + H)
    out = ternary_ultrametric_attention(q.to(DEV), torch.from_numpy(kp).to(DEV), torch.from_numpy(vp).to(DEV),
                                        ks.to(DEV), vs.to(DEV), router.to(DEV), **kw)
    ref = oracle(q, kp, vp, ks, vs, router, H // Hkv, **kw)
    err = np.abs(out.float().cpu().numpy() - ref).max()
    assert err <= 5e-3 * max(1.0, np.abs(ref).max()), err


def test_ternary_attention_fp16_scales_and_short_router():
    # fp16 scales, and a router with fewer blocks than N needs (padded with zeros)
    q, kp, vp, ks, vs, router = make(1, 2, 2, 700, 128, seed=9, scale_dtype=torch.float16)
    short = router[:, :, :3]
    out = ternary_ultrametric_attention(q.to(DEV), torch.from_numpy(kp).to(DEV), torch.from_numpy(vp).to(DEV),
                                        ks.to(DEV), vs.to(DEV), short.to(DEV), req_depth=2)
    ref = oracle(q, kp, vp, ks, vs, short, 1, req_depth=2)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 5e-3 * max(1.0, np.abs(ref).max())


def test_quantized_kv_round_trip_through_attention():
    # K / V quantized on the GPU, attention checked against the oracle on the same codes
    g = torch.Generator().manual_seed(3)
    Z, H, N, D = 1, 2, 512, 128
    q = torch.randn(Z, H, N, D, generator=g).half().to(DEV)
    k = torch.randn(Z, H, N, D, generator=g).to(DEV)
    v = torch.randn(Z, H, N, D, generator=g).to(DEV)
    kp, ks = ternary_quantize_pack(k)
    vp, vs = ternary_quantize_pack(v)
    router = torch.randint(0, 2, (Z, H, N // 128, 3), generator=g, dtype=torch.int32)
    out = ternary_ultrametric_attention(q, kp, vp, ks, vs, router.to(DEV))
    ref = ot.ternary_attention_ref(q.float().cpu().numpy(), kp.cpu().numpy(), vp.cpu().numpy(), ks.cpu().numpy(),
                                   vs.cpu().numpy(), router.numpy())
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 5e-3 * max(1.0, np.abs(ref).max())


def test_ids_above_the_arity_match_level_by_level():
    # the reference compares routing ids level by level whatever p is: ids >= p
    # (here 0..3 with the default p = 2) must not alias into extra matches
    q, kp, vp, ks, vs, router = make(1, 2, 2, 1024, 64, seed=21, TD=3, p=4)
    out = ternary_ultrametric_attention(q.to(DEV), torch.from_numpy(kp).to(DEV), torch.from_numpy(vp).to(DEV),
                                        ks.to(DEV), vs.to(DEV), router.to(DEV), req_depth=2)
    ref = oracle(q, kp, vp, ks, vs, router, 1, req_depth=2)
    assert np.abs(out.float().cpu().numpy() - ref).max() <= 5e-3 * max(1.0, np.abs(ref).max())
    from ultrametric.ternary import ternary_block_lists
    bl = ternary_block_lists(router.to(DEV), 2, 128)
    sel = ot.block_selection(router.numpy(), 2, 128, router.shape[2])
    assert int(bl.counts.sum()) == int(sel.sum())
