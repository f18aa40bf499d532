"""CPU checks of the router's straight-through soft bias (surgery.py:566-588,
topology.py:456-485): ``expected_block_distance``, the block means of
``block_list_prefill`` and ``ste_soft_block_bias``, each against a
brute-force restatement with explicit per-pair, per-level loops in float64
(values and autograd gradients)."""

import itertools
import math

import torch

from ultrametric.surgery import _block_mean, expected_block_distance, ste_soft_block_bias


def _probs(shape, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.softmax(torch.randn(*shape, generator=g, dtype=torch.float64), -1)


def _loop_distance(a):
    """dist[b, h, i, j] = L - sum_l min_{l' <= l} m_l'(i, j), m_l(i, j) = sum_p a[i, l, p] a[j, l, p];
    with the tie-breaking residual 0.05 * 2^(l - (L - 1)) * (m_l - m_l.detach()) per level."""
    B, H, NB, L, P = a.shape
    rows = []
    for b, h in itertools.product(range(B), range(H)):
        grid = []
        for i in range(NB):
            row = []
            for j in range(NB):
                run = None
                total = 0.0
                for l in range(L):
                    m = (a[b, h, i, l] * a[b, h, j, l]).sum()
                    run = m if run is None else torch.minimum(run, m)
                    w = 0.05 * 2.0 ** (l - (L - 1))
                    total = total + run + (w * m - (w * m).detach())
                row.append(L - total)
            grid.append(torch.stack(row))
        rows.append(torch.stack(grid))
    return torch.stack(rows).view(B, H, NB, NB)


def test_expected_block_distance_values_and_gradient():
    a = _probs((1, 2, 5, 3, 4), seed=1).requires_grad_(True)
    a2 = a.detach().clone().requires_grad_(True)
    d = expected_block_distance(a, p=4)
    ref = _loop_distance(a2)
    assert torch.allclose(d, ref, atol=1e-12, rtol=0)
    w = _probs((1, 2, 5, 5), seed=2)
    (d * w).sum().backward()
    (ref * w).sum().backward()
    assert torch.allclose(a.grad, a2.grad, atol=1e-12, rtol=0)
    # the diagonal: a block shares every level with itself up to its own agreement mass
    assert torch.all(d.detach().diagonal(dim1=-2, dim2=-1) < 3.0)


def test_expected_block_distance_one_hot_counts_unshared_levels():
    # one-hot assignments: the distance is the number of levels after the first disagreement
    idx = torch.tensor([[0, 1, 2], [0, 1, 3], [0, 2, 2], [1, 1, 2]])
    a = torch.nn.functional.one_hot(idx, 4).to(torch.float64).view(1, 1, 4, 3, 4)
    d = expected_block_distance(a, p=4)[0, 0]
    for i, j in itertools.product(range(4), range(4)):
        shared = 0
        for l in range(3):
            if idx[i, l] != idx[j, l]:
                break
            shared += 1
        assert d[i, j].item() == 3 - shared


def test_block_mean_of_valid_tokens():
    S, RB = 13, 4
    a = _probs((1, 2, S, 2, 3), seed=3)
    got = _block_mean(a, S, RB)
    assert got.shape == (1, 2, 4, 2, 3)
    for blk in range(4):
        lo, hi = blk * RB, min(S, (blk + 1) * RB)
        assert torch.allclose(got[:, :, blk], a[:, :, lo:hi].mean(dim=2), atol=1e-14, rtol=0)


def test_ste_soft_block_bias_is_zero_with_the_gathered_gradient():
    L, r, P, NB = 4, 2, 4, 6
    a = _probs((1, 2, NB, L, P), seed=4).requires_grad_(True)
    a2 = a.detach().clone().requires_grad_(True)
    g = torch.Generator().manual_seed(5)
    lists = torch.randint(0, NB, (1, 2, NB, 3), generator=g, dtype=torch.int32)
    lists[..., 2] = -1                      # clamped into [0, NB), as the reference's safe_lists
    bias = ste_soft_block_bias(a, lists, r, P)
    assert bias.shape == (1, 2, NB, 3) and torch.all(bias == 0)
    up = _probs((1, 2, NB, 3), seed=6)
    (bias * up).sum().backward()
    logits = ((L - r) - _loop_distance(a2)) / 0.5
    gathered = torch.gather(logits, -1, lists.clamp(0, NB - 1).long())
    (gathered * up).sum().backward()
    # the bias is computed in float32, as the reference's blk_assign.float()
    assert torch.allclose(a.grad, a2.grad, atol=1e-5, rtol=1e-5)
    assert a.grad.abs().sum() > 0
