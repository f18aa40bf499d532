"""Pins the decode oracle (oracle/decode.py) on the CPU.

  * req_depth = 0 without sink/local equals dense paged attention computed by
    a pure-Python token loop (benchmarks/benchmark_serving.py:11-73 with every
    page selected), on shuffled block tables and ragged context lengths;
  * a pure-Python per-page selection loop (prefix match on the physical
    page's routing vector, sink page 0, last local pages) fed to the same
    token loop, at tree depths {1, 3, 5, 6, 7, 10} as in
    tests/test_llama_surgery.py:355-398;
  * ctx = 0 gives zeros; a one-token sequence returns that token's V row;
  * GQA grouping equals the H_kv = H call on repeated caches.
"""

import math

import numpy as np
import pytest

from oracle import decode as od


def make(B=3, H=4, Hkv=4, D=8, page=4, pages=12, TD=3, p=2, seed=0, lens=(13, 7, 1)):
    rng = np.random.default_rng(seed)
    q = rng.standard_normal((B, H, D))
    kc = rng.standard_normal((pages, Hkv, page, D))
    vc = rng.standard_normal((pages, Hkv, page, D))
    max_pages = max(-(-l // page) for l in lens)
    tables = np.stack([rng.permutation(pages)[:max_pages] for _ in range(B)]).astype(np.int32)
    ctx = np.array(lens, dtype=np.int32)
    router = rng.integers(0, p, size=(pages, H, TD)).astype(np.int32)
    qr = rng.integers(0, p, size=(B, H, TD)).astype(np.int32)
    return q, kc, vc, tables, ctx, router, qr


def selected_loop(tables, ctx, router, qr, b, h, r, local, sink, page):
    n = -(-int(ctx[b]) // page)
    sel = []
    for l in range(n):
        ph = int(tables[b][l])
        m = all(int(router[ph][h][i]) == int(qr[b][h][i]) for i in range(r))
        if sink and l == 0:
            m = True
        if local > 0 and l >= n - local:
            m = True
        if m:
            sel.append(l)
    return sel


def loop_attend(q, kc, vc, tables, ctx, b, h, pages_sel, page, group):
    scores, rows = [], []
    D = q.shape[-1]
    for l in pages_sel:
        ph = int(tables[b][l])
        for t in range(min(page, int(ctx[b]) - l * page)):
            scores.append(sum(float(a) * float(c) for a, c in zip(q[b][h], kc[ph][h // group][t])) / math.sqrt(D))
            rows.append(vc[ph][h // group][t])
    if not scores:
        return [0.0] * D
    mx = max(scores)
    w = [math.exp(s - mx) for s in scores]
    return [sum(wi * float(r[d]) for wi, r in zip(w, rows)) / sum(w) for d in range(D)]


def test_depth_zero_is_dense_paged():
    q, kc, vc, tables, ctx, router, qr = make()
    ref = od.decode_reference(q, kc, vc, tables, ctx, router, qr, 0)
    dense = od.dense_paged_loop(q, kc, vc, tables, ctx)
    assert np.allclose(ref, dense, atol=1e-12)


@pytest.mark.parametrize("TD", [1, 3, 5, 6, 7, 10])
@pytest.mark.parametrize("local,sink", [(1, True), (0, False), (2, False)])
def test_selection_against_loop(TD, local, sink):
    q, kc, vc, tables, ctx, router, qr = make(TD=TD, seed=TD, lens=(40, 35, 9))
    r = min(3, TD)
    ref = od.decode_reference(q, kc, vc, tables, ctx, router, qr, r, local_blocks=local, sink_block=sink)
    for b in range(3):
        for h in range(4):
            sel = selected_loop(tables, ctx, router, qr, b, h, r, local, sink, 4)
            exp = loop_attend(q, kc, vc, tables, ctx, b, h, sel, 4, 1)
            assert np.allclose(ref[b, h], exp, atol=1e-12)


def test_ctx_zero_and_single_token():
    q, kc, vc, tables, ctx, router, qr = make(lens=(0, 1, 5))
    ref = od.decode_reference(q, kc, vc, tables, ctx, router, qr, 0)
    assert np.all(ref[0] == 0)
    assert np.allclose(ref[1], vc[tables[1, 0], :, 0])
    # req_depth above TD clamps to TD; negative clamps to 0 (kernel_decode.py:141)
    a = od.decode_reference(q, kc, vc, tables, ctx, router, qr, 99, sink_block=True)
    b = od.decode_reference(q, kc, vc, tables, ctx, router, qr, 3, sink_block=True)
    assert np.array_equal(a, b)
    assert np.array_equal(od.decode_reference(q, kc, vc, tables, ctx, router, qr, -4),
                          od.decode_reference(q, kc, vc, tables, ctx, router, qr, 0))


def test_gqa_equals_repeat():
    q, kc, vc, tables, ctx, router, qr = make(H=4, Hkv=2, seed=5, lens=(17, 30, 3))
    a = od.decode_reference(q, kc, vc, tables, ctx, router, qr, 2, local_blocks=1, sink_block=True)
    b = od.decode_reference(q, np.repeat(kc, 2, axis=1), np.repeat(vc, 2, axis=1), tables, ctx, router,
                            qr, 2, local_blocks=1, sink_block=True)
    assert np.array_equal(a, b)


def test_routed_bytes_counts_group_union_once():
    q, kc, vc, tables, ctx, router, qr = make(H=4, Hkv=2, seed=6, lens=(17, 30, 3))
    nbytes, pages = od.routed_page_bytes(tables, ctx, router, qr, 2, 4, 8, 2, 0)
    # req_depth 0: every page of every sequence, once per kv head
    assert pages == 2 * sum(-(-int(c) // 4) for c in ctx)
    assert nbytes == 2 * int(ctx.sum()) * 8 * 2 * 2


@pytest.mark.parametrize("TD,bpl", [(1, 1), (4, 1), (5, 2), (8, 4), (16, 2), (2, 16), (32, 1), (3, 10)])
def test_pack_codes_prefix_equality(TD, bpl):
    # brute force: for every depth r the masked code comparison equals the
    # level-by-level comparison, and the packing is invertible
    rng = np.random.default_rng(TD * 100 + bpl)
    base = 1 << bpl
    hi = min(base, 3)                     # few distinct values -> many prefix matches
    a = rng.integers(0, hi, (300, TD))
    b = a.copy()
    cut = rng.integers(0, TD + 1, 300)
    for i in range(300):                  # b agrees with a on a random prefix, then random
        b[i, cut[i]:] = rng.integers(0, base, TD - cut[i])
    a[-1] = base - 1                      # extreme values survive packing
    b[-1] = base - 1
    ca, cb = od.pack_codes(a, bpl), od.pack_codes(b, bpl)
    for r in range(TD + 2):
        m = od.prefix_mask(TD, bpl, r)
        rr = min(r, TD)
        want = (a[:, :rr] == b[:, :rr]).all(-1)
        assert np.array_equal(((ca ^ cb) & m) == 0, want), r
    for lev in range(TD):
        shift = bpl * (TD - 1 - lev)
        got = (ca.astype(np.uint64) >> np.uint64(shift)) & np.uint64(base - 1)
        assert np.array_equal(got, a[:, lev])


def test_pack_codes_rejects_overflowing_levels():
    with pytest.raises(AssertionError):
        od.pack_codes(np.array([[4]]), 2)
    with pytest.raises(AssertionError):
        od.pack_codes(np.zeros((1, 9)), 4)
