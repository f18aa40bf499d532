"""Host model of a paged KV cache for the GPU tests: each row's token history
(K / V rows and routing levels) and the physical pages, block tables and
page router (first token's levels) that the decode oracle
(oracle/decode.py) reads, rebuilt from that history alone."""

import numpy as np

TD, P_ARITY, BPL = 4, 4, 2


class HostModel:
    """Per-row token history: K / V rows (float32) and routing levels (H, TD)."""

    def __init__(self, B, Hkv, H, D):
        self.k = [np.zeros((Hkv, 0, D), np.float32) for _ in range(B)]
        self.v = [np.zeros((Hkv, 0, D), np.float32) for _ in range(B)]
        self.lv = [np.zeros((H, 0, TD), np.int64) for _ in range(B)]

    def add(self, b, k, v, lv):
        self.k[b] = np.concatenate([self.k[b], k], 1)
        self.v[b] = np.concatenate([self.v[b], v], 1)
        self.lv[b] = np.concatenate([self.lv[b], lv], 1)

    def lens(self):
        return [x.shape[1] for x in self.k]


def oracle_inputs(cache, host, layer_pages, H):
    """Physical K / V pages, block tables and the page router rebuilt from the history."""
    B = len(host.k)
    PS, P = cache.page_size, cache.num_pages
    Hkv, D = cache.kv_heads, cache.head_dim
    kc = np.zeros((P, Hkv, PS, D), np.float32)
    vc = np.zeros_like(kc)
    router = np.zeros((P, H, TD), np.int32)
    bt = np.zeros((B, cache.max_pages), np.int32)
    for b in range(B):
        n = host.k[b].shape[1]
        pages = layer_pages[b]
        bt[b, :len(pages)] = pages
        for l in range(-(-n // PS)):
            t0, t1 = l * PS, min(n, (l + 1) * PS)
            kc[pages[l], :, :t1 - t0] = host.k[b][:, t0:t1]
            vc[pages[l], :, :t1 - t0] = host.v[b][:, t0:t1]
            router[pages[l]] = host.lv[b][:, t0]
    return kc, vc, bt, router
