#!/usr/bin/env python3
"""Benchmark of the block-sparse attention hot path on one MI355X.

Headline (BASELINE.json `metric`, config 2): block-sparse prefill TFLOP/s on
computed tiles at N = 8192 — bf16, H = 32, D = 128, route block 128, causal,
tree-routed lists (p = 4 depth 3, LCA depth >= 2, + diagonal + sink). One
step = sync-free block-list build + prefill forward over those lists, inputs
resident in HBM. `value` = FLOP_alg / step time, FLOP_alg = 4 * D * 128^2 *
sum(counts) (every listed 128x128 tile counted in full).

Also reported: the prefill kernel alone (HIP events around back-to-back
launches on its stream; `roofline` is built from it), the list build alone,
the same step in one launch (routed_block_attention with the branch arity:
the build runs inside the prefill kernel),
sparse paged decode on config 4 (GB/s of routed KV bytes), the backward on
config 2 (dQ, dK, dV; algorithmic TFLOP/s = 2.5 x the forward's), the
ternary packed-K/V prefill over config 2's lists, config 5 end to end (a
32-layer Llama-3.1-8B-shaped decoder, 16384-token prefill, whole forward and
attention share, block-list attention at r = 2, 3, 4 against dense SDPA), and CPU baselines on the host
cores (below).
Untimed steps run back to back for --spinup-ms before the warmup steps, so
that the timed steps run at the GPU's steady clocks. The config-3 density
sweep runs by default (--no-sweep skips it). CPU baselines (--no-cpu skips
them, --cpu-quick keeps only config 2's): the fp32 masked-dense reference on
the host cores for configs 1, 2, 3 (N <= 8192 all heads; N = 32768 one head
x 32) and one config-5 layer (two heads x 16), and the float64 decode oracle
over all 64 x 32 (sequence, head) pairs of config 4; each a median of 3 runs
after a warm-up, recorded with the CPU model, cores and torch threads.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--spinup-ms MS] [--no-cpu] [--cpu-quick]
                       [--no-decode] [--no-backward] [--no-ternary] [--no-c5] [--no-sweep]
Only one GPU is supported: --gpus N > 1 exits with a message.
"""

import argparse
import json
import math
import os
import platform
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "sparse-ai_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PROFILES = os.path.join(ROOT, "profiles")


def profiled_traffic(name):
    """HBM bytes per launch recorded in profiles/<name> (rocprofv3 FETCH_SIZE / WRITE_SIZE
    passes scaled by a 256 MiB copy; the file gives the commands), or None."""
    path = os.path.join(PROFILES, name)
    if not os.path.exists(path):
        return None
    with open(path) as fh:
        for line in fh:
            if line.startswith("traffic_bytes_per_launch:"):
                return int(line.split(":", 1)[1])
    return None


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--spinup-ms", type=float, default=200.0,
                    help="untimed steps run back to back for this long before the warmup steps, so that "
                         "the timed steps run at the GPU's steady clocks")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--cpu-quick", action="store_true",
                    help="CPU baseline of config 2 only (the headline), not the per-config records")
    ap.add_argument("--no-decode", action="store_true", help="skip the decode measurement")
    ap.add_argument("--no-backward", action="store_true", help="skip the backward measurement")
    ap.add_argument("--no-ternary", action="store_true", help="skip the ternary packed-K/V measurement")
    ap.add_argument("--no-c5", action="store_true", help="skip the config-5 32-layer model measurement")
    ap.add_argument("--cpu-heads", type=int, default=32, help="heads timed for the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0,
                    help="minimum CPU work for the CPU baseline (whole passes over --cpu-heads)")
    ap.add_argument("--no-sweep", action="store_true",
                    help="skip config 3: the density sweep at N in {2048, 8192, 32768} against the dense case")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="also run a plain 256 MiB device copy (reference for HBM byte counters)")
    return ap.parse_args()


def cpu_model():
    """CPU model string plus family / model / stepping and socket count from /proc/cpuinfo."""
    fields, sockets = {}, set()
    try:
        with open("/proc/cpuinfo") as fh:
            for line in fh:
                if ":" not in line:
                    continue
                key, val = (x.strip() for x in line.split(":", 1))
                if key == "physical id":
                    sockets.add(val)
                elif key in ("model name", "cpu family", "model", "stepping", "vendor_id") and key not in fields:
                    fields[key] = val
    except OSError:
        pass
    name = fields.get("model name") or platform.processor() or platform.machine()
    extra = ", ".join(f"{k} {fields[k]}" for k in ("vendor_id", "cpu family", "model", "stepping") if k in fields)
    return f"{name} ({extra}; {max(1, len(sockets))} socket(s))" if extra else name


def cpu_info(torch):
    return {"cpu_model": cpu_model(), "cpu_cores": os.cpu_count(), "torch_threads": torch.get_num_threads(),
            "torch": torch.__version__}


def median_wall(fn, runs=3):
    """One warm-up call, then the median wall time (s) of `runs` calls (BASELINE: >= 3 runs)."""
    fn()
    ts = []
    for _ in range(runs):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def cpu_baselines(torch, wl, dev):
    """Per-configuration CPU baselines (masked-dense fp32 reference on the host cores;
    configs 1 and 3 at N <= 8192 on all heads, config 3 at N = 32768 on one head scaled by 32,
    config 5 on two of the 32 heads of one layer scaled by 16). Each record: wall time (median of
    3 runs after a warm-up), FLOP_alg of the timed work and the equivalent TFLOP/s."""
    from oracle import attention as oa
    from ultrametric import block_lists_from_mask
    out = {}
    # config 1: fp32, all 4 heads
    c1 = wl.config1()
    bm1 = c1["block_mask"][0]
    bl1 = block_lists_from_mask(c1["block_mask"].to(dev), is_causal=True)
    f1 = wl.prefill_flops(bl1.counts, 64, 64)
    w1 = median_wall(lambda: oa.masked_attention_torch_fp32(c1["q"][0], c1["k"][0], c1["v"][0], bm1, 64, True))
    out["config1"] = {"shape": "fp32 Z1 H4 N1024 D64 RB64 causal, Bernoulli(0.25) + diag + sink", "seed": 1,
                      "heads_timed": 4, "wall_ms": round(w1 * 1e3, 3), "flop_alg": f1,
                      "tflops": round(f1 / w1 / 1e12, 5)}
    log(f"cpu config1 {w1 * 1e3:.1f} ms")
    # config 3: one timing per N (the masked-dense work does not depend on the density),
    # FLOP_alg per density of that N's listed tiles
    for N in (2048, 8192, 32768):
        NB = N // 128
        heads = 32 if N <= 8192 else 1
        g = torch.Generator().manual_seed(3)
        q, k, v = (torch.randn(1, heads, N, 128, generator=g).to(torch.bfloat16) for _ in range(3))
        bm = wl.bernoulli_block_mask(1, heads, NB, 0.25, seed=3 + int(0.25 * 1e6))[0]
        w = median_wall(lambda: oa.masked_attention_torch_fp32(q[0], k[0], v[0], bm, 128, True))
        per = {}
        for rho in (1.0, 0.5, 0.25, 0.0625, 0.016):
            m = wl.bernoulli_block_mask(1, 32, NB, rho, seed=3 + int(rho * 1e6))
            cnt = m.sum(-1).to(torch.int32)
            f = wl.prefill_flops(cnt[:, :heads], 128, 128)
            per[str(rho)] = {"flop_alg": f * (32 // heads), "tflops": round(f / w / 1e12, 5)}
        out[f"config3_N{N}"] = {
            "shape": f"bf16 Z1 H32 N{N} D128 RB128 causal, fp32 masked-dense on the host", "seed": 3,
            "heads_timed": heads, "scaled_to_32_heads": heads != 32,
            "wall_ms": round(w * 1e3 * (32 // heads), 3), "wall_ms_timed": round(w * 1e3, 3), "per_density": per}
        log(f"cpu config3 N={N} {w * 1e3:.1f} ms on {heads} head(s)")
        del q, k, v
    # config 5: one layer's attention at N = 16384 (32 q / 8 kv heads), two query heads timed
    g = torch.Generator().manual_seed(5)
    S5, heads5 = 16384, 2
    q5 = torch.randn(heads5, S5, 128, generator=g).to(torch.bfloat16)
    k5 = torch.randn(1, S5, 128, generator=g).to(torch.bfloat16)
    v5 = torch.randn(1, S5, 128, generator=g).to(torch.bfloat16)
    a5 = torch.randn(1, 32, S5, 4, 4, generator=g)
    from oracle import blocks as ob
    from oracle import surgery as osg
    route = osg.majority_route(a5.numpy(), 2, 128)
    bl5 = ob.build_block_lists(route, 2, is_causal=True, sink_block=True, local_blocks=1, arity=4)
    bm5 = torch.from_numpy(ob.lists_to_mask(bl5.lists, bl5.counts))[0, :heads5]
    w5 = median_wall(lambda: oa.masked_attention_torch_fp32(q5, k5, v5, bm5, 128, True))
    f5 = wl.prefill_flops(torch.from_numpy(bl5.counts)[0, :heads5], 128, 128)
    out["config5_layer"] = {
        "shape": "one Llama-3.1-8B attention layer: bf16 N16384 32 q / 8 kv heads D128 RB128, r 2 of 4 levels, "
                 "p 4, sink + 1 local block; fp32 masked-dense on the host", "seed": 5,
        "heads_timed": heads5, "scaled_to_32_heads": True, "wall_ms": round(w5 * 1e3 * 16, 3),
        "wall_ms_timed": round(w5 * 1e3, 3), "flop_alg": f5 * 16, "tflops": round(f5 / w5 / 1e12, 5)}
    log(f"cpu config5 layer {w5 * 1e3:.1f} ms on {heads5} heads")
    return out


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def time_launches(fn, reps, torch):
    """Average GPU time per call of `fn` over `reps` back-to-back calls (HIP events on
    torch's current stream, which is where the kernels are launched)."""
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    s.record()
    for _ in range(reps):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / reps


def spin_up(fn, ms, torch):
    """Calls `fn` back to back for `ms` milliseconds (untimed), then synchronizes: the
    first tens of milliseconds of continuous work run below the GPU's steady clocks
    (the config-2 step measured 90.6 then 80.9 us in two consecutive 200-step blocks).
    Returns the number of calls."""
    n = 0
    end = time.perf_counter() + ms * 1e-3
    while time.perf_counter() < end:
        fn()
        n += 1
    torch.cuda.synchronize()
    return n


def density_sweep(torch, wl, nat, dev, reps):
    """Config 3: bf16, H32, D128, causal, route block 128; per head Bernoulli(rho) over the
    lower-triangular blocks + diagonal + sink, rho in {1, .5, .25, .0625, .016}, N in
    {2048, 8192, 32768}. Each point times the prefill kernel over those lists (raw ABI,
    HIP events); the dense case of the same build is rho = 1 (every causal block listed);
    torch's scaled_dot_product_attention (causal) is timed as an external dense reference.
    Returns one record per point: listed fraction of causal blocks, time, TFLOP/s on listed
    tiles, speedup over the dense case of the same build and over SDPA."""
    from ultrametric import block_lists_from_mask
    import torch.nn.functional as F
    out = []
    Z, H, D, RB = 1, 32, 128, 128
    for N in (2048, 8192, 32768):
        NB = N // RB
        g = torch.Generator(device=dev).manual_seed(3)
        q, k, v = (torch.randn(Z, H, N, D, generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
                   for _ in range(3))
        o = torch.empty_like(q)
        st = [nat.strides(t) for t in (q, k, v, o)]
        stream = nat.stream(dev)
        causal_blocks = Z * H * NB * (NB + 1) // 2
        dense_ms = None
        with torch.no_grad():
            sdpa = lambda: F.scaled_dot_product_attention(q, k, v, is_causal=True)  # noqa: E731
            try:
                sdpa_ms = time_launches(sdpa, reps, torch)
            except RuntimeError:
                sdpa_ms = None
            for rho in (1.0, 0.5, 0.25, 0.0625, 0.016):
                mask = wl.bernoulli_block_mask(Z, H, NB, rho, seed=3 + int(rho * 1e6)).to(dev)
                bl = block_lists_from_mask(mask, is_causal=True)
                lists = bl.lists.contiguous()
                tiles = int(bl.counts.sum())

                def fwd():
                    nat.check(nat.lib().sa_block_sparse_fwd(
                        nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(o), None, nat.ptr(lists), nat.ptr(bl.counts),
                        None, 0, Z, H, H, N, D, RB, bl.max_count, st[0], st[1], st[2], st[3], None,
                        1.0 / math.sqrt(D), 1, 1, stream))
                ms = time_launches(fwd, reps, torch)
                if rho == 1.0:
                    dense_ms = ms
                flop = 4.0 * D * RB * RB * tiles
                out.append({"N": N, "rho": rho, "listed_fraction_causal": round(tiles / causal_blocks, 5),
                            "ms": round(ms, 5), "tflops": round(flop / (ms * 1e-3) / 1e12, 1),
                            "speedup_vs_dense_same_build": round(dense_ms / ms, 3),
                            "speedup_vs_sdpa": None if sdpa_ms is None else round(sdpa_ms / ms, 3),
                            "sdpa_ms": None if sdpa_ms is None else round(sdpa_ms, 5)})
                log(f"sweep N={N} rho={rho}: {ms * 1e3:.1f} us, listed {tiles / causal_blocks:.4f} of causal blocks")
                del mask, bl, lists
        del q, k, v, o
        torch.cuda.empty_cache()
    return out



def surgery_model_c5(torch, dev, args):
    """Config 5 end to end, as the reference times it (experiments/bench_surgery_prefill.py:
    81-108, 146-178): a 32-layer Llama-3.1-8B-shaped decoder (random-init bf16 weights, seeded
    N(0, 1) tree-routing scores per layer, p 4, 4 levels) runs a 16384-token prefill of seeded
    random token ids, without the LM head. Conditions: dense_sdpa (the unmodified model: torch's
    SDPA, causal, key / value heads repeated) and block_list@r for r in {2, 3, 4} (route-block
    vote, sync-free lists, GQA block-sparse prefill); block_list@0 lists every causal block, the
    dense model on this build's kernel. Each condition: one untimed pass that
    collects the list statistics, `warm` untimed passes, then `reps` timed passes; medians of
    the whole forward (HIP events) and of the summed attention-block time (events around each
    layer's projections + RoPE + routing + attention + output projection, the reference's
    attention-module hooks)."""
    from ultrametric.llama_model import LLAMA31_8B, SurgeryLlama
    warm, reps, S = 2, 5, 16384
    log("config 5: building the 32-layer model")
    model = SurgeryLlama(LLAMA31_8B, device=dev, seed=0)
    g = torch.Generator(device="cpu").manual_seed(0)
    ids = torch.randint(0, LLAMA31_8B.vocab, (1, S), generator=g).to(dev)
    med = lambda xs: sorted(xs)[len(xs) // 2]  # noqa: E731
    conds = []
    for name, attn, r in (("dense_sdpa", "sdpa", 0), ("block_list@0", "block_list", 0),
                          ("block_list@2", "block_list", 2), ("block_list@3", "block_list", 3),
                          ("block_list@4", "block_list", 4)):
        model.attention, model.r = attn, r
        rec = {"condition": name}
        with torch.no_grad():
            if attn == "block_list":
                model(ids, collect_stats=True)
                st = model.last_stats
                rec["block_density"] = round(sum(x["block_density"] for x in st) / len(st), 5)
                rec["measured_budget"] = round(sum(x["mean_allowed_keys"] for x in st) /
                                               sum(x["mean_causal_keys"] for x in st), 5)
            for _ in range(warm):
                model(ids)
            torch.cuda.synchronize()
            torch.cuda.reset_peak_memory_stats(dev)
            totals, attns = [], []
            for _ in range(reps):
                model.attn_events = []
                s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                s.record()
                model(ids)
                e.record()
                torch.cuda.synchronize()
                totals.append(s.elapsed_time(e))
                attns.append(sum(a.elapsed_time(b) for a, b in model.attn_events))
                model.attn_events = None
        rec.update({"total_ms": round(med(totals), 2), "total_ms_all": [round(x, 2) for x in totals],
                    "attn_ms": round(med(attns), 2),
                    "peak_mem_gb": round(torch.cuda.max_memory_allocated(dev) / 1024 ** 3, 2)})
        log(f"config 5 {name}: forward {rec['total_ms']:.1f} ms, attention {rec['attn_ms']:.1f} ms")
        conds.append(rec)
    dense = conds[0]
    for rec in conds[1:]:
        rec["speedup_total_vs_dense"] = round(dense["total_ms"] / rec["total_ms"], 3)
        rec["speedup_attn_vs_dense"] = round(dense["attn_ms"] / rec["attn_ms"], 3)
    del model, ids
    return {
        "workload": "config5: Llama-3.1-8B-shaped decoder, 32 layers, d 4096, 32 q / 8 kv heads, D 128, SwiGLU "
                    "14336, RoPE theta 5e5, random-init bf16 weights; per-layer seeded N(0,1) routing scores "
                    "(p 4, 4 levels), route block 128, local window 16 (1 block), sink; 16384-token prefill of "
                    "seeded random ids, no LM head",
        "timing": f"median of {reps} forwards after {warm} warmup + 1 statistics pass; attn_ms = summed HIP-event "
                  "time of the 32 attention blocks (q/k/v projections, RoPE, routing, attention, o projection)",
        "conditions": conds,
    }

def main():
    args = parse_args()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              f"(asked for --gpus {args.gpus}, WORLD_SIZE {world}).", file=sys.stderr)
        sys.exit(2)

    import torch

    import sparse_workloads as wl
    from ultrametric import block_list_attention, build_block_lists, routed_block_attention, ultrametric_decode
    from ultrametric import _native as nat

    if not torch.cuda.is_available():
        print("bench.py needs a HIP GPU", file=sys.stderr)
        sys.exit(2)
    if not nat.available():
        raise RuntimeError("libsparseattn.so is not built")
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)

    # ---------------- config 2: build + prefill -------------------------------------
    log("generating config 2")
    c = wl.config2(device=dev)
    q, k, v, router = c["q"], c["k"], c["v"], c["router"]
    Z, H, N, D = q.shape
    RB = c["route_block"]

    def build():
        return build_block_lists(router, 2, is_causal=True, sink_block=True, arity=4)

    bl = build()
    counts = bl.counts
    flop_alg = wl.prefill_flops(counts, D, RB)
    n_tiles = int(counts.sum())
    total_tiles = Z * H * (N // RB) ** 2
    causal_tiles = Z * H * (N // RB) * (N // RB + 1) // 2
    mask = wl.lists_to_block_mask(bl.lists, counts)
    useful = wl.useful_prefill_flops(mask, RB, N, D, True)

    def step():
        return block_list_attention(q, k, v, build(), route_block=RB, is_causal=True)

    def step_fused():
        # the same step in one launch: the list build runs inside the prefill kernel
        return routed_block_attention(q, k, v, router, 2, route_block=RB, is_causal=True, sink_block=True, arity=4)

    with torch.no_grad():
        spin_steps = spin_up(step, args.spinup_ms, torch)   # untimed, before the warmup steps
        log(f"spin-up {spin_steps} steps, warmup {args.warmup}")
        for _ in range(args.warmup):
            step()
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        s.record()
        for _ in range(args.steps):
            step()
        e.record()
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
        ms_step = s.elapsed_time(e) / args.steps
        log(f"timed {args.steps} steps: {ms_step * 1e3:.1f} us/step (wall {wall * 1e3 / args.steps * 1e3:.1f} us)")

        reps = max(50, args.steps)
        fused_step_ms = time_launches(step_fused, reps, torch)
        assert torch.equal(step(), step_fused()), "fused step disagrees with the two-launch step"

        # raw ABI launches of the fused build + prefill, back to back
        out = torch.empty_like(q)
        lists_f = torch.empty_like(bl.lists)
        counts_f = torch.empty_like(counts)
        st = [nat.strides(t) for t in (q, k, v, out)]
        lib = nat.lib()
        scale = 1.0 / math.sqrt(D)
        stream = nat.stream(dev)

        # arguments converted once: the launches, not Python call overhead
        fargs = (nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(out), None, nat.ptr(router),
                 nat.DTYPE_CODES[router.dtype], nat.strides(router), router.shape[-1], None, 2, 4, 1, 0,
                 nat.ptr(lists_f), nat.ptr(counts_f), Z, H, H, N, D, RB, st[0], st[1], st[2], st[3], scale, 1, 1,
                 stream)
        fused_fn = lib.sa_routed_block_sparse_fwd

        def fused():
            nat.check(fused_fn(*fargs))

        # the step's dominant kernel: the prefill over prebuilt lists, raw ABI launches
        lists = bl.lists.contiguous()
        out2 = torch.empty_like(q)

        pargs = (nat.ptr(q), nat.ptr(k), nat.ptr(v), nat.ptr(out2), None, nat.ptr(lists), nat.ptr(counts), None,
                 0, Z, H, H, N, D, RB, bl.max_count, st[0], st[1], st[2], st[3], None, scale, 1, 1, stream)
        fwd_fn = lib.sa_block_sparse_fwd

        def fwd():
            nat.check(fwd_fn(*pargs))

        # alternating rounds, medians: a single block can catch a transient clock state
        fl, pl = [], []
        for _ in range(3):
            fl.append(time_launches(fused, reps, torch))
            pl.append(time_launches(fwd, reps, torch))
        fused_ms, fwd_ms = sorted(fl)[1], sorted(pl)[1]
        build_ms = time_launches(build, reps, torch)
        ref_out = block_list_attention(q, k, v, bl, route_block=RB, is_causal=True)
        assert torch.equal(out, ref_out) and torch.equal(out2, ref_out), "raw-ABI launch disagrees with the API"
        assert torch.equal(lists_f, bl.lists) and torch.equal(counts_f, counts), "fused lists differ"
    log(f"prefill kernel {fwd_ms * 1e3:.1f} us, build API call {build_ms * 1e3:.1f} us (host-bound); fused build + "
        f"prefill: kernel "
        f"{fused_ms * 1e3:.1f} us, step {fused_step_ms * 1e3:.1f} us")

    value = flop_alg / (ms_step * 1e-3) / 1e12
    achieved = flop_alg / (fwd_ms * 1e-3) / 1e12
    result = {
        "metric": "block-sparse prefill TFLOP/s (computed tiles) at N=8K",
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "spinup_steps": spin_steps,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded N(0,1) Q/K/V, seeded tree routing)",
        "config": {
            "workload": "config2: block-sparse prefill fwd, B1 H32 N8192 D128, route block 128, causal, "
                        "p=4 depth-3 tree routing (LCA>=2) + diagonal + sink; step = sync-free list build + fwd",
            "global_batch": 1, "seq_len": N, "heads": H, "head_dim": D, "route_block": RB,
            "active_tiles": n_tiles, "tile_density_full": round(n_tiles / total_tiles, 5),
            "tile_density_causal": round(n_tiles / causal_tiles, 5),
            "flop_alg": flop_alg, "flop_useful_token_exact": useful,
            "useful_fraction_of_computed": round(useful / flop_alg, 4),
            "parallelism": "single GPU",
        },
        "prefill_kernel_ms": round(fwd_ms, 5),
        "build_ms": round(build_ms, 5),
        "build_note": "back-to-back build_block_lists API calls: bound by the host call (checks, allocation), "
                      "the build kernel itself is ~5 us (rocprofv3) and overlaps the previous prefill in a step",
        "fused_build_prefill": {"kernel_ms": round(fused_ms, 5), "ms_per_step": round(fused_step_ms, 5),
                                "api": "routed_block_attention(..., arity=4): one launch, lists written out"},
        "roofline": {
            "kernel": "prefill_mfma_kernel<bf16, D=128, 4 waves, causal>",
            "bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS, "unit": "TFLOP/s",
            "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
            "traffic": profiled_traffic("prefill_mfma_config2_bf16.md"),
            "traffic_source": "profiles/prefill_mfma_config2_bf16.md",
            "unique_hbm_bytes": 4 * q.numel() * q.element_size(),
        },
    }
    # Both roofs for the same launch: config 2's arithmetic intensity (FLOP_alg per
    # unique HBM byte) sits below the ridge point, so the HBM roof binds first.
    uniq = 4 * q.numel() * q.element_size()
    t_mfma_us = flop_alg / (PEAK_BF16_TFLOPS * 1e12) * 1e6
    t_hbm_us = uniq / (PEAK_HBM_GBS * 1e9) * 1e6
    result["roofline"]["hbm_view"] = {
        "achieved_gbs_unique": round(uniq / (fwd_ms * 1e-3) / 1e9, 1),
        "frac_of_hbm_peak": round(uniq / (fwd_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4),
        "intensity_flop_per_byte": round(flop_alg / uniq, 1),
        "ridge_flop_per_byte": round(PEAK_BF16_TFLOPS * 1e12 / (PEAK_HBM_GBS * 1e9), 1),
        "roof_time_us": {"mfma": round(t_mfma_us, 2), "hbm": round(t_hbm_us, 2)},
        "frac_of_binding_roof": round(max(t_mfma_us, t_hbm_us) / (fwd_ms * 1e3), 4),
    }

    if args.calibrate_copy:
        # A plain copy of known size: under `rocprofv3 --pmc FETCH_SIZE` / `WRITE_SIZE`
        # its dispatch reads / writes exactly 256 MiB, which calibrates those counters.
        src = torch.empty(128 * 1024 * 1024, dtype=torch.bfloat16, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        result["calibration_copy_bytes"] = src.numel() * src.element_size()
        del src, dst

    # ---------------- config 2 backward (dQ, dK, dV through the public API) ------------
    if not args.no_backward:
        from ultrametric.block_list import _launch_bwd
        with torch.no_grad():
            out_b, lse_b = block_list_attention(q, k, v, bl, route_block=RB, is_causal=True, return_lse=True)
        g = torch.Generator(device="cpu").manual_seed(5)
        dout_b = torch.randn(q.shape, generator=g).to(q.dtype).to(dev)
        scale_b = 1.0 / math.sqrt(D)

        def bwd():
            return _launch_bwd(dout_b, q, k, v, out_b, lse_b, bl.lists, bl.counts, bl.max_count, None, RB, True,
                               scale_b)

        for _ in range(3):
            bwd()
        # as for the prefill step: the first tens of milliseconds of continuous
        # work run below steady clocks (the first 20 calls measured ~10% slower)
        spin_up(bwd, args.spinup_ms, torch)
        bwd_ms = time_launches(bwd, max(20, args.steps // 5), torch)
        bwd_flop = 2.5 * flop_alg      # S, dP, dV, dK, dQ: five products of the forward's two
        result["backward"] = {
            "workload": "config2 backward: delta + dQ over lists, dK / dV over transposed lists, bf16",
            "ms_per_call": round(bwd_ms, 5),
            "flop_alg": bwd_flop,
            "tflops_alg": round(bwd_flop / (bwd_ms * 1e-3) / 1e12, 1),
            "includes": "transposed lists, work plan (one host read), all kernels",
        }
        log(f"backward {bwd_ms * 1e3:.1f} us/call, {bwd_flop / (bwd_ms * 1e-3) / 1e12:.0f} TFLOP/s algorithmic")
        del out_b, lse_b, dout_b

    # ---------------- ternary packed K / V over config 2's lists -------------------------
    if not args.no_ternary:
        from ultrametric import ternary_quantize_pack
        qh = q.half()
        kp, ksc = ternary_quantize_pack(k)
        vp, vsc = ternary_quantize_pack(v)
        tout = torch.empty_like(qh)
        targs = (nat.ptr(qh), nat.ptr(kp), nat.ptr(vp), nat.ptr(ksc), nat.ptr(vsc), 0, nat.ptr(lists),
                 nat.ptr(counts), bl.max_count, nat.ptr(tout), Z, H, H, N, D, 0, nat.strides(qh), nat.strides(kp),
                 nat.strides(vp), nat.strides(ksc), nat.strides(vsc), nat.strides(tout), stream)
        tfn = nat.lib().sa_ternary_prefill_fwd

        def tern():
            nat.check(tfn(*targs))

        tern_ms = time_launches(tern, max(50, args.steps), torch)
        result["ternary"] = {
            "workload": "config2 lists, fp16 Q, K / V quantized to 2-bit ternary codes + fp32 row scales "
                        "(64 B per key row instead of 512)",
            "ms_per_call": round(tern_ms, 5),
            "tflops": round(flop_alg / (tern_ms * 1e-3) / 1e12, 1),
            "kv_bytes": kp.numel() * 4 * 2 + ksc.numel() * 4 * 2,
            "kv_bytes_bf16": k.numel() * 2 * 2,
        }
        log(f"ternary prefill {tern_ms * 1e3:.1f} us, {flop_alg / (tern_ms * 1e-3) / 1e12:.0f} TFLOP/s")
        del qh, kp, vp, ksc, vsc, tout

    # ---------------- config 5: 32-layer Llama-shaped prefill, block-list vs dense SDPA ---
    if not args.no_c5:
        result["surgery_prefill_c5"] = surgery_model_c5(torch, dev, args)
        torch.cuda.empty_cache()

    # ---------------- config 3: density sweep ------------------------------------------
    if not args.no_sweep:
        result["sweep"] = density_sweep(torch, wl, nat, dev, reps=max(20, args.steps // 4))

    # ---------------- config 4: sparse paged decode -----------------------------------
    if not args.no_decode:
        log("generating config 4")
        w = wl.config4(device=dev)
        kw = dict(req_depth=w.req_depth, local_blocks=w.local_blocks, sink_block=w.sink_block)
        b_alg, upages = wl.decode_routed_bytes(w)
        B, Hq, Dd = w.q.shape
        P, Hkv, PS, _ = w.k_cache.shape
        TD = w.q_router.shape[-1]
        max_pages = w.block_tables.shape[1]
        ws_bytes = nat.lib().sa_decode_workspace_bytes(B, Hq, Hkv, Dd, max_pages)
        ws = torch.empty(ws_bytes, dtype=torch.uint8, device=dev) if ws_bytes else None
        dout = torch.empty_like(w.q)
        bt = w.block_tables.to(torch.int32)
        ctxl = w.context_lens.to(torch.int32).contiguous()
        # raw ABI launches with prebuilt arguments: the kernel, not Python call overhead
        dargs = (nat.ptr(w.q), nat.ptr(w.k_cache), nat.ptr(w.v_cache), nat.ptr(bt), nat.ptr(ctxl),
                 nat.ptr(w.router), nat.ptr(w.q_router), nat.ptr(dout), B, Hq, Hkv, Dd, PS, TD, max_pages, P,
                 w.req_depth, w.local_blocks, int(w.sink_block), nat.strides(w.q), nat.strides(w.k_cache),
                 nat.strides(w.v_cache), nat.strides(bt), nat.strides(w.router), nat.strides(w.q_router),
                 nat.strides(dout), None if ws is None else nat.ptr(ws), ws_bytes,
                 nat.dtype_code(w.q.dtype, (torch.float32, torch.bfloat16, torch.float16)),
                 stream)
        dec_fn = nat.lib().sa_sparse_paged_decode

        def dec():
            nat.check(dec_fn(*dargs))

        with torch.no_grad():
            spin_up(dec, args.spinup_ms, torch)   # the GPU idled while config 4 was generated
            for _ in range(args.warmup):
                dec()
            dec_ms = time_launches(dec, max(50, args.steps), torch)
            api_out = ultrametric_decode(w.q, w.k_cache, w.v_cache, w.block_tables, w.context_lens, w.router,
                                         w.q_router, **kw)
            assert torch.equal(api_out, dout), "raw-ABI decode disagrees with the public API"
        meta_bytes = int(w.context_lens.add(15).div(16, rounding_mode="floor").sum()) * (4 + 32 * 4 * 4)
        dec_gbs = b_alg / (dec_ms * 1e-3) / 1e9
        result["decode"] = {
            "workload": "config4: 64 seqs, L~U[4096,32768], GQA 32/8, D128, page 16, p=4 depth-4 routing "
                        "(req_depth 4) + sink + last 4 pages, bf16",
            "ms_per_call": round(dec_ms, 5),
            "routed_kv_bytes": b_alg, "unique_pages": upages,
            "routing_metadata_bytes": meta_bytes,
            "gbs_routed": round(dec_gbs, 1),
            "roofline": {"kernel": "decode_kernel<bf16, D=128, G=4, mode 0 (reference router)>", "bound": "hbm", "achieved": round(dec_gbs, 1),
                         "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(dec_gbs / PEAK_HBM_GBS, 4),
                         "traffic": profiled_traffic("decode_config4_bf16.md"),
                         "traffic_source": "profiles/decode_config4_bf16.md"},
        }
        log(f"decode {dec_ms * 1e3:.1f} us/call, {dec_gbs:.0f} GB/s on routed bytes")

        # same decode with packed routing codes: 4 bytes per (page, head) instead of 4 * TD
        from ultrametric.kernel_decode import pack_routing_codes
        bpl = max(1, int(max(w.router.max().item(), w.q_router.max().item())).bit_length())
        pc, qc = pack_routing_codes(w.router, bpl), pack_routing_codes(w.q_router, bpl)
        pout = torch.empty_like(w.q)
        pargs = list(dargs)
        pargs[5], pargs[6], pargs[7] = nat.ptr(pc), nat.ptr(qc), nat.ptr(pout)
        pargs[23], pargs[24] = nat.strides(pc), nat.strides(qc)
        pargs.insert(14, bpl)
        pdec_fn = nat.lib().sa_sparse_paged_decode_codes

        def pdec():
            nat.check(pdec_fn(*pargs))

        with torch.no_grad():
            for _ in range(args.warmup):
                pdec()
            pdec_ms = time_launches(pdec, max(50, args.steps), torch)
        assert torch.equal(pout, dout), "packed-code decode disagrees with the int32-level decode"
        pgbs = b_alg / (pdec_ms * 1e-3) / 1e9
        result["decode"]["packed_codes"] = {
            "bits_per_level": bpl, "ms_per_call": round(pdec_ms, 5), "gbs_routed": round(pgbs, 1),
            "routing_metadata_bytes": int(w.context_lens.add(15).div(16, rounding_mode="floor").sum()) * (4 + 32 * 4),
            "frac": round(pgbs / PEAK_HBM_GBS, 4),
        }
        log(f"decode (packed codes) {pdec_ms * 1e3:.1f} us/call, {pgbs:.0f} GB/s on routed bytes")

        # packed codes stored per sequence in logical page order (serving layout)
        from ultrametric.kernel_decode import sequence_page_codes
        sc = sequence_page_codes(pc, bt, bits=TD * bpl)
        sout = torch.empty_like(w.q)
        sargs = list(pargs)
        sargs[5], sargs[7] = nat.ptr(sc), nat.ptr(sout)
        sargs[24] = nat.strides(sc)
        sargs.insert(6, sc.element_size())
        sdec_fn = nat.lib().sa_sparse_paged_decode_seq_codes

        def sdec():
            nat.check(sdec_fn(*sargs))

        with torch.no_grad():
            for _ in range(args.warmup):
                sdec()
            sdec_ms = time_launches(sdec, max(50, args.steps), torch)
        assert torch.equal(sout, pout), "sequence-code decode disagrees with the page-code decode"
        sgbs = b_alg / (sdec_ms * 1e-3) / 1e9
        result["decode"]["sequence_codes"] = {
            "bits_per_level": bpl, "ms_per_call": round(sdec_ms, 5), "gbs_routed": round(sgbs, 1),
            "routing_metadata_bytes": int(w.context_lens.add(15).div(16, rounding_mode="floor").sum())
            * (4 + 32 * sc.element_size()),
            "frac": round(sgbs / PEAK_HBM_GBS, 4),
            "layout": f"(B, H, max_pages) {8 * sc.element_size()}-bit codes in logical page order, read with the block table",
        }
        # the roofline is quoted on the serving layout (sequence codes); the reference
        # layout (int32 levels per physical page and head) scans ~36 MB of scattered
        # router lines on top of the routed bytes, so it sits beside it
        result["decode"]["roofline_reference_layout"] = result["decode"]["roofline"]
        result["decode"]["roofline"] = {
            "kernel": "decode_kernel<bf16, D=128, G=4, mode 2 (sequence codes)>", "bound": "hbm",
            "achieved": round(sgbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s", "frac": round(sgbs / PEAK_HBM_GBS, 4),
            "traffic": profiled_traffic("decode_config4_seqcodes_bf16.md"),
            "traffic_source": "profiles/decode_config4_seqcodes_bf16.md"}
        log(f"decode (sequence codes) {sdec_ms * 1e3:.1f} us/call, {sgbs:.0f} GB/s on routed bytes")

        if not args.no_cpu:
            # decode: the float64 loop oracle (the reference's _ultrametric_decode_reference
            # semantics, GQA grouped) over all 64 sequences x 32 heads of config 4 (with
            # --cpu-quick the first 4 sequences). Only the pages some head of a sequence selects
            # are copied to the host; every other table slot points at a page whose routing
            # vector matches no query, so the oracle selects exactly what it would on the full
            # cache.
            import numpy as np
            from oracle import decode as od
            ns = 4 if args.cpu_quick else B
            r_d = min(max(int(w.req_depth), 0), TD)
            ctx_t = w.context_lens[:ns].long()
            npg_t = (ctx_t + PS - 1) // PS
            lpos = torch.arange(max_pages, device=dev)[None, :]
            valid = lpos < npg_t[:, None]
            phys = w.block_tables[:ns].long().clamp(0, P - 1)
            sel = (w.router[phys][..., :r_d] == w.q_router[:ns, None, :, :r_d]).all(-1).any(-1)
            if w.sink_block:
                sel |= lpos == 0
            if w.local_blocks > 0:
                sel |= lpos >= (npg_t[:, None] - w.local_blocks)
            sel &= valid
            used = torch.unique(phys[sel])
            remap = torch.zeros(P, dtype=torch.long, device=dev)
            remap[used] = torch.arange(1, used.numel() + 1, device=dev)
            bt_c = torch.where(sel, remap[phys], torch.zeros_like(phys)).cpu().numpy()
            ctx_s = ctx_t.cpu().numpy()

            def compact(t):
                body = t[used].float()
                return torch.cat([torch.zeros_like(body[:1]), body]).cpu().numpy()

            kc_s, vc_s = compact(w.k_cache), compact(w.v_cache)
            r_s = w.router[used].cpu().numpy()
            r_s = np.concatenate([np.full((1,) + r_s.shape[1:], -1, dtype=r_s.dtype), r_s])
            q_s = w.q[:ns].float().cpu().numpy()
            qr_s = w.q_router[:ns].cpu().numpy()
            dcpu_s = median_wall(lambda: od.decode_reference(q_s, kc_s, vc_s, bt_c, ctx_s, r_s, qr_s, **kw))
            b_s, _ = od.routed_page_bytes(bt_c, ctx_s, r_s, qr_s, Hkv, PS, Dd, 2, **kw)
            result["decode"]["cpu_baseline"] = {
                "value": round(b_s / dcpu_s / 1e9, 4), "unit": "GB/s", "cores": torch.get_num_threads(),
                "kind": "port",
                "sample": f"float64 decode oracle (oracle/decode.py decode_reference, the reference's "
                          f"_ultrametric_decode_reference loop) on {ns} of {B} sequences x all {Hq} heads, "
                          f"median of 3 passes after a warm-up: {dcpu_s * 1e3:.1f} ms per pass; value = "
                          f"routed bytes of those sequences / wall time per pass",
                "wall_ms": round(dcpu_s * 1e3, 3), "bytes_alg": int(b_s), "sequences": ns, "seed": 4,
            }
            log(f"decode cpu baseline {dcpu_s * 1e3:.1f} ms per pass over {ns} sequences")
            del kc_s, vc_s
        del w

    # ---------------- CPU baseline (oracle, host cores) --------------------------------
    if not args.no_cpu:
        from oracle import attention as oa
        heads = list(range(min(args.cpu_heads, H)))
        qc, kc, vc = (t[0, heads].cpu() for t in (q, k, v))
        mk = mask[0, heads].cpu()
        oa.masked_attention_torch_fp32(qc[:1, :256], kc[:1, :256], vc[:1, :256], mk[:1, :2, :2], RB, True)
        # whole passes over the sampled heads until at least --cpu-seconds of CPU work
        passes, t0 = 0, time.perf_counter()
        while True:
            oa.masked_attention_torch_fp32(qc, kc, vc, mk, RB, True)
            passes += 1
            if time.perf_counter() - t0 >= args.cpu_seconds:
                break
        cpu_s = (time.perf_counter() - t0) / passes
        flop_sample = wl.prefill_flops(counts[0, heads], D, RB)
        result["cpu_baseline"] = {
            "value": round(flop_sample / cpu_s / 1e12, 4), "unit": "TFLOP/s",
            "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"fp32 masked-dense oracle (oracle/attention.py masked_attention_torch_fp32, the "
                      f"reference's masked_reference_attention formulation, query-chunked 2048) on "
                      f"{len(heads)} of {H} heads of config 2; {passes} passes, {cpu_s:.2f} s per pass; "
                      f"value = FLOP_alg of those heads' listed tiles / wall time per pass",
            "cpu_model": cpu_model(),
            "os_cpu_count": os.cpu_count(),
            "torch": torch.__version__,
            "wall_ms": round(cpu_s * 1e3, 3), "flop_alg": flop_sample, "seed": 2,
        }
        log(f"cpu baseline {cpu_s:.2f} s per pass over {len(heads)} heads ({passes} passes)")
        if not args.cpu_quick:
            rec = {"info": cpu_info(torch)}
            rec["config2"] = {"shape": "bf16 Z1 H32 N8192 D128 RB128 causal, tree routing p4 depth 3 LCA >= 2 "
                                       "+ diag + sink; fp32 masked-dense on the host", "seed": 2,
                              "heads_timed": len(heads), "wall_ms": round(cpu_s * 1e3, 3),
                              "flop_alg": flop_sample, "tflops": result["cpu_baseline"]["value"]}
            rec.update(cpu_baselines(torch, wl, dev))
            if "decode" in result and "cpu_baseline" in result["decode"]:
                rec["config4"] = dict(result["decode"]["cpu_baseline"])
            result["cpu_baselines"] = rec

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
