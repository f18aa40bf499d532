"""CPU oracle for the block-sparse attention hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU with numpy (float64 for attention, exact
integer arithmetic for block lists), the reference algorithms of sparse-ai's
``src/ultrametric`` hot path. Every function names the reference file:line it
follows. It is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it. The shipped ``ultrametric`` package never imports it and has no
CPU fallback.

Modules:
  blocks     — routing codes, structural masks, block-list compaction,
               pairwise block-mask reference, transposed lists.
  attention  — token masks and masked-dense attention (out and LSE), float64
               numpy, plus the fp32 torch variant timed as the CPU baseline.
  decode     — sparse paged decode reference (GQA by head grouping), and
               the packed per-page routing codes.
  surgery    — the surgery caller's route-block majority vote and its
               allowed-key statistics.
  ternary    — ternary quantize / pack / unpack and the causal block-sparse
               prefill over packed K / V (llama_surgery).

Parity pinning: see the header of each module for the checks that pin it
(known-answer tests from the reference's own tests, closed forms, brute
force on tiny inputs). The reference ships no golden vectors for this path;
tests/golden/ holds this build's own fixtures (written from this oracle).
"""
