// Sparse paged decode with tree-routed page selection (gfx950).
//
// Semantics follow ultrametric_decode (src/ultrametric/kernel_decode.py:22-247)
// and its CPU reference (:129-185): for sequence b and query head h, logical
// page l (of n = ceil(ctx/page) pages) is attended iff the routing vector of
// its PHYSICAL page, router[block_tables[b, l], h, :r], equals
// q_router[b, h, :r] (r = req_depth clamped to [0, TD]), or l == 0 with
// sink_block, or l >= n - local_blocks. Tokens >= ctx are masked, scale is
// 1/sqrt(D), heads with no selected page and sequences with ctx <= 0 output
// zeros. GQA: k/v caches hold H_kv heads; query head h reads kv head
// h / (H / H_kv), and each K/V page is loaded once for the G = H / H_kv query
// heads of its group.
//
// decode_kernel: one workgroup (4 waves) per (sequence b, kv head, split).
// A split owns a contiguous range of logical pages (one split unless
// B * H_kv is too small to fill the GPU) and walks it 4096/G pages at a time:
//   phase A1 — G consecutive lanes share a page: all lanes load the page's
//     block-table entry, then lane j loads head j's routing vector (one
//     16-byte load when the router rows allow it, so a page's G vectors are
//     one contiguous read); a ballot turns the G match bits into the page's
//     head mask (forced pages: all heads). The passes of a range run in
//     groups of 16 (two groups, 2048 pages, at G = 4); a group issues its
//     loads back to back;
//   phase A2 — the selected pages are compacted into LDS in ascending logical
//     order (per-thread counts, wave prefix sum, per-wave offsets);
//   phase B — the 4 waves take selected pages round-robin with up to 2 pages
//     in flight per wave (register ring indexed by compile-time constants).
//     16 lanes cover one token row of D elements (one vector load each) and
//     the 4 lane groups take tokens g, g+4, ... of the page; QK uses packed
//     bf16/f16 dot products on the raw words; each lane group keeps its own
//     base-2 online-softmax state per head, so no cross-lane traffic happens
//     per page.
// The state survives across ranges in registers. At the end lane groups and
// waves are merged; with one split the workgroup writes out directly,
// otherwise it writes (m, l, acc[D]) partials that decode_merge_kernel
// combines. Consecutive work items (the kv heads of one sequence, which read
// the same block-table and router rows) are placed on one XCD.
#include "mfma_util.h"
#include <mutex>

namespace sa {
namespace {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = kDecWaves * 64;
constexpr int kMaxTD = 64;
constexpr int kTargetWorkgroups = 512;                   // ~2 per CU on MI355X

struct DecParams {
  const void* q;
  const void* kc;
  const void* vc;
  const int32_t* bt;
  const int32_t* ctx;
  const int32_t* router;
  const int32_t* qr;
  void* out;
  float* part;
  int B, H, Hkv, D, PS, TD, max_pages, P, r, local, sink, G, splits;
  int vec_router;  // router rows allow one 16-byte load of 4 levels per (page, head)
  const uint32_t* codes;    // packed mode: (P, H) page routing codes, or NULL
  const uint32_t* qcodes;   // packed mode: (B, H) query routing codes
  int64_t cs0, cs1, cs2, qcs0, qcs1;
  int lvec;                 // logical codes: rows allow 2 x 16-byte loads per 8 pages
  int logical;              // codes are (B, H, max_pages) in logical page order
  int code_bytes;           // logical codes: 1, 2 or 4 bytes per code
  const void* lcodes;       // logical codes (element size code_bytes)
  uint32_t code_mask;       // bits of the first r levels (0 when r == 0)
  int64_t qs0, qs1, qs2;
  int64_t ks0, ks1, ks2;
  int64_t vs0, vs1, vs2;
  int64_t bts0, bts1;
  int64_t rs0, rs1, rs2;
  int64_t qrs0, qrs1, qrs2;
  int64_t os0, os1, os2;
  float qk_scale;
  int mfma_b;               // phase B on MFMA (see decode_kernel)
  int kvdiv;                // work item's kv-head index / kvdiv = the cache head (1, or H / H_kv
                            // when the group size has no kernel and each query head is its own item)
};

// DPL consecutive elements (unit stride) kept as raw 32-bit words.
template <typename T, int DPL>
struct RowRegs {
  static constexpr int kWords = DPL * static_cast<int>(sizeof(T)) / 4 > 0 ? DPL * static_cast<int>(sizeof(T)) / 4 : 1;
  uint32_t w[kWords];
};

template <typename T, int DPL>
__device__ __forceinline__ void load_row(const T* ptr, RowRegs<T, DPL>& r) {
  constexpr int BYTES = DPL * static_cast<int>(sizeof(T));
  if constexpr (BYTES % 16 == 0) {
#pragma unroll
    for (int i = 0; i < BYTES / 16; ++i) {
      const uint4 u = reinterpret_cast<const uint4*>(ptr)[i];
      r.w[4 * i] = u.x; r.w[4 * i + 1] = u.y; r.w[4 * i + 2] = u.z; r.w[4 * i + 3] = u.w;
    }
  } else if constexpr (BYTES == 8) {
    const uint2 u = *reinterpret_cast<const uint2*>(ptr);
    r.w[0] = u.x; r.w[1] = u.y;
  } else if constexpr (BYTES == 4) {
    r.w[0] = *reinterpret_cast<const uint32_t*>(ptr);
  } else {  // 2 bytes (one 16-bit element)
    r.w[0] = *reinterpret_cast<const uint16_t*>(ptr);
  }
}

template <typename T, int DPL>
__device__ __forceinline__ float row_elem(const RowRegs<T, DPL>& r, int e) {
  if constexpr (sizeof(T) == 4) {
    return __uint_as_float(r.w[e]);
  } else {
    const uint32_t word = r.w[e >> 1];
    const uint32_t bits = (e & 1) ? (word >> 16) : (word & 0xffffu);
    if constexpr (std::is_same<T, bf16_t>::value) return bf16_bits_to_float(bits);
    else return f16_bits_to_float(bits);
  }
}

// Raw bits of one element (16-bit types zero-extended).
template <typename T>
__device__ __forceinline__ uint32_t elem_bits(const T* p) {
  if constexpr (sizeof(T) == 4) return __float_as_uint(*reinterpret_cast<const float*>(p));
  else return *reinterpret_cast<const uint16_t*>(p);
}

// Dot product of two rows held as raw words (same packing as RowRegs): packed
// 2-element dot products with fp32 accumulation for bf16 / f16
// (v_dot2c_f32_bf16 / v_dot2c_f32_f16; both products are exact in fp32), fp32
// FMAs otherwise.
template <typename T, int DPL>
__device__ __forceinline__ float row_dot(const uint32_t* a, const RowRegs<T, DPL>& b) {
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < RowRegs<T, DPL>::kWords; ++i) {
    if constexpr (std::is_same<T, bf16_t>::value) {
      s = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a[i]), __builtin_bit_cast(bf16x2_t, b.w[i]), s,
                                          false);
    } else if constexpr (std::is_same<T, f16_t>::value) {
      s = __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a[i]), __builtin_bit_cast(f16x2_t, b.w[i]), s, false);
    } else {
      s = fmaf(__uint_as_float(a[i]), __uint_as_float(b.w[i]), s);
    }
  }
  return s;
}

// MODE 0: int32 routing levels per (physical page, head) (the reference's
// router). MODE 1: packed routing codes per (physical page, head); the
// phase-A registers are then small enough for 2048-page ranges at G >= 4.
// MODE 2: packed codes per (sequence, head, logical page): a workgroup's codes
// are contiguous, so thread t reads the codes and block-table entries of
// pages 8t .. 8t+7 of a 2048-page range with wide loads issued in the
// prologue, and builds their head masks in registers (no ballot).
// MB: phase B on MFMA (16-bit K / V, D in {32, 64, 128}, pages of at most 16
// tokens, 16-byte aligned rows): per page S^T = K Q^T on 16x16x32 tiles (lane
// = head of the group, 4 tokens per lane), O^T += V^T P^T on 16x16x16 tiles
// with V^T read through this wave's LDS slot by transposing reads.
template <typename T, int D, int G, int MODE, bool MB>
__global__ __launch_bounds__(kDecThreads) __attribute__((amdgpu_waves_per_eu(G * D <= 512 ? 2 : 1)))
void decode_kernel(DecParams p) {
  static_assert(!MB || (sizeof(T) == 2 && (D == 32 || D == 64 || D == 128) && G <= 16), "MFMA phase B shapes");
  constexpr bool PACKED = MODE == 1;
  constexpr bool LOGICAL = MODE == 2;
  constexpr int DPL = D / 16;
  // Phase A layout: G consecutive lanes share one page (lane j reads head j's
  // routing vector, so a page's G vectors are one contiguous 16*G-byte read);
  // a pass covers kPagesPerPass pages and a range kPasses passes.
  constexpr int kPagesPerPass = kDecThreads / G;
  constexpr int kPasses = (PACKED && G >= 4) ? 32 : 16;
  // Phase A1 runs in halves of kPasses passes; a range of up to 2048 pages
  // (two halves when one covers at most 1024) then has one compaction and one
  // phase B.
  constexpr int kHalf = kPagesPerPass * kPasses;
  constexpr int kHalves = (!LOGICAL && kHalf <= 1024) ? 2 : 1;
  constexpr int kRange = LOGICAL ? 2048 : kHalf * kHalves;
  constexpr int kPagesPerThread = kRange / kDecThreads;
  static_assert(!LOGICAL || kPagesPerThread == 8, "logical codes: 8 pages per thread");
  __shared__ int32_t page_phys[LOGICAL ? 1 : kRange];
  __shared__ uint8_t page_mask[LOGICAL ? 1 : kRange];
  __shared__ int32_t sel_phys[kRange];
  __shared__ int32_t sel_meta[kRange];
  __shared__ int32_t qroute[G][kMaxTD];
  __shared__ int32_t wave_count[kDecWaves];
  __shared__ float red_m[kDecWaves][G];
  __shared__ float red_l[kDecWaves][G];
  __shared__ float red_acc[kDecWaves][G][D];
  // MFMA phase B: one page of V rows per wave (16 rows of 2D bytes), 32-byte
  // units of row r stored at unit u ^ vunit(r).
  __shared__ __attribute__((aligned(16))) char vstage[kDecWaves][MB ? 32 * D : 16];
  // MFMA phase B: K rows of the wave's early page (16-byte chunk c of row r at
  // position c ^ (r mod chunks per row)), and the early pages' physical ids.
  // (Only where the LDS still fits two workgroups per CU: ranges of at most
  // 2048 pages.)
  constexpr bool EARLY = MB && kRange <= 2048;
  __shared__ __attribute__((aligned(16))) char kstage[kDecWaves][EARLY ? 32 * D : 16];
  __shared__ int32_t early_phys[kDecWaves];

  // Work items ordered (b, kv head, split); consecutive items (the kv heads of
  // one sequence, which read the same block-table row and router rows) share
  // an XCD.
  const int work = xcd_remap(blockIdx.x, gridDim.x);
  const int split = work % p.splits;
  const int bk = work / p.splits;
  const int kvh = bk % p.Hkv;
  const int b = bk / p.Hkv;
  const int kvm = kvh / p.kvdiv;   // the cache's kv head
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h0 = kvh * G;
  const int gl = tid % G;       // head (within the group) whose routing vector this lane checks
  const int pslot = tid / G;    // page slot within a pass

  // A memory round trip costs microseconds under load, so every load that
  // does not depend on another is issued before the first wait: the first
  // range's block-table entries (split 0 starts at page 0 whatever the
  // context length), the context length, the query routing vectors and Q.
  const bool prefetched = split == 0 && p.max_pages > 0;
  // Block-table entries of pages lb .. lb + kPagesPerThread - 1 (clamped to
  // the table; 16-byte reads when the row is contiguous and aligned).
  auto load_bt = [&](int lb, int (&ph)[kPagesPerThread]) {
    if (kPagesPerThread % 4 == 0 && p.bts1 == 1 && (p.bts0 & 3) == 0 && (lb & 3) == 0 &&
        (reinterpret_cast<uintptr_t>(p.bt) & 15) == 0 && lb + kPagesPerThread <= p.max_pages) {
      const int4* src = reinterpret_cast<const int4*>(p.bt + static_cast<int64_t>(b) * p.bts0 + lb);
#pragma unroll
      for (int c = 0; c < kPagesPerThread / 4; ++c) {
        const int4 u = src[c];
        ph[4 * c] = u.x; ph[4 * c + 1] = u.y; ph[4 * c + 2] = u.z; ph[4 * c + 3] = u.w;
      }
    } else {
#pragma unroll
      for (int j = 0; j < kPagesPerThread; ++j) ph[j] = p.bt[b * p.bts0 + min(lb + j, p.max_pages - 1) * p.bts1];
    }
  };
  int phys0[LOGICAL ? 1 : kPagesPerThread];
  // Logical codes: block-table entries and the G heads' codes of pages
  // lb .. lb + 7 (indices clamped to the table; results past the range are
  // discarded).
  auto load_logical = [&](int lb, uint32_t (&cw)[G][8], int (&ph)[8]) {
    if (p.bts1 == 1 && (p.bts0 & 3) == 0 && (lb & 3) == 0 && (reinterpret_cast<uintptr_t>(p.bt) & 15) == 0 &&
        lb + 8 <= p.max_pages) {
      // 8 consecutive entries, 16-byte aligned: two 16-byte reads
      const int4* src = reinterpret_cast<const int4*>(p.bt + static_cast<int64_t>(b) * p.bts0 + lb);
      const int4 u0 = src[0], u1 = src[1];
      ph[0] = u0.x; ph[1] = u0.y; ph[2] = u0.z; ph[3] = u0.w;
      ph[4] = u1.x; ph[5] = u1.y; ph[6] = u1.z; ph[7] = u1.w;
    } else {
#pragma unroll
      for (int j = 0; j < 8; ++j) ph[j] = p.bt[b * p.bts0 + min(lb + j, p.max_pages - 1) * p.bts1];
    }
    const char* cb = static_cast<const char*>(p.lcodes);
    if (p.lvec && (lb & 7) == 0 && lb + 8 <= p.max_pages) {
      // 8 consecutive codes: one 8-, 16- or 32-byte read per head
#pragma unroll
      for (int g = 0; g < G; ++g) {
        const char* src = cb + (b * p.cs0 + (h0 + g) * p.cs1 + lb) * p.code_bytes;
        if (p.code_bytes == 1) {
          const uint2 a = *reinterpret_cast<const uint2*>(src);
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            cw[g][j] = (a.x >> (8 * j)) & 0xffu;
            cw[g][4 + j] = (a.y >> (8 * j)) & 0xffu;
          }
        } else if (p.code_bytes == 2) {
          const uint4 a = *reinterpret_cast<const uint4*>(src);
          const uint32_t w4[4] = {a.x, a.y, a.z, a.w};
#pragma unroll
          for (int j = 0; j < 8; ++j) cw[g][j] = (w4[j >> 1] >> (16 * (j & 1))) & 0xffffu;
        } else {
          const uint4 a = reinterpret_cast<const uint4*>(src)[0], c = reinterpret_cast<const uint4*>(src)[1];
          cw[g][0] = a.x; cw[g][1] = a.y; cw[g][2] = a.z; cw[g][3] = a.w;
          cw[g][4] = c.x; cw[g][5] = c.y; cw[g][6] = c.z; cw[g][7] = c.w;
        }
      }
    } else {
#pragma unroll
      for (int g = 0; g < G; ++g) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int64_t i = b * p.cs0 + (h0 + g) * p.cs1 + min(lb + j, p.max_pages - 1) * p.cs2;
          cw[g][j] = p.code_bytes == 1 ? static_cast<uint32_t>(reinterpret_cast<const uint8_t*>(cb)[i])
                   : p.code_bytes == 2 ? static_cast<uint32_t>(reinterpret_cast<const uint16_t*>(cb)[i])
                                       : reinterpret_cast<const uint32_t*>(cb)[i];
        }
      }
    }
  };
  uint32_t lcw0[LOGICAL ? G : 1][8];
  int lph0[8];
  if (prefetched) {
    if constexpr (LOGICAL) {
      load_logical(8 * tid, lcw0, lph0);
    } else {
      load_bt(kPagesPerThread * tid, phys0);
    }
  }
  const int ctx = p.ctx[b];
  int n = ctx > 0 ? (ctx + p.PS - 1) / p.PS : 0;
  if (n > p.max_pages) n = p.max_pages;  // block-table bound (memory safety)
  // This split's logical page range [pa, pz). Split boundaries are rounded
  // down to multiples of 8 pages, so that every range starts 16-byte aligned
  // in the block table and the code arrays (the vector reads below).
  const int pa = static_cast<int>((static_cast<long long>(n) * split) / p.splits) & ~7;
  const int pz = split + 1 == p.splits ? n
                                       : static_cast<int>((static_cast<long long>(n) * (split + 1)) / p.splits) & ~7;

  const int grp = lane >> 4, sub = lane & 15;
  constexpr int QW = RowRegs<T, DPL>::kWords;
  uint32_t qw[G][QW];  // this lane's D/16 query elements per head, raw
  // One vector read per head when the lane's D/16 elements are contiguous and aligned.
  constexpr int kQBytes = DPL * static_cast<int>(sizeof(T));
  constexpr int kQAlign = kQBytes >= 16 ? 16 : kQBytes;
  const bool qvec = p.qs2 == 1 && ((p.qs0 | p.qs1) * static_cast<int64_t>(sizeof(T))) % kQAlign == 0 &&
                    (reinterpret_cast<uintptr_t>(p.q) % kQAlign) == 0;
  float m_s[G], l_s[G], acc[G][DPL];
  // MFMA phase B state: Q^T operand (lane l: head l % 16, elements
  // 32 c + 8 (l / 16) .. +8), O^T tiles (lane l: head l % 16, d = 16 t + 4 (l / 16) + i),
  // the running maximum of head l % 16 and this lane's part of its sum.
  constexpr int KC = MB ? D / 32 : 1;
  constexpr int DT16 = MB ? D / 16 : 1;
  const int t16 = lane & 15, kg = lane >> 4;
  u32x4_t qop[KC];
  f32x4_t oacc[DT16];
  float mb_m = -INFINITY, mb_l = 0.f;
  if constexpr (MB) {
#pragma unroll
    for (int t = 0; t < DT16; ++t) oacc[t] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < KC; ++c) qop[c] = u32x4_t{0u, 0u, 0u, 0u};
    if (t16 < G) {
      const T* qp = static_cast<const T*>(p.q) + b * p.qs0 + (h0 + t16) * p.qs1;
      const bool qv16 = p.qs2 == 1 && ((p.qs0 | p.qs1) * 2) % 16 == 0 && (reinterpret_cast<uintptr_t>(p.q) & 15) == 0;
#pragma unroll
      for (int c = 0; c < KC; ++c) {
        const int d0 = 32 * c + 8 * kg;
        if (qv16) {
          qop[c] = *reinterpret_cast<const u32x4_t*>(qp + d0);
        } else {
          uint32_t w[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            w[e] = elem_bits<T>(qp + (d0 + 2 * e) * p.qs2) | (elem_bits<T>(qp + (d0 + 2 * e + 1) * p.qs2) << 16);
          }
          qop[c] = u32x4_t{w[0], w[1], w[2], w[3]};
        }
      }
    }
  }
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const T* qp = static_cast<const T*>(p.q) + b * p.qs0 + (h0 + g) * p.qs1 + sub * DPL * p.qs2;
#pragma unroll
    for (int i = 0; i < QW; ++i) qw[g][i] = 0u;
    if (MB) {
      // phase B reads qop
    } else if (qvec) {
      RowRegs<T, DPL> qr;
      load_row<T, DPL>(qp, qr);
#pragma unroll
      for (int i = 0; i < QW; ++i) qw[g][i] = qr.w[i];
    } else {
#pragma unroll
      for (int e = 0; e < DPL; ++e) {
        const uint32_t bits = elem_bits<T>(qp + e * p.qs2);
        if constexpr (sizeof(T) == 4) qw[g][e] = bits;
        else qw[g][e >> 1] |= bits << (16 * (e & 1));
      }
    }
#pragma unroll
    for (int e = 0; e < DPL; ++e) acc[g][e] = 0.f;
    m_s[g] = -INFINITY;
    l_s[g] = 0.f;
  }
  if constexpr (!LOGICAL) {
    if (prefetched) {
#pragma unroll
      for (int j = 0; j < kPagesPerThread; ++j) page_phys[kPagesPerThread * tid + j] = phys0[j];
    }
  }
  if constexpr (!PACKED && !LOGICAL) {   // the code modes carry no level-wise query router
    for (int i = tid; i < G * p.r; i += kDecThreads) {
      const int g = i / p.r, lev = i % p.r;
      qroute[g][lev] = p.qr[b * p.qrs0 + (h0 + g) * p.qrs1 + lev * p.qrs2];
    }
  }
  uint32_t qcode = 0u;
  if constexpr (PACKED) qcode = p.qcodes[b * p.qcs0 + (h0 + gl) * p.qcs1];
  uint32_t qc[LOGICAL ? G : 1];
  if constexpr (LOGICAL) {
#pragma unroll
    for (int g = 0; g < G; ++g) qc[g] = p.qcodes[b * p.qcs0 + (h0 + g) * p.qcs1];
  }
  // MFMA phase B, split 0: the forced pages need no routing, so up to one per
  // wave (the sink page, then the last pages of a sequence that fits the first
  // range) is loaded straight into LDS during phase A and folded in first;
  // phase A2 leaves them out. Wave 0 takes page 0 when it is the sink, the
  // next waves take pages n-1, n-2, ...
  const int e_lim = min(pz, kRange);
  const int e_s0 = (EARLY && prefetched && p.sink && n > 0 && e_lim > 0) ? 1 : 0;
  const int e_m0 = (EARLY && prefetched && n <= e_lim) ? min(p.local, kDecWaves - e_s0) : 0;
  const int e_lo = max(n - e_m0, e_s0);   // early local pages: [e_lo, n)
  auto is_early = [&](int l) { return (e_s0 && l == 0) || (l >= e_lo && l < n); };
  auto early_wave = [&](int l) { return (e_s0 && l == 0) ? 0 : e_s0 + (n - 1 - l); };
  int early_l = -1;
  if (e_s0 && wave == 0) early_l = 0;
  else if (wave >= e_s0 && n - 1 - (wave - e_s0) >= e_lo) early_l = n - 1 - (wave - e_s0);
  if constexpr (EARLY && LOGICAL) {
    if (prefetched) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int l = 8 * tid + j;
        if (l < e_lim && is_early(l)) early_phys[early_wave(l)] = lph0[j];
      }
    }
  }
  __syncthreads();
  if constexpr (EARLY) {
    if (early_l >= 0) {
      const int ph = LOGICAL ? early_phys[wave] : page_phys[early_l];
      if (ph >= 0 && ph < p.P) {
        constexpr int CPR = D / 8;
        constexpr int RSH = D == 128 ? 0 : (D == 64 ? 1 : 2);
        const int valid = min(p.PS, ctx - early_l * p.PS);
        const T* kpage = static_cast<const T*>(p.kc) + ph * p.ks0 + kvm * p.ks1;
        const T* vpage = static_cast<const T*>(p.vc) + ph * p.vs0 + kvm * p.vs1;
        const uint32_t kdst = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SA_LDS char*)kstage[wave]));
        const uint32_t vdst = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SA_LDS char*)vstage[wave]));
#pragma unroll
        for (int i = 0; i < KC; ++i) {
          // LDS chunk position 64 i + lane: row r, position pos; fetch the global chunk stored there
          const int pos_all = 64 * i + lane;
          const int r = pos_all / CPR, pos = pos_all % CPR;
          const int rr = min(r, valid - 1);
          const int kc = pos ^ (r & (CPR - 1));
          const int vc = 2 * ((pos >> 1) ^ ((r >> RSH) & (D / 16 - 1))) + (pos & 1);
          dma16(kpage + rr * p.ks2 + 8 * kc, __builtin_amdgcn_readfirstlane(kdst + 1024u * i));
          dma16(vpage + rr * p.vs2 + 8 * vc, __builtin_amdgcn_readfirstlane(vdst + 1024u * i));
        }
      } else {
        early_l = -1;   // not selected (the page id is out of range)
      }
    }
  }
  int qmine[4] = {0, 0, 0, 0};  // this lane's head's first four query levels (vector path)
  if constexpr (!PACKED && !LOGICAL) {
#pragma unroll
    for (int lev = 0; lev < 4; ++lev) qmine[lev] = lev < p.r ? qroute[gl][lev] : 0;
  }

  // Phase A's barriers order LDS traffic only: wait for this wave's LDS
  // accesses, then s_barrier (no fence, which would also wait for the early
  // pages' direct-to-LDS loads).
  auto lds_barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };
  for (int r0 = pa; r0 < pz; r0 += kRange) {
    const int r1 = min(pz, r0 + kRange);
    // ---- phase A1: block table + routing vectors -> per-page head mask ---------
    // All loads are unconditional (indices clamped into range) so they issue
    // back to back; out-of-range results are discarded afterwards.
    // The prefetched first range holds entries for pages past r1 as well:
    // their routing vectors are not loaded (and the pages are never selected).
    const bool use_pre = prefetched && r0 == 0;
    const int cnt = r1 - r0;
    int mm[kPagesPerThread];
    int phj[LOGICAL ? 8 : 1];
    if constexpr (LOGICAL) {
      uint32_t cw[G][8];
      int ph[8];
      if (use_pre) {
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          ph[j] = lph0[j];
#pragma unroll
          for (int g = 0; g < G; ++g) cw[g][j] = lcw0[g][j];
        }
      } else {
        load_logical(r0 + 8 * tid, cw, ph);
      }
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int l = r0 + 8 * tid + j;
        const bool valid = 8 * tid + j < cnt && ph[j] >= 0 && ph[j] < p.P;
        const bool forced = (p.sink && l == 0) || (p.local > 0 && l >= n - p.local);
        int m = 0;
#pragma unroll
        for (int g = 0; g < G; ++g) m |= (((cw[g][j] ^ qc[g]) & p.code_mask) == 0u) << g;
        mm[j] = valid ? (forced ? (1 << G) - 1 : m) : 0;
        phj[j] = ph[j];
      }
    } else {
    if (!use_pre) {
      // the range's block-table entries into LDS (the prologue did the first range's)
      int ph[kPagesPerThread];
      load_bt(r0 + kPagesPerThread * tid, ph);
#pragma unroll
      for (int j = 0; j < kPagesPerThread; ++j) page_phys[kPagesPerThread * tid + j] = ph[j];
      lds_barrier();
    }
    for (int hf = 0; hf < kHalves; ++hf) {
    const int hb = r0 + hf * kHalf;                  // first page of this half
    if (hb >= r1) break;
    int phys[kPasses];
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) phys[ps] = page_phys[hf * kHalf + ps * kPagesPerPass + pslot];
    bool hit[kPasses];
    if constexpr (PACKED) {
      // Packed codes: one 32-bit word per (page, head); the first r levels
      // agree iff the code bits under code_mask agree.
      uint32_t cv[kPasses];
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int ph = (phys[ps] >= 0 && phys[ps] < p.P) ? phys[ps] : 0;
        const bool need = hb + ps * kPagesPerPass + pslot < r1;
        cv[ps] = need ? p.codes[ph * p.cs0 + (h0 + gl) * p.cs1] : ~qcode;
      }
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) hit[ps] = ((cv[ps] ^ qcode) & p.code_mask) == 0u;
    } else {
    if (p.vec_router) {
      int4 rv[kPasses];
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int ph = (phys[ps] >= 0 && phys[ps] < p.P) ? phys[ps] : 0;
        const bool need = hb + ps * kPagesPerPass + pslot < r1;
        rv[ps] = need ? *reinterpret_cast<const int4*>(p.router + ph * p.rs0 + (h0 + gl) * p.rs1)
                      : int4{0, 0, 0, 0};
      }
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        bool ok = true;
        if (p.r > 0) ok = ok && rv[ps].x == qmine[0];
        if (p.r > 1) ok = ok && rv[ps].y == qmine[1];
        if (p.r > 2) ok = ok && rv[ps].z == qmine[2];
        if (p.r > 3) ok = ok && rv[ps].w == qmine[3];
        hit[ps] = ok;
      }
    } else {
#pragma unroll
      for (int ps = 0; ps < kPasses; ++ps) {
        const int ph = (phys[ps] >= 0 && phys[ps] < p.P) ? phys[ps] : 0;
        const int32_t* rv = p.router + ph * p.rs0 + (h0 + gl) * p.rs1;
        bool ok = hb + ps * kPagesPerPass + pslot < r1;
        for (int lev = 0; ok && lev < p.r; ++lev) {
          if (rv[lev * p.rs2] != qroute[gl][lev]) {
            ok = false;
            break;
          }
        }
        hit[ps] = ok;
      }
    }
    }
#pragma unroll
    for (int ps = 0; ps < kPasses; ++ps) {
      const int l = hb + ps * kPagesPerPass + pslot;
      const bool valid = l < r1 && phys[ps] >= 0 && phys[ps] < p.P;
      const bool forced = (p.sink && l == 0) || (p.local > 0 && l >= n - p.local);
      const uint64_t bal = __ballot(valid && (forced || hit[ps]));
      if (gl == 0) {
        const int m = static_cast<int>((bal >> (lane - gl)) & ((1u << G) - 1u));
        page_mask[hf * kHalf + ps * kPagesPerPass + pslot] = static_cast<uint8_t>(m);
      }
    }
    }   // halves
    lds_barrier();
#pragma unroll
    for (int j = 0; j < kPagesPerThread; ++j) {
      const int l = tid * kPagesPerThread + j;
      mm[j] = l < cnt ? page_mask[l] : 0;
    }
    }
    // ---- phase A2: compact selected pages in ascending logical order -----------
    if constexpr (MB) {
      if (r0 == pa && (e_s0 | e_m0)) {
#pragma unroll
        for (int j = 0; j < kPagesPerThread; ++j) {
          if (is_early(r0 + kPagesPerThread * tid + j)) mm[j] = 0;
        }
      }
    }
    int mine = 0;
#pragma unroll
    for (int j = 0; j < kPagesPerThread; ++j) mine += mm[j] != 0;
    int incl = mine;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(incl, off);
      if (lane >= off) incl += y;
    }
    if (lane == 63) wave_count[wave] = incl;
    lds_barrier();
    int pos = incl - mine, nsel = 0;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const int cw = wave_count[w];
      if (w < wave) pos += cw;
      nsel += cw;
    }
#pragma unroll
    for (int j = 0; j < kPagesPerThread; ++j) {
      if (mm[j] != 0) {
        const int l = tid * kPagesPerThread + j;
        if constexpr (LOGICAL) sel_phys[pos] = phj[j];
        else sel_phys[pos] = page_phys[l];
        sel_meta[pos] = l | (mm[j] << 16);
        ++pos;
      }
    }
    lds_barrier();

    // ---- phase B: gather + attend the selected pages ----------------------------
    // fetch() loads K and V rows of one page into a register buffer; attend()
    // folds a fetched page into the online softmax. Buffers are only ever
    // indexed by compile-time constants (so they stay in registers).
    using Rows = RowRegs<T, DPL>[4];
    auto fetch = [&](int i, int tc, Rows& kx, Rows& vx) {
      const int ph = sel_phys[i];
      const int lp = r0 + (sel_meta[i] & 0xffff);
      const int valid = min(p.PS, ctx - lp * p.PS);
      const T* kpage = static_cast<const T*>(p.kc) + ph * p.ks0 + kvm * p.ks1 + sub * DPL;
      const T* vpage = static_cast<const T*>(p.vc) + ph * p.vs0 + kvm * p.vs1 + sub * DPL;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int tok = min(tc + 4 * it + grp, valid - 1);   // masked rows reread a valid row
        load_row<T, DPL>(kpage + tok * p.ks2, kx[it]);
        load_row<T, DPL>(vpage + tok * p.vs2, vx[it]);
      }
    };
    auto attend = [&](int i, int tc, const Rows& kx, const Rows& vx) {
      const int lp = r0 + (sel_meta[i] & 0xffff);
      const int hmask = sel_meta[i] >> 16;
      const int valid = min(p.PS, ctx - lp * p.PS);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (!((hmask >> g) & 1)) continue;
        float s[4];
        float mloc = -INFINITY;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const float sc = row16_sum(row_dot<T, DPL>(qw[g], kx[it])) * p.qk_scale;
          s[it] = (tc + 4 * it + grp) < valid ? sc : -INFINITY;
          mloc = fmaxf(mloc, s[it]);
        }
        const float m_new = fmaxf(m_s[g], mloc);
        const float m_ref = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = fast_exp2(m_s[g] - m_ref);
        float lsum = l_s[g] * alpha;
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[g][e] *= alpha;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          const float pv = fast_exp2(s[it] - m_ref);
          lsum += pv;
#pragma unroll
          for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(pv, row_elem<T, DPL>(vx[it], e), acc[g][e]);
        }
        l_s[g] = lsum;
        m_s[g] = m_new;
      }
    };
    if constexpr (MB) {
      // MFMA phase B. A page's 16 token rows (rows past the context reread the
      // last valid row; their scores are masked, so p = 0): K in the A-operand
      // layout of the 16x16x32 product (lane l: token l % 16, elements
      // 32 c + 8 (l / 16) .. +8), V as consecutive 16-byte chunks (chunk
      // l + 64 j), written to the wave's LDS slot when the page is folded in.
      // A wave keeps kBufs pages in flight, as the VALU path below.
      constexpr int CPR = D / 8;                    // 16-byte chunks per row
      constexpr int RSH = D == 128 ? 0 : (D == 64 ? 1 : 2);   // log2(rows per 256 bytes)
      constexpr int kBufs = D == 128 ? 2 : 4;
      auto vunit = [](int r) { return (r >> RSH) & (D / 16 - 1); };
      char* vs = vstage[wave];
      // Folds logical page lp (heads in hmask) into the state: K operands in
      // kx; V rows in vx are first written to the wave's LDS slot when write_v
      // (the early page's V rows are already there).
      auto fold = [&](int lp, int hmask, const u32x4_t (&kx)[KC], const u32x4_t (&vx)[KC], bool write_v) {
        const int valid = min(p.PS, ctx - lp * p.PS);
        if (write_v) {
#pragma unroll
          for (int j = 0; j < KC; ++j) {
            const int ci = lane + 64 * j;
            const int row = ci / CPR, cc = ci % CPR;
            *reinterpret_cast<SA_LDS u32x4_t*>((SA_LDS char*)vs + row * 2 * D + 32 * ((cc >> 1) ^ vunit(row)) +
                                               16 * (cc & 1)) = vx[j];
          }
        }
        f32x4_t st = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int c = 0; c < KC; ++c) st = Mma16<T>::k32(kx[c], qop[c], st);
        const bool hsel = (hmask >> t16) & 1;   // lanes of heads >= G: bit clear
        float s[4];
        float mloc = -INFINITY;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          s[e] = (hsel && 4 * kg + e < valid) ? st[e] * p.qk_scale : -INFINITY;
          mloc = fmaxf(mloc, s[e]);
        }
        mloc = fmaxf(mloc, __shfl_xor(mloc, 16));
        mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
        // O is rescaled only when a head's maximum grows by more than 2^8.
        if (__any(mloc > mb_m + 8.f)) {
          const float m_new = fmaxf(mb_m, mloc);
          const float alpha = fast_exp2(mb_m - (m_new == -INFINITY ? 0.f : m_new));
          mb_l *= alpha;
#pragma unroll
          for (int t = 0; t < DT16; ++t) oacc[t] *= alpha;
          mb_m = m_new;
        }
        const float mref = mb_m == -INFINITY ? 0.f : mb_m;
        float pe[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          pe[e] = fast_exp2(s[e] - mref);
          mb_l += pe[e];
        }
        const u32x2_t pb{Mma16<T>::pack(pe[0], pe[1]), Mma16<T>::pack(pe[2], pe[3])};
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");   // this page's V rows are in LDS
        // lane l addresses row 4 (l / 16) + (l % 16) / 4, columns 16 t + 4 (l % 4) .. +3, and
        // receives column 16 t + l % 16 of rows 4 (l / 16) .. +3: V^T in the A layout.
        const int vr0 = 4 * kg + (t16 >> 2);
#pragma unroll
        for (int t = 0; t < DT16; ++t) {
          SA_LDS s16x4_t* a = (SA_LDS s16x4_t*)((SA_LDS char*)vs + vr0 * 2 * D + 32 * (t ^ vunit(vr0)) +
                                                8 * (t16 & 3));
          const u32x2_t va = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(a));
          oacc[t] = Mma16<T>::k16(va, pb, oacc[t]);
        }
      };
      if (EARLY && r0 == pa && early_l >= 0) {
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");   // the early page's direct-to-LDS loads
        u32x4_t kx[KC];
#pragma unroll
        for (int c = 0; c < KC; ++c) {
          kx[c] = *reinterpret_cast<SA_LDS u32x4_t*>((SA_LDS char*)kstage[wave] + t16 * 2 * D +
                                                     16 * ((4 * c + kg) ^ (t16 & (CPR - 1))));
        }
        fold(early_l, (1 << G) - 1, kx, kx, false);
      }
      if (wave < nsel) {
        const int last = wave + ((nsel - 1 - wave) / kDecWaves) * kDecWaves;
        u32x4_t kr[kBufs][KC], vr[kBufs][KC];
        auto fetch_mb = [&](int i, u32x4_t (&kx)[KC], u32x4_t (&vx)[KC]) {
          const int ph = sel_phys[i];
          const int lp = r0 + (sel_meta[i] & 0xffff);
          const int valid = min(p.PS, ctx - lp * p.PS);
          const T* kpage = static_cast<const T*>(p.kc) + ph * p.ks0 + kvm * p.ks1;
          const T* vpage = static_cast<const T*>(p.vc) + ph * p.vs0 + kvm * p.vs1;
          const int kt = min(t16, valid - 1);
#pragma unroll
          for (int c = 0; c < KC; ++c) {
            kx[c] = *reinterpret_cast<const u32x4_t*>(kpage + kt * p.ks2 + 32 * c + 8 * kg);
          }
#pragma unroll
          for (int j = 0; j < KC; ++j) {
            const int ci = lane + 64 * j;
            const int row = min(ci / CPR, valid - 1);
            vx[j] = *reinterpret_cast<const u32x4_t*>(vpage + row * p.vs2 + 8 * (ci % CPR));
          }
        };
        auto attend_mb = [&](int i, const u32x4_t (&kx)[KC], const u32x4_t (&vx)[KC]) {
          fold(r0 + (sel_meta[i] & 0xffff), sel_meta[i] >> 16, kx, vx, true);
        };
#pragma unroll
        for (int b2 = 0; b2 < kBufs - 1; ++b2) fetch_mb(min(wave + b2 * kDecWaves, last), kr[b2], vr[b2]);
        for (int base = wave; base <= last; base += kBufs * kDecWaves) {
#pragma unroll
          for (int b2 = 0; b2 < kBufs; ++b2) {
            const int i = base + b2 * kDecWaves;
            if (i > last) break;
            fetch_mb(min(i + (kBufs - 1) * kDecWaves, last), kr[(b2 + kBufs - 1) % kBufs],
                     vr[(b2 + kBufs - 1) % kBufs]);
            attend_mb(i, kr[b2], vr[b2]);
          }
        }
      }
    } else if (p.PS <= 16) {
      // Whole page per fetch. A wave keeps kDecBufs pages in flight: page
      // i + (kDecBufs-1)*waves is requested before page i is folded in.
      // Fetch indices past the end are clamped to the wave's last page (a
      // reread that hits cache), so every iteration issues the same loads and
      // the load counter waits stay static.
      // Pages in flight per wave: 3 when a page costs <= 16 registers per
      // lane (16-bit D <= 64, fp32 D <= 32), 2 up to 32 registers, else 1
      // (two resident workgroups per CU matter more than a deeper ring).
      constexpr int kDecBufs = 8 * QW <= 16 ? 3 : (8 * QW <= 32 ? 2 : 1);
      if (wave < nsel) {
        const int last = wave + ((nsel - 1 - wave) / kDecWaves) * kDecWaves;
        Rows kx[kDecBufs], vx[kDecBufs];
#pragma unroll
        for (int b2 = 0; b2 < kDecBufs - 1; ++b2) fetch(min(wave + b2 * kDecWaves, last), 0, kx[b2], vx[b2]);
        for (int base = wave; base <= last; base += kDecBufs * kDecWaves) {
#pragma unroll
          for (int b2 = 0; b2 < kDecBufs; ++b2) {
            const int i = base + b2 * kDecWaves;
            if (i > last) break;
            fetch(min(i + (kDecBufs - 1) * kDecWaves, last), 0, kx[(b2 + kDecBufs - 1) % kDecBufs],
                  vx[(b2 + kDecBufs - 1) % kDecBufs]);
            attend(i, 0, kx[b2], vx[b2]);
          }
        }
      }
    } else {
      // Larger pages: 16 tokens at a time, no cross-page prefetch.
      for (int i = wave; i < nsel; i += kDecWaves) {
        const int lp = r0 + (sel_meta[i] & 0xffff);
        const int valid = min(p.PS, ctx - lp * p.PS);
        for (int tc = 0; tc < valid; tc += 16) {
          Rows kx, vx;
          fetch(i, tc, kx, vx);
          attend(i, tc, kx, vx);
        }
      }
    }
    __syncthreads();  // sel_* is rewritten by the next range
  }

  // ---- merge lane groups, then waves ---------------------------------------------
  if constexpr (MB) {
    float lw = mb_l;
    lw += __shfl_xor(lw, 16);
    lw += __shfl_xor(lw, 32);
    if (t16 < G) {
      if (kg == 0) {
        red_m[wave][t16] = mb_m;
        red_l[wave][t16] = lw;
      }
#pragma unroll
      for (int t = 0; t < DT16; ++t) {
#pragma unroll
        for (int e = 0; e < 4; ++e) red_acc[wave][t16][16 * t + 4 * kg + e] = oacc[t][e];
      }
    }
  }
#pragma unroll
  for (int g = 0; g < (MB ? 0 : G); ++g) {
    float mw = fmaxf(m_s[g], __shfl_xor(m_s[g], 16));
    mw = fmaxf(mw, __shfl_xor(mw, 32));
    const float mref = mw == -INFINITY ? 0.f : mw;
    const float sc = fast_exp2(m_s[g] - mref);
    float lw = l_s[g] * sc;
    lw += __shfl_xor(lw, 16);
    lw += __shfl_xor(lw, 32);
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      float a = acc[g][e] * sc;
      a += __shfl_xor(a, 16);
      a += __shfl_xor(a, 32);
      acc[g][e] = a;
    }
    if (lane == 0) {
      red_m[wave][g] = mw;
      red_l[wave][g] = lw;
    }
    if (grp == 0) {
#pragma unroll
      for (int e = 0; e < DPL; ++e) red_acc[wave][g][sub * DPL + e] = acc[g][e];
    }
  }
  __syncthreads();
  for (int i = tid; i < G * D; i += kDecThreads) {
    const int g = i / D, d = i % D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) mx = fmaxf(mx, red_m[w][g]);
    const float mref = mx == -INFINITY ? 0.f : mx;
    float a = 0.f, lsum = 0.f;
#pragma unroll
    for (int w = 0; w < kDecWaves; ++w) {
      const float sc = fast_exp2(red_m[w][g] - mref);
      a += red_acc[w][g][d] * sc;
      lsum += red_l[w][g] * sc;
    }
    if (p.splits == 1) {
      T* op = static_cast<T*>(p.out) + b * p.os0 + (h0 + g) * p.os1;
      Elem<T>::store(op + d * p.os2, lsum > 0.f ? a / lsum : 0.f);
    } else {
      float* dst = p.part + ((static_cast<int64_t>(b) * p.H + h0 + g) * p.splits + split) * (D + 2);
      dst[2 + d] = a;
      if (d == 0) {
        dst[0] = mx;
        dst[1] = lsum;
      }
    }
  }
}

template <typename T>
__global__ __launch_bounds__(64) void decode_merge_kernel(DecParams p) {
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D;
  T* op = static_cast<T*>(p.out) + b * p.os0 + h * p.os1;
  const float* src = p.part + static_cast<int64_t>(bh) * p.splits * (D + 2);
  float mx = -INFINITY;
  for (int s = 0; s < p.splits; ++s) mx = fmaxf(mx, src[s * (D + 2)]);
  const float mref = mx == -INFINITY ? 0.f : mx;
  float lsum = 0.f;
  for (int s = 0; s < p.splits; ++s) lsum += src[s * (D + 2) + 1] * fast_exp2(src[s * (D + 2)] - mref);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float a = 0.f;
    for (int s = 0; s < p.splits; ++s) a += src[s * (D + 2) + 2 + d] * fast_exp2(src[s * (D + 2)] - mref);
    Elem<T>::store(op + d * p.os2, lsum > 0.f ? a / lsum : 0.f);
  }
}

template <typename T, int D, int MODE, bool MB>
void launch_dpm(DecParams& p, dim3 g, hipStream_t s) {
  switch (p.G) {
    case 1: hipLaunchKernelGGL((decode_kernel<T, D, 1, MODE, MB>), g, dim3(kDecThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((decode_kernel<T, D, 2, MODE, MB>), g, dim3(kDecThreads), 0, s, p); break;
    case 4: hipLaunchKernelGGL((decode_kernel<T, D, 4, MODE, MB>), g, dim3(kDecThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((decode_kernel<T, D, 8, MODE, MB>), g, dim3(kDecThreads), 0, s, p); break;
  }
}

template <typename T, int D, int MODE>
void launch_dp(DecParams& p, dim3 g, hipStream_t s) {
  if constexpr (sizeof(T) == 2 && (D == 32 || D == 64 || D == 128)) {
    if (p.mfma_b) {
      launch_dpm<T, D, MODE, true>(p, g, s);
      return;
    }
  }
  launch_dpm<T, D, MODE, false>(p, g, s);
}

template <typename T, int D>
void launch_d(DecParams& p, dim3 g, hipStream_t s) {
  if (p.codes && p.logical) launch_dp<T, D, 2>(p, g, s);
  else if (p.codes) launch_dp<T, D, 1>(p, g, s);
  else launch_dp<T, D, 0>(p, g, s);
}

template <typename T>
int launch_decode(DecParams& p, hipStream_t s) {
  const long long wg = static_cast<long long>(p.B) * p.Hkv * p.splits;
  if (wg > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  dim3 g(static_cast<unsigned>(wg));
  switch (p.D) {
    case 16: launch_d<T, 16>(p, g, s); break;
    case 32: launch_d<T, 32>(p, g, s); break;
    case 64: launch_d<T, 64>(p, g, s); break;
    case 128: launch_d<T, 128>(p, g, s); break;
    default: launch_d<T, 256>(p, g, s); break;
  }
  int rc = check_launch("sparse paged decode kernel");
  if (rc != SA_OK || p.splits == 1) return rc;
  hipLaunchKernelGGL((decode_merge_kernel<T>), dim3(p.B * p.H), dim3(64), 0, s, p);
  return check_launch("sparse paged decode merge kernel");
}

// Splits per (sequence, kv head): enough workgroups to fill the GPU, never
// more than one per 256 pages.
int splits_for(int B, int H_kv, int max_pages) {
  const long long pairs = static_cast<long long>(B) * H_kv;
  if (pairs <= 0) return 1;
  long long s = (kTargetWorkgroups + pairs - 1) / pairs;
  const long long cap = max_pages <= 0 ? 1 : (max_pages + 255) / 256;
  if (s > cap) s = cap;
  return static_cast<int>(s < 1 ? 1 : s);
}

}  // namespace
}  // namespace sa

namespace sa {
namespace {
// Work items per sequence: the kv heads when the group size G = H / H_kv has a
// kernel (1, 2, 4, 8; one item serves the G query heads of a kv head), else the
// query heads (G = 1 items, each reading kv head h / G).
bool group_has_kernel(int G) { return G == 1 || G == 2 || G == 4 || G == 8; }
int grid_kv_heads(int H, int H_kv) { return group_has_kernel(H / H_kv) ? H_kv : H; }
}  // namespace
}  // namespace sa

extern "C" size_t sa_decode_workspace_bytes(int B, int H, int H_kv, int D, int max_pages) {
  if (B <= 0 || H <= 0 || H_kv <= 0 || D <= 0 || H % H_kv != 0) return 0;
  const int splits = sa::splits_for(B, sa::grid_kv_heads(H, H_kv), max_pages);
  if (splits == 1) return 0;
  return static_cast<size_t>(B) * H * splits * (D + 2) * sizeof(float);
}

namespace sa {
namespace {

// Shared by the two decode entry points: router / q_router (int32 levels) or
// codes / qcodes (packed words, bpl bits per level, level 0 highest).
int decode_impl(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
                const int32_t* context_lens, const int32_t* router, const int32_t* q_router,
                const uint32_t* codes, const uint32_t* qcodes, int bpl, int logical, void* out, int B,
                int H, int H_kv,
                int D, int page_size, int TD, int max_pages, int num_phys_pages, int req_depth,
                int local_blocks, int sink_block, const int64_t* q_strides, const int64_t* k_strides,
                const int64_t* v_strides, const int64_t* bt_strides, const int64_t* r_strides,
                const int64_t* qr_strides, const int64_t* o_strides, void* workspace,
                size_t workspace_bytes, int dtype, void* stream) {
  using namespace sa;
  if (B < 0 || H < 0 || H_kv <= 0 || (H > 0 && H % H_kv != 0)) return fail(SA_EINVAL, "bad B/H/H_kv");
  const int G_real = H > 0 ? H / H_kv : 1;
  // Group sizes without a kernel run one work item per query head (G = 1).
  const int G = group_has_kernel(G_real) ? G_real : 1;
  if (!is_pow2(D) || D < 16 || D > 256) {
    return fail(SA_EUNSUPPORTED, "head_dim must be a power of two in [16, 256]");
  }
  if (page_size < 1) return fail(SA_EINVAL, "page size must be >= 1");
  if (TD < 1) return fail(SA_EINVAL, "tree depth must be >= 1");
  if (TD > kMaxTD) return fail(SA_EUNSUPPORTED, "tree depth > 64 is not supported");
  if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16) {
    return fail(SA_EINVAL, "dtype must be f32, bf16 or f16");
  }
  if (max_pages < 0 || num_phys_pages < 0) return fail(SA_EINVAL, "negative page counts");
  if (static_cast<long long>(B) * H == 0) return SA_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !out ||
      (codes ? (!qcodes) : (!router || !q_router))) {
    return fail(SA_EINVAL, "NULL tensor argument");
  }
  if (!q_strides || !k_strides || !v_strides || !bt_strides || !r_strides || !qr_strides || !o_strides) {
    return fail(SA_EINVAL, "NULL strides");
  }
  if (k_strides[3] != 1 || v_strides[3] != 1) {
    return fail(SA_EUNSUPPORTED, "k_cache / v_cache need unit stride along head_dim");
  }
  // Each lane loads D/16 consecutive elements with vector loads of up to 16
  // bytes, so rows and base pointers must be aligned to that size.
  const int64_t esize = dtype == SA_DTYPE_F32 ? 4 : 2;
  int64_t align = (D / 16) * esize;
  if (align > 16) align = 16;
  for (int i = 0; i < 3; ++i) {
    if ((k_strides[i] * esize) % align != 0 || (v_strides[i] * esize) % align != 0) {
      return fail(SA_EUNSUPPORTED, "k_cache / v_cache strides break vector alignment");
    }
  }
  if (reinterpret_cast<uintptr_t>(k_cache) % align != 0 ||
      reinterpret_cast<uintptr_t>(v_cache) % align != 0) {
    return fail(SA_EUNSUPPORTED, "k_cache / v_cache base pointers break vector alignment");
  }
  const size_t need = sa_decode_workspace_bytes(B, H, H_kv, D, max_pages);
  if (need > 0 && (!workspace || workspace_bytes < need)) {
    return fail(SA_EINVAL, "workspace too small: need " + std::to_string(need) + " bytes");
  }

  DecParams p{};
  p.q = q; p.kc = k_cache; p.vc = v_cache; p.bt = block_tables; p.ctx = context_lens;
  p.router = router; p.qr = q_router; p.out = out; p.part = static_cast<float*>(workspace);
  p.B = B; p.H = H; p.Hkv = grid_kv_heads(H, H_kv); p.D = D; p.PS = page_size; p.TD = TD;
  p.kvdiv = group_has_kernel(G_real) ? 1 : G_real;
  p.max_pages = max_pages; p.P = num_phys_pages;
  p.r = req_depth < 0 ? 0 : (req_depth > TD ? TD : req_depth);
  p.local = local_blocks; p.sink = sink_block != 0; p.G = G;
  p.splits = splits_for(B, p.Hkv, max_pages);
  if (codes) {
    p.codes = codes;
    p.qcodes = qcodes;
    p.logical = logical;
    p.cs0 = r_strides[0]; p.cs1 = r_strides[1];
    if (logical) {
      p.cs2 = r_strides[2];
      p.code_bytes = logical;
      p.lcodes = codes;
      // 8 codes per thread with one aligned read: rows and base aligned to 8 codes
      const int64_t al = 8 * logical >= 16 ? 16 / logical : 8;
      p.lvec = p.cs2 == 1 && p.cs0 % al == 0 && p.cs1 % al == 0 &&
               (reinterpret_cast<uintptr_t>(codes) % static_cast<uintptr_t>(al * logical)) == 0;
    }
    p.qcs0 = qr_strides[0]; p.qcs1 = qr_strides[1];
    const int shift = bpl * (TD - p.r);
    p.code_mask = p.r == 0 ? 0u : (shift >= 32 ? 0u : (0xFFFFFFFFu << shift));
  } else {
    p.vec_router = r_strides[2] == 1 && TD >= 4 && p.r <= 4 && r_strides[0] % 4 == 0 &&
                   r_strides[1] % 4 == 0 && (reinterpret_cast<uintptr_t>(router) & 15) == 0;
  }
  p.qs0 = q_strides[0]; p.qs1 = q_strides[1]; p.qs2 = q_strides[2];
  p.ks0 = k_strides[0]; p.ks1 = k_strides[1]; p.ks2 = k_strides[2];
  p.vs0 = v_strides[0]; p.vs1 = v_strides[1]; p.vs2 = v_strides[2];
  p.bts0 = bt_strides[0]; p.bts1 = bt_strides[1];
  if (!codes) {
    p.rs0 = r_strides[0]; p.rs1 = r_strides[1]; p.rs2 = r_strides[2];
    p.qrs0 = qr_strides[0]; p.qrs1 = qr_strides[1]; p.qrs2 = qr_strides[2];
  }
  p.os0 = o_strides[0]; p.os1 = o_strides[1]; p.os2 = o_strides[2];
  p.qk_scale = (1.0f / sqrtf(static_cast<float>(D))) * kLog2e;
  // MFMA phase B: 16-bit K / V, D in {32, 64, 128}, pages of at most 16
  // tokens, 16-byte aligned K / V rows (one 16-byte load per lane and row chunk).
  bool kv16 = (reinterpret_cast<uintptr_t>(k_cache) & 15) == 0 && (reinterpret_cast<uintptr_t>(v_cache) & 15) == 0;
  for (int i = 0; i < 3; ++i) kv16 = kv16 && (k_strides[i] * esize) % 16 == 0 && (v_strides[i] * esize) % 16 == 0;
  p.mfma_b = dtype != SA_DTYPE_F32 && (D == 32 || D == 64 || D == 128) && page_size <= 16 && kv16;
  hipStream_t s = as_stream(stream);
  if (dtype == SA_DTYPE_F32) return launch_decode<float>(p, s);
  if (dtype == SA_DTYPE_BF16) return launch_decode<bf16_t>(p, s);
  return launch_decode<f16_t>(p, s);
}

// Packs (rows, H, TD) int32 routing levels into one word per (row, head):
// level l occupies bits [bpl (TD-1-l), bpl (TD-l)), so level 0 is highest and
// a prefix of r levels is the top bpl r bits.
__global__ __launch_bounds__(256) void pack_codes_kernel(const int32_t* r, int64_t s0, int64_t s1, int64_t s2,
                                                          int rows, int H, int TD, int bpl, uint32_t* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  if (i >= static_cast<int64_t>(rows) * H) return;
  const int row = static_cast<int>(i / H), h = static_cast<int>(i % H);
  const uint32_t m = bpl >= 32 ? 0xFFFFFFFFu : ((1u << bpl) - 1u);
  uint32_t c = 0;
  for (int l = 0; l < TD; ++l) c = (c << bpl) | (static_cast<uint32_t>(r[row * s0 + h * s1 + l * s2]) & m);
  out[i] = c;
}

}  // namespace
}  // namespace sa

extern "C" int sa_sparse_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                                      const int32_t* block_tables, const int32_t* context_lens,
                                      const int32_t* router, const int32_t* q_router, void* out,
                                      int B, int H, int H_kv, int D, int page_size, int TD,
                                      int max_pages, int num_phys_pages, int req_depth,
                                      int local_blocks, int sink_block, const int64_t* q_strides,
                                      const int64_t* k_strides, const int64_t* v_strides,
                                      const int64_t* bt_strides, const int64_t* r_strides,
                                      const int64_t* qr_strides, const int64_t* o_strides,
                                      void* workspace, size_t workspace_bytes, int dtype,
                                      void* stream) {
  return sa::decode_impl(q, k_cache, v_cache, block_tables, context_lens, router, q_router, nullptr, nullptr, 0, 0,
                         out, B, H, H_kv, D, page_size, TD, max_pages, num_phys_pages, req_depth, local_blocks,
                         sink_block, q_strides, k_strides, v_strides, bt_strides, r_strides, qr_strides,
                         o_strides, workspace, workspace_bytes, dtype, stream);
}

extern "C" int sa_sparse_paged_decode_codes(const void* q, const void* k_cache, const void* v_cache,
                                            const int32_t* block_tables, const int32_t* context_lens,
                                            const uint32_t* page_codes, const uint32_t* q_codes, void* out,
                                            int B, int H, int H_kv, int D, int page_size, int TD,
                                            int bits_per_level, int max_pages, int num_phys_pages,
                                            int req_depth, int local_blocks, int sink_block,
                                            const int64_t* q_strides, const int64_t* k_strides,
                                            const int64_t* v_strides, const int64_t* bt_strides,
                                            const int64_t* pc_strides, const int64_t* qc_strides,
                                            const int64_t* o_strides, void* workspace,
                                            size_t workspace_bytes, int dtype, void* stream) {
  using namespace sa;
  if (bits_per_level < 1 || bits_per_level > 16) return fail(SA_EINVAL, "bits_per_level must lie in [1, 16]");
  if (TD < 1 || static_cast<long long>(TD) * bits_per_level > 32) {
    return fail(SA_EINVAL, "tree depth x bits_per_level must be in [1, 32]");
  }
  if (!pc_strides || !qc_strides) return fail(SA_EINVAL, "NULL strides");
  return decode_impl(q, k_cache, v_cache, block_tables, context_lens, nullptr, nullptr, page_codes, q_codes,
                     bits_per_level, 0, out, B, H, H_kv, D, page_size, TD, max_pages, num_phys_pages, req_depth,
                     local_blocks, sink_block, q_strides, k_strides, v_strides, bt_strides, pc_strides,
                     qc_strides, o_strides, workspace, workspace_bytes, dtype, stream);
}

extern "C" int sa_sparse_paged_decode_seq_codes(const void* q, const void* k_cache, const void* v_cache,
                                                const int32_t* block_tables, const int32_t* context_lens,
                                                const void* seq_codes, int code_bytes, const uint32_t* q_codes,
                                                void* out,
                                                int B, int H, int H_kv, int D, int page_size, int TD,
                                                int bits_per_level, int max_pages, int num_phys_pages,
                                                int req_depth, int local_blocks, int sink_block,
                                                const int64_t* q_strides, const int64_t* k_strides,
                                                const int64_t* v_strides, const int64_t* bt_strides,
                                                const int64_t* sc_strides, const int64_t* qc_strides,
                                                const int64_t* o_strides, void* workspace,
                                                size_t workspace_bytes, int dtype, void* stream) {
  using namespace sa;
  if (bits_per_level < 1 || bits_per_level > 16) return fail(SA_EINVAL, "bits_per_level must lie in [1, 16]");
  if (TD < 1 || static_cast<long long>(TD) * bits_per_level > 32) {
    return fail(SA_EINVAL, "tree depth x bits_per_level must be in [1, 32]");
  }
  if (!sc_strides || !qc_strides) return fail(SA_EINVAL, "NULL strides");
  if (code_bytes != 1 && code_bytes != 2 && code_bytes != 4) return fail(SA_EINVAL, "code_bytes must be 1, 2 or 4");
  if (static_cast<long long>(TD) * bits_per_level > 8 * code_bytes) {
    return fail(SA_EINVAL, "tree depth x bits_per_level exceeds the code width");
  }
  return decode_impl(q, k_cache, v_cache, block_tables, context_lens, nullptr, nullptr,
                     static_cast<const uint32_t*>(seq_codes), q_codes, bits_per_level, code_bytes, out, B, H, H_kv, D, page_size, TD, max_pages, num_phys_pages, req_depth,
                     local_blocks, sink_block, q_strides, k_strides, v_strides, bt_strides, sc_strides,
                     qc_strides, o_strides, workspace, workspace_bytes, dtype, stream);
}

extern "C" int sa_pack_page_codes(const int32_t* router, const int64_t* strides, int rows, int H, int TD,
                                  int bits_per_level, uint32_t* codes, void* stream) {
  using namespace sa;
  if (rows < 0 || H < 0 || TD < 1) return fail(SA_EINVAL, "bad rows/H/TD");
  if (bits_per_level < 1 || bits_per_level > 16 || static_cast<long long>(TD) * bits_per_level > 32) {
    return fail(SA_EINVAL, "need 1 <= bits_per_level <= 16 and tree depth x bits_per_level <= 32");
  }
  const long long n = static_cast<long long>(rows) * H;
  if (n == 0) return SA_OK;
  if (!router || !strides || !codes) return fail(SA_EINVAL, "NULL argument");
  const long long g = (n + 255) / 256;
  if (g > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  hipLaunchKernelGGL(pack_codes_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, as_stream(stream), router,
                     strides[0], strides[1], strides[2], rows, H, TD, bits_per_level, codes);
  return check_launch("page-code packing kernel");
}

// ---- no-allocation decode: split-KV partials in a file-scope device array ------
// One array per GPU, held until the process ends. Host code never passes the
// array's name to a kernel (in host code it is a stand-in, not a device
// address): the address each device gives for it is looked up once, with that
// device current, and kept per device.
namespace sa {
namespace {
constexpr size_t kNoAllocScratchBytes = static_cast<size_t>(8) << 20;   // every D <= 128 case fits
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace
}  // namespace sa

static __device__ __align__(256) unsigned char scratch[sa::kNoAllocScratchBytes];

namespace sa {
namespace {
// Device address of `scratch` on the current device (looked up on the first call there).
int scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(SA_ELAUNCH, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(SA_EUNSUPPORTED, "device index beyond the scratch table");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
      return fail(SA_ELAUNCH, std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    }
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return SA_OK;
}
}  // namespace
}  // namespace sa

extern "C" size_t sa_noalloc_scratch_bytes(void) { return sa::kNoAllocScratchBytes; }

extern "C" int sa_sparse_paged_decode_seq_codes_noalloc(
    const void* q, const void* k_cache, const void* v_cache, const int32_t* block_tables,
    const int32_t* context_lens, const void* seq_codes, int code_bytes, const uint32_t* q_codes, void* out, int B,
    int H, int H_kv, int D, int page_size, int TD, int bits_per_level, int max_pages, int num_phys_pages,
    int req_depth, int local_blocks, int sink_block, const int64_t* q_strides, const int64_t* k_strides,
    const int64_t* v_strides, const int64_t* bt_strides, const int64_t* sc_strides, const int64_t* qc_strides,
    const int64_t* o_strides, int dtype, void* stream) {
  using namespace sa;
  const size_t need = sa_decode_workspace_bytes(B, H, H_kv, D, max_pages);
  if (need > kNoAllocScratchBytes) {
    return fail(SA_EINVAL, "split-KV partials need " + std::to_string(need) + " bytes, more than the " +
                               std::to_string(kNoAllocScratchBytes) + " of the no-allocation scratch");
  }
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_on_current_device(&ws);
    if (rc != SA_OK) return rc;
  }
  return sa_sparse_paged_decode_seq_codes(q, k_cache, v_cache, block_tables, context_lens, seq_codes, code_bytes,
                                          q_codes, out, B, H, H_kv, D, page_size, TD, bits_per_level, max_pages,
                                          num_phys_pages, req_depth, local_blocks, sink_block, q_strides,
                                          k_strides, v_strides, bt_strides, sc_strides, qc_strides, o_strides, ws,
                                          need > 0 ? kNoAllocScratchBytes : 0, dtype, stream);
}
