// Block-sparse attention forward over block lists (gfx950).
//
// Semantics follow _block_list_fwd_kernel (src/ultrametric/block_list.py:387-470):
// for each query row, scores s = q.k * sm_scale (+ soft bias of the listed
// block) over the keys of the row's listed key blocks only, token-level
// causal / tail masking, base-2 online softmax with the all-masked guard
// (m_ref = 0 while every score seen is -inf), out = acc / l (0 when l == 0),
// lse = (m + log2 l) * ln2 (-inf when l == 0). P is rounded to the input
// element type before the PV product, as the reference does (p.to(v.dtype)).
//
// Two kernels:
//  * prefill_mfma_kernel — bf16/fp16, D in {32, 64, 128, 256}, route_block % 32 == 0.
//    A workgroup of NW waves owns BM = 32*NW query rows of one route block;
//    Q stays in registers as MFMA operands. Each wave computes S^T = K Q^T on
//    32x32x16 MFMA tiles, so lane (i + 32h) holds 16 keys of query i per
//    tile: row max / row sum need one exchange with lane ^ 32
//    (permlane32_swap), and the O^T = V^T P^T accumulator is rescaled with a
//    per-lane scalar, lazily (only when a row max grows by more than 2^8).
//    K/V tiles of BN = 32 keys stream through a 3-stage LDS ring filled by
//    direct-to-LDS loads (global_load_lds_dwordx4, no VGPR staging); rows
//    are stored with an XOR swizzle on 16-byte chunks, K is read as
//    row-major 16-byte MFMA operands and V through ds_read_b64_tr_b16
//    (transposing reads), both bank-conflict free. Workgroup ids are
//    remapped so that each XCD works on a contiguous range of heads (shared
//    K/V blocks hit that XCD's L2).
//  * prefill_generic_kernel — any of fp32/bf16/fp16, D power of two in
//    [16, 256], any route block: 16 lanes per query row, fp32 FMA math, used
//    for fp32 inputs (true fp32, no TF32 shortcut) and shapes the MFMA path
//    does not cover.
#include "mfma_util.h"

#include <algorithm>
#include <type_traits>

namespace sa {
namespace {

struct FwdParams {
  const void* q;
  const void* k;
  const void* v;
  void* out;
  float* lse;
  const int32_t* lists;
  const int32_t* counts;
  const void* sb;
  int sb_dtype;
  int64_t sbs0, sbs1, sbs2, sbs3;
  int64_t qs0, qs1, qs2, qs3;
  int64_t ks0, ks1, ks2, ks3;
  int64_t vs0, vs1, vs2, vs3;
  int64_t os0, os1, os2, os3;
  int Z, H, Hkv, N, RB, NB, max_count, group;
  float qk_scale;  // sm_scale * log2(e)
  int is_causal;
  int mtiles;      // query tiles per (z, h)
  int total_wg;
  int hgroup;      // MFMA kernel: heads whose query tiles are dealt together, longest first
  // Fused list build (sa_routed_block_sparse_fwd): routing ids -> each row's
  // list in the kernel, written back to lists_out / counts_out.
  const void* router;
  int64_t rs0, rs1, rs2, rs3;
  int router_i64, TD, depth_uniform, sink, local;
  const int64_t* depth_dev;
  uint64_t base;
  int32_t* lists_out;
  int32_t* counts_out;
};

__device__ __forceinline__ float load_bias(const FwdParams& p, int z, int h, int qb, int t) {
  const int64_t off = z * p.sbs0 + h * p.sbs1 + qb * p.sbs2 + t * p.sbs3;
  if (p.sb_dtype == SA_DTYPE_F32) return static_cast<const float*>(p.sb)[off] * kLog2e;
  if (p.sb_dtype == SA_DTYPE_BF16)
    return Elem<bf16_t>::load(static_cast<const bf16_t*>(p.sb) + off) * kLog2e;
  return Elem<f16_t>::load(static_cast<const f16_t*>(p.sb) + off) * kLog2e;
}

// Round p to the element type of V, as the reference's p.to(v.dtype).
template <typename T> __device__ __forceinline__ float round_to(float x);
template <> __device__ __forceinline__ float round_to<float>(float x) { return x; }
template <> __device__ __forceinline__ float round_to<bf16_t>(float x) {
  return bf16_bits_to_float(float_to_bf16_bits(x));
}
template <> __device__ __forceinline__ float round_to<f16_t>(float x) {
  return f16_bits_to_float(float_to_f16_bits(x));
}

constexpr int kListSeg = 256;  // MFMA path: list entries staged in LDS at a time

// ============================================================================
// Generic kernel: 16 query rows per workgroup, 16 lanes per row.
// ============================================================================
template <typename T, int D>
__global__ __launch_bounds__(256) void prefill_generic_kernel(FwdParams p) {
  constexpr int BMG = 16, BNG = 16, DPL = D / 16;
  __shared__ float ks[BNG][D];
  __shared__ float vs[BNG][D];

  const int work = xcd_remap(blockIdx.x, p.total_wg);
  const int zh = work / p.mtiles;
  const int mt = p.mtiles - 1 - work % p.mtiles;
  const int z = zh / p.H, h = zh % p.H, kvh = h / p.group;
  const int tid = threadIdx.x;
  const int qi = tid / 16, sub = tid % 16;
  const int m0 = mt * BMG;
  const int qpos = m0 + qi;
  const bool qvalid = qpos < p.N;
  const int qb = m0 / p.RB;
  const int64_t row = static_cast<int64_t>(zh) * p.NB + qb;
  const int count = min(max(p.counts[row], 0), p.max_count);
  const int32_t* list = p.lists + row * p.max_count;

  const T* qp = static_cast<const T*>(p.q) + z * p.qs0 + h * p.qs1;
  const T* kp = static_cast<const T*>(p.k) + z * p.ks0 + kvh * p.ks1;
  const T* vp = static_cast<const T*>(p.v) + z * p.vs0 + kvh * p.vs1;

  float qv[DPL], acc[DPL];
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = e * 16 + sub;
    qv[e] = qvalid ? Elem<T>::load(qp + qpos * p.qs2 + d * p.qs3) : 0.f;
    acc[e] = 0.f;
  }
  float m_i = -INFINITY, l_i = 0.f;
  const int q_last = m0 + BMG - 1;

  for (int t = 0; t < count; ++t) {
    const int kb = list[t];
    const float bias = p.sb ? load_bias(p, z, h, qb, t) : 0.f;
    for (int s0 = 0; s0 < p.RB; s0 += BNG) {
      const int key0 = kb * p.RB + s0;
      if (static_cast<unsigned>(key0) >= static_cast<unsigned>(p.N)) break;
      if (p.is_causal && key0 > q_last) break;  // every later key is masked too
      __syncthreads();
      for (int idx = tid; idx < BNG * D; idx += 256) {
        const int j = idx / D, d = idx % D, key = key0 + j;
        const bool kv_ok = static_cast<unsigned>(key) < static_cast<unsigned>(p.N);
        ks[j][d] = kv_ok ? Elem<T>::load(kp + key * p.ks2 + d * p.ks3) : 0.f;
        vs[j][d] = kv_ok ? Elem<T>::load(vp + key * p.vs2 + d * p.vs3) : 0.f;
      }
      __syncthreads();
      float sc[BNG];
      float mloc = -INFINITY;
#pragma unroll
      for (int j = 0; j < BNG; ++j) {
        float part = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) part = fmaf(qv[e], ks[j][e * 16 + sub], part);
        float s = row16_sum(part) * p.qk_scale + bias;
        const int key = key0 + j;
        const bool keep = static_cast<unsigned>(key) < static_cast<unsigned>(p.N) &&
                          (!p.is_causal || key <= qpos);
        s = keep ? s : -INFINITY;
        sc[j] = s;
        mloc = fmaxf(mloc, s);
      }
      const float m_new = fmaxf(m_i, mloc);
      const float m_ref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = fast_exp2(m_i - m_ref);
      l_i *= alpha;
#pragma unroll
      for (int e = 0; e < DPL; ++e) acc[e] *= alpha;
#pragma unroll
      for (int j = 0; j < BNG; ++j) {
        const float pj = fast_exp2(sc[j] - m_ref);
        l_i += pj;
        const float pr = round_to<T>(pj);
#pragma unroll
        for (int e = 0; e < DPL; ++e) acc[e] = fmaf(pr, vs[j][e * 16 + sub], acc[e]);
      }
      m_i = m_new;
    }
  }

  if (qvalid) {
    const float l_safe = l_i == 0.f ? 1.f : l_i;
    T* op = static_cast<T*>(p.out) + z * p.os0 + h * p.os1 + qpos * p.os2;
#pragma unroll
    for (int e = 0; e < DPL; ++e) Elem<T>::store(op + (e * 16 + sub) * p.os3, acc[e] / l_safe);
    if (p.lse && sub == 0) p.lse[static_cast<int64_t>(zh) * p.N + qpos] = (m_i + fast_log2(l_i)) * kLn2;
  }
}

// ============================================================================
// MFMA kernel (bf16 / fp16).
// ============================================================================

// S: pipeline stages (K+V tiles of BN keys; S - 1 in flight while one is
// computed). WPE: waves per SIMD the register budget is sized for.
// FUSED: the row's block list is built in the kernel from the routing ids
// (sync-free, code matching, NB <= 64 NW) instead of read from p.lists.
template <typename T, int D, int NW, bool CAUSAL, int S, int WPE, bool FUSED>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(WPE)))
void prefill_mfma_kernel(FwdParams p) {
  constexpr int BN = 32;               // keys per pipeline stage
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 32;
  constexpr int CPR = D / 8;           // 16-byte chunks per row
  constexpr int ROWB = D * 2;          // bytes per K / V row
  constexpr int TILEB = BN * ROWB;     // one K (or V) tile
  constexpr int STAGEB = 2 * TILEB;    // K tile, then V tile
  constexpr int KS = D / 16;           // MFMA k-steps of S^T = K Q^T
  constexpr int DT = D / 32;           // 32-row O^T tiles
  constexpr int NKI = TILEB / 1024;    // 1-KB direct-to-LDS loads per K tile
  constexpr int LPW = 2 * NKI / NW;    // loads per wave per stage (K and V)
  constexpr int RSH = D >= 128 ? 0 : (D == 64 ? 1 : 2);  // log2(rows per 256 B), 0 for rows of 256 B or more
  static_assert((2 * NKI) % NW == 0, "loads must split evenly over waves");
  static_assert(S >= 3 && S <= 4, "pipeline stages");
  // O is rescaled only when a row maximum grows by more than this (log2
  // units); until then p = exp2(s - m_ref) <= 2^8.
  constexpr float kRescale = 8.f;

  __shared__ __attribute__((aligned(1024))) char stage_lds[S * STAGEB];
  __shared__ int32_t list_lds[kListSeg];
  __shared__ float bias_lds[kListSeg];
  __shared__ int32_t wave_hits[NW];

  const int work = xcd_remap(blockIdx.x, p.total_wg);
  // Work order within an XCD's range: groups of hgroup heads, query tiles
  // dealt longest (last) first across the group's heads. hgroup = 1 keeps a
  // head's K / V together in L2 (sparse lists); with long lists the dispatch
  // tail matters more and the host deals four heads together.
  int zh, mt;
  if (p.hgroup <= 1) {
    zh = work / p.mtiles;
    mt = p.mtiles - 1 - work % p.mtiles;
  } else {
    const int grp = work / (p.hgroup * p.mtiles), gi = work % (p.hgroup * p.mtiles);
    const int in_grp = min(p.hgroup, p.Z * p.H - grp * p.hgroup);
    zh = grp * p.hgroup + gi % in_grp;
    mt = p.mtiles - 1 - gi / in_grp;
  }
  const int z = zh / p.H, h = zh % p.H, kvh = h / p.group;
  const int m0 = mt * BM;
  const int qb = m0 / p.RB;
  const int64_t row = static_cast<int64_t>(zh) * p.NB + qb;
  int count = FUSED ? 0 : min(max(p.counts[row], 0), p.max_count);
  const int32_t* list = p.lists + row * p.max_count;
  const int spb = p.RB / BN;
  const int lspb = __builtin_ctz(spb);   // spb = route_block / 32 is a power of two

  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63;
  const int li = lane & 31, kh = lane >> 5;
  const int qw0 = m0 + wave * 32;
  const int qpos = qw0 + li;
  const int N = p.N;

  const char* qbase = reinterpret_cast<const char*>(static_cast<const T*>(p.q) + z * p.qs0 + h * p.qs1);
  const char* kbase = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + z * p.ks0 + kvh * p.ks1);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + z * p.vs0 + kvh * p.vs1);
  const uint32_t qsb = static_cast<uint32_t>(p.qs2) * 2u;
  const uint32_t ksb = static_cast<uint32_t>(p.ks2) * 2u;
  const uint32_t vsb = static_cast<uint32_t>(p.vs2) * 2u;

  // Q^T operand, resident for the whole row: lane (li + 32 kh) holds
  // Q[qpos][16 s + 8 kh .. +8]. Rows past N read row N-1 (never stored).
  // A negative scale is folded into Q's sign so that c = |scale| > 0 and the
  // row maximum of the raw dot products maps to the maximum score.
  const uint32_t qsign = p.qk_scale < 0.f ? 0x80008000u : 0u;
  const float c = fmaxf(fabsf(p.qk_scale), 1e-30f);
  u32x4_t qf[KS];
  {
    const uint32_t qoff = __umul24(static_cast<uint32_t>(min(qpos, N - 1)), qsb) + 16u * kh;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qf[s] = *reinterpret_cast<const u32x4_t*>(qbase + qoff + 32u * s) ^ qsign;
    }
  }

  // ---- LDS layout of a stage: K tile then V tile, BN rows of ROWB bytes,
  // 16-byte chunk c of row r stored at position c ^ f(r):
  //   K: f = (r >> RSH) & (CPR-1)  -> the 16 rows read by one MFMA operand
  //      fetch hit 16 distinct 16-byte bank groups;
  //   V: f = 4 sigma(r) + 2 tau(r) -> XORs the 64-byte segment (sigma) and
  //      32-byte half (tau) of a row, so that the 4 rows x 32 bytes of a
  //      16-lane transpose read (ds_read_b64_tr_b16) and the 4 rows x 64
  //      bytes of a 32-lane one land in distinct banks of a 128-byte and of
  //      a 256-byte bank window alike.
  auto fk = [](int r) { return (r >> RSH) & (CPR - 1); };
  auto vsig = [](int r) { return D >= 128 ? (r & 3) : (D == 64 ? ((r >> 1) & 1) : 0); };
  auto vtau = [](int r) { return D == 64 ? (r & 1) : ((r >> 1) & 1); };
  auto fv = [&](int r) { return 4 * vsig(r) + 2 * vtau(r); };

  // Direct-to-LDS loads: load i of this wave fills 1-KB block `blk` of the
  // K (isk) or V tile: lane L writes slot 64 blk + L = (row, position), and
  // fetches the global chunk that belongs at that position. Whether a load
  // targets K or V depends on the wave only (uniform).
  uint32_t goff[LPW];   // byte offset of the lane's chunk from the tile's first row
  int grow[LPW];        // the lane's row inside the tile
#pragma unroll
  for (int i = 0; i < LPW; ++i) {
    const int q = wave * LPW + i;
    const bool isk = q < NKI;
    const int slot = (isk ? q : q - NKI) * 64 + lane;
    const int r = slot / CPR, pos = slot % CPR;
    const int cc = pos ^ (isk ? fk(r) : fv(r));
    grow[i] = r;
    goff[i] = __umul24(static_cast<uint32_t>(r), isk ? ksb : vsb) + 16u * cc;
  }
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SA_LDS char*)stage_lds));
  // Issues the K and V loads of the tile whose first key is key0 into stage stg.
  auto issue = [&](int key0, int stg) {
    if (key0 >= 0 && key0 + BN <= N) {
      // Whole tile in range: one scalar base per tile, per-lane 32-bit offsets.
      const char* kt = kbase + static_cast<size_t>(key0) * ksb;
      const char* vt = vbase + static_cast<size_t>(key0) * vsb;
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int q = wave * LPW + i;
        const bool isk = q < NKI;
        const uint32_t dst = __builtin_amdgcn_readfirstlane(
            lds_base + stg * STAGEB + (isk ? 0 : TILEB) + (isk ? q : q - NKI) * 1024);
        dma16_s(isk ? kt : vt, goff[i], dst);
      }
    } else {
      // Rows outside [0, N) read a valid row: their scores are masked to
      // -inf, so p = 0 and the data never reaches the output.
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int q = wave * LPW + i;
        const bool isk = q < NKI;
        const char* gb = isk ? kbase : vbase;
        const uint32_t rs = isk ? ksb : vsb;
        const uint32_t rr = static_cast<uint32_t>(min(max(key0 + grow[i], 0), N - 1));
        const char* src = gb + __umul24(rr, rs) + (goff[i] - __umul24(static_cast<uint32_t>(grow[i]), rs));
        const uint32_t dst = __builtin_amdgcn_readfirstlane(
            lds_base + stg * STAGEB + (isk ? 0 : TILEB) + (isk ? q : q - NKI) * 1024);
        dma16(src, dst);
      }
    }
  };

  // LDS read addresses (lane bases; stage / k-step / tile offsets are immediates).
  // K operand of S^T: lane (m + 32 kh) reads row m, chunk 2 s + kh.
  uint32_t k_rd[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) k_rd[s] = li * ROWB + 16 * ((2 * s + kh) ^ fk(li));
  // V^T operand of O^T += V^T P^T via transpose reads: in each 16-lane group
  // (g = lane / 16, j = lane % 16) lane j addresses row 4 kh + (j >> 2)
  // (+ 16 s2 + 8 for the second half) and columns 4 (j & 3) + 16 (g & 1) of
  // the 32-column tile dt; the hardware hands lane i the values of column
  // i (+16 (g & 1)) of the four addressed rows. Rows r and r + 8 share the
  // swizzle, so the row offsets stay immediates; one address per tile dt.
  uint32_t v_rd[DT];
  {
    const int g = lane >> 4, j = lane & 15;
    const int vr = 4 * kh + (j >> 2);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      v_rd[dt] = TILEB + vr * ROWB + 64 * (dt ^ vsig(vr)) + 32 * ((g & 1) ^ vtau(vr)) + 16 * ((j & 3) >> 1) +
                 8 * (j & 1);
    }
  }

  f32x16_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16_t{};
  float m_i = -INFINITY, l_i = 0.f;

  // The first S - 1 tiles come from the row's first list entries (the first
  // two when a route block holds one tile), read with uniform loads at entry:
  // their K / V loads are issued before the row's count and list have
  // arrived. The row has max_count readable entries; issue() clamps any key
  // out of range, so this is safe for short or empty rows too (loads that no
  // tile consumes are drained before the kernel ends).
  if constexpr (FUSED) {
    // This row's list from the routing ids, as build_block_lists does with
    // `arity` (block_list.py:212-229,263-278): code = sum_l id_l [l < depth]
    // base^l (wrapping 64-bit), match = equal codes, then local band OR, sink
    // OR, causal AND; key block kb is thread kb (NB <= NT), the ballot and the
    // waves' hit counts give its slot. The first query tile of the route
    // block writes the row back (sync-free layout: NB columns, zero padded).
    const int depth = p.depth_dev ? static_cast<int>(p.depth_dev[h]) : p.depth_uniform;
    auto code_of = [&](int blk) {
      uint64_t code = 0, pw = 1;
      for (int l = 0; l < p.TD; ++l) {
        if (l < depth) {
          const int64_t off = z * p.rs0 + h * p.rs1 + blk * p.rs2 + l * p.rs3;
          const int64_t id = p.router_i64 ? static_cast<const int64_t*>(p.router)[off]
                                          : static_cast<int64_t>(static_cast<const int32_t*>(p.router)[off]);
          code += static_cast<uint64_t>(id) * pw;
        }
        pw *= p.base;
      }
      return code;
    };
    const int kb = tid;
    bool m = false;
    if (kb < p.NB) {
      m = code_of(kb) == code_of(qb);
      const int diff = qb > kb ? qb - kb : kb - qb;
      if (p.local > 0 && diff <= p.local) m = true;
      if (p.sink && kb == 0) m = true;
      if (CAUSAL && kb > qb) m = false;
    }
    const uint64_t hits = __ballot(m);
    if (lane == 0) wave_hits[wave] = static_cast<int>(__popcll(hits));
    __syncthreads();
    int before = 0;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const int c = wave_hits[w];
      before += w < wave ? c : 0;
      count += c;
    }
    const int pos = before + static_cast<int>(__builtin_amdgcn_mbcnt_hi(
                                 static_cast<uint32_t>(hits >> 32),
                                 __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(hits), 0u)));
    if (m) {
      list_lds[pos] = kb;
      bias_lds[pos] = 0.f;
    }
    if (m0 % p.RB == 0 && kb < p.NB) {
      int32_t* out_row = p.lists_out + row * p.NB;
      if (m) out_row[pos] = kb;
      if (kb >= count) out_row[kb] = 0;
      if (kb == 0) p.counts_out[row] = count;
    }
    __syncthreads();
  }
  const int e0 = FUSED ? (count > 0 ? __builtin_amdgcn_readfirstlane(list_lds[0]) : 0)
                       : (p.max_count > 0 ? list[0] : 0);
  const int e1 = FUSED ? (count > 1 ? __builtin_amdgcn_readfirstlane(list_lds[1]) : e0)
                       : (p.max_count > 1 ? list[1] : 0);
  auto early_key = [&](int m) { return ((m >> lspb) == 0 ? e0 : e1) * p.RB + (m & (spb - 1)) * BN; };
#pragma unroll
  for (int st0 = 0; st0 < S - 1; ++st0) issue(early_key(st0), st0);

  // Folds tile n (first key key0, held in stage stg) into the running state.
  auto compute = [&](int n, int key0, int stg) {
    const bool skip = qw0 >= N || static_cast<unsigned>(key0) >= static_cast<unsigned>(N) ||
                      (CAUSAL && key0 > qw0 + 31);
    if (skip) return;
    const float bias = bias_lds[n >> lspb];
    char* sbase = stage_lds + stg * STAGEB;

    // S^T = K Q^T (raw dot products); register v of lane (i + 32 h) holds key
    // 8 (v >> 2) + 4 h + (v & 3) of query i.
    u32x4_t ka[KS];
#pragma unroll
    for (int s = 0; s < KS; ++s) ka[s] = *reinterpret_cast<const u32x4_t*>(sbase + k_rd[s]);
    f32x16_t st = f32x16_t{};
#pragma unroll
    for (int s = 0; s < KS; ++s) st = Mma<T>::mma(ka[s], qf[s], st);

    const bool need_mask = key0 + BN > N || (CAUSAL && key0 + BN - 1 > qw0);
    if (need_mask) {
      int lim = N - 1 - key0;
      if (CAUSAL) lim = min(lim, qpos - key0);
      lim -= 4 * kh;
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        if (8 * (v >> 2) + (v & 3) > lim) st[v] = -INFINITY;
      }
    }
    float mraw = st[0];
#pragma unroll
    for (int v = 1; v < 16; ++v) mraw = fmaxf(mraw, st[v]);
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mraw), __float_as_uint(mraw), false, false);
      mraw = fmaxf(mraw, fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
    }
    const float mtile = mraw * c + bias;   // this tile's row max, scaled log2 units
    if (__any(mtile > m_i + kRescale)) {
      const float m_new = fmaxf(m_i, mtile);
      const float alpha = fast_exp2(m_i - (m_new == -INFINITY ? 0.f : m_new));
      l_i *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      m_i = m_new;
    }
    const float nb = bias - (m_i == -INFINITY ? 0.f : m_i);
    u32x4_t pb[2];
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      float pv[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        pv[e] = fast_exp2(fmaf(st[8 * s2 + e], c, nb));
        l_i += pv[e];
      }
      pb[s2] = u32x4_t{Mma<T>::pack(pv[0], pv[1]), Mma<T>::pack(pv[2], pv[3]),
                       Mma<T>::pack(pv[4], pv[5]), Mma<T>::pack(pv[6], pv[7])};
    }
    // O^T += V^T P^T. MFMA k-index 8 kh + e of step s2 is key 16 s2 + 4 kh + e
    // (e < 4) or 16 s2 + 8 + 4 kh + (e - 4): the first / second transpose read.
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint32_t vb = v_rd[dt];
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        SA_LDS s16x4_t* a0 = (SA_LDS s16x4_t*)((SA_LDS char*)sbase + vb + (16 * s2) * ROWB);
        SA_LDS s16x4_t* a1 = (SA_LDS s16x4_t*)((SA_LDS char*)sbase + vb + (16 * s2 + 8) * ROWB);
        const u32x2_t lo = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(a0));
        const u32x2_t hi = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(a1));
        acc[dt] = Mma<T>::mma(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, pb[s2], acc[dt]);
      }
    }
  };

  // The row's list is walked in segments of at most kListSeg blocks, each
  // staged in LDS (with its soft-bias values, zero when there is none). Tile
  // m of a segment covers keys list[m / spb] * RB + (m % spb) * BN .. +BN.
  for (int seg = 0; seg < count; seg += kListSeg) {
    const int seg_n = min(count - seg, kListSeg);
    if (seg > 0) __syncthreads();   // every wave is done with the previous segment
    if constexpr (!FUSED) {
      for (int t = tid; t < seg_n; t += NT) {
        list_lds[t] = list[seg + t];
        bias_lds[t] = p.sb ? load_bias(p, z, h, qb, seg + t) : 0.f;
      }
    }
    __syncthreads();
    // No compiler-visible load may be outstanding once the pipeline runs (the
    // explicit vmcnt waits below count only the pipeline's own loads; the
    // early tiles of segment 0 are among them).
    __builtin_amdgcn_s_waitcnt(0);
    const int total = seg_n * spb;
    auto tile_key0 = [&](int m) { return list_lds[m >> lspb] * p.RB + (m & (spb - 1)) * BN; };

    // Pipeline: tiles n+1 .. n+S-2 stay in flight while tile n is computed;
    // tile n+S-1 is issued into the stage tile n-1 used, once every wave has
    // passed the barrier that follows tile n-1's compute. Key offsets of the
    // tiles held by each stage live in registers; the list entry of the next
    // tile to issue is read one step ahead.
    int key_of[S];
#pragma unroll
    for (int st0 = 0; st0 < S - 1; ++st0) {
      if (seg == 0) {
        key_of[st0] = early_key(st0);   // already issued
      } else {
        key_of[st0] = st0 < total ? tile_key0(st0) : 0;
        if (st0 < total) issue(key_of[st0], st0);
      }
    }
    key_of[S - 1] = 0;
    int next_key = S - 1 < total ? tile_key0(S - 1) : 0;
    int n = 0;
    auto step = [&](auto stg_c) {
      constexpr int stg = decltype(stg_c)::value;
      if (n >= total) return;
      wait_tiles<LPW, S - 2>(total - 1 - n);
      barrier_only();
      if (n + S - 1 < total) {
        constexpr int nst = (stg + S - 1) % S;
        key_of[nst] = next_key;
        issue(next_key, nst);
        if (n + S < total) next_key = tile_key0(n + S);
      }
      compute(n, key_of[stg], stg);
      ++n;
    };
    while (n < total) {
      step(std::integral_constant<int, 0>{});
      step(std::integral_constant<int, 1>{});
      if constexpr (S > 2) step(std::integral_constant<int, 2>{});
      if constexpr (S > 3) step(std::integral_constant<int, 3>{});
    }
  }

  wait_vmcnt<0>();   // early tiles of an empty or short row
  const float l_tot = l_i + __shfl_xor(l_i, 32);
  if (qpos < N) {
    const float inv = 1.f / (l_tot == 0.f ? 1.f : l_tot);
    T* op = static_cast<T*>(p.out) + z * p.os0 + h * p.os1 + qpos * p.os2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * kh;
        const u32x2_t val{Mma<T>::pack(acc[dt][4 * g] * inv, acc[dt][4 * g + 1] * inv),
                          Mma<T>::pack(acc[dt][4 * g + 2] * inv, acc[dt][4 * g + 3] * inv)};
        *reinterpret_cast<u32x2_t*>(op + d) = val;
      }
    }
    if (p.lse && kh == 0) {
      p.lse[static_cast<int64_t>(zh) * N + qpos] = (m_i + fast_log2(l_tot)) * kLn2;
    }
  }
}

// ---- host dispatch -------------------------------------------------------------
template <typename T>
int launch_generic(FwdParams& p, int D, hipStream_t stream) {
  p.mtiles = (p.N + 15) / 16;
  p.total_wg = p.Z * p.H * p.mtiles;
  dim3 g(p.total_wg), b(256);
  switch (D) {
    case 16: hipLaunchKernelGGL((prefill_generic_kernel<T, 16>), g, b, 0, stream, p); break;
    case 32: hipLaunchKernelGGL((prefill_generic_kernel<T, 32>), g, b, 0, stream, p); break;
    case 64: hipLaunchKernelGGL((prefill_generic_kernel<T, 64>), g, b, 0, stream, p); break;
    case 128: hipLaunchKernelGGL((prefill_generic_kernel<T, 128>), g, b, 0, stream, p); break;
    case 256: hipLaunchKernelGGL((prefill_generic_kernel<T, 256>), g, b, 0, stream, p); break;
    default: return fail(SA_EUNSUPPORTED, "head_dim must be a power of two in [16, 256]");
  }
  return check_launch("block-sparse prefill (generic) kernel");
}

template <typename T, int D, int NW, int S, int WPE>
void launch_mfma_shape(FwdParams& p, hipStream_t stream) {
  p.mtiles = (p.N + NW * 32 - 1) / (NW * 32);
  p.total_wg = p.Z * p.H * p.mtiles;
  dim3 g(p.total_wg), b(NW * 64);
  if (p.router) {
    if (p.is_causal)
      hipLaunchKernelGGL((prefill_mfma_kernel<T, D, NW, true, S, WPE, true>), g, b, 0, stream, p);
    else
      hipLaunchKernelGGL((prefill_mfma_kernel<T, D, NW, false, S, WPE, true>), g, b, 0, stream, p);
    return;
  }
  if (p.is_causal)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, D, NW, true, S, WPE, false>), g, b, 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_mfma_kernel<T, D, NW, false, S, WPE, false>), g, b, 0, stream, p);
}

// Three pipeline stages (48 KB of LDS at D = 128) and a register budget of
// three waves per SIMD: three workgroups share a CU, so one workgroup's
// prologue / epilogue latency overlaps the others' MFMA work.
template <typename T, int D, int NW>
void launch_mfma_variant(FwdParams& p, hipStream_t stream) {
  if constexpr (D == 256) {
    // Q (64 registers) and O (128) of a 32-row slice: one wave per SIMD, one
    // workgroup per CU (three 32 KB stages).
    launch_mfma_shape<T, D, NW, 3, 1>(p, stream);
  } else {
    launch_mfma_shape<T, D, NW, 3, 3>(p, stream);
  }
}

template <typename T, int D>
int launch_mfma_d(FwdParams& p, hipStream_t stream) {
  const int RB = p.RB;
  if (RB % 128 == 0) launch_mfma_variant<T, D, 4>(p, stream);
  else if (RB == 64) launch_mfma_variant<T, D, 2>(p, stream);
  else if constexpr (D != 256) launch_mfma_variant<T, D, 1>(p, stream);  // RB == 32 (D = 256 needs RB >= 64)
  return check_launch("block-sparse prefill (MFMA) kernel");
}

template <typename T>
int launch_mfma(FwdParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 32: return launch_mfma_d<T, 32>(p, stream);
    case 64: return launch_mfma_d<T, 64>(p, stream);
    case 256: return launch_mfma_d<T, 256>(p, stream);
    default: return launch_mfma_d<T, 128>(p, stream);
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

}  // namespace
}  // namespace sa

namespace sa {
namespace {

// Routing ids of the fused entry point (sa_routed_block_sparse_fwd).
struct FusedRouting {
  const void* router;
  int router_dtype;
  const int64_t* strides;
  int TD;
  const int64_t* depth_dev;
  int depth_uniform;
  int64_t base;
  int sink_block, local_blocks;
};

int fwd_impl(const void* q, const void* k, const void* v, void* out, float* lse, const int32_t* lists,
             const int32_t* counts, const void* soft_bias, int soft_bias_dtype, int Z, int H, int H_kv, int N,
             int D, int route_block, int max_count, const int64_t* q_strides, const int64_t* k_strides,
             const int64_t* v_strides, const int64_t* o_strides, const int64_t* sb_strides, float sm_scale,
             int dtype, int is_causal, void* stream, const FusedRouting* fz, int32_t* lists_out,
             int32_t* counts_out) {
  if (!q_strides || !k_strides || !v_strides || !o_strides) return fail(SA_EINVAL, "NULL strides");
  if (Z < 0 || H < 0 || N < 0 || H_kv <= 0 || (H > 0 && H % H_kv != 0)) {
    return fail(SA_EINVAL, "bad Z/H/H_kv/N");
  }
  if (!is_pow2(D) || D < 16) return fail(SA_EINVAL, "head_dim must be a power of two >= 16");
  if (D > 256) return fail(SA_EUNSUPPORTED, "head_dim > 256 is not supported");
  if (!is_pow2(route_block) || route_block < 16) {
    return fail(SA_EINVAL, "route_block must be a power of two >= 16");
  }
  if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16) {
    return fail(SA_EINVAL, "dtype must be f32, bf16 or f16");
  }
  if (soft_bias && (!sb_strides || (soft_bias_dtype != SA_DTYPE_F32 &&
                                    soft_bias_dtype != SA_DTYPE_BF16 &&
                                    soft_bias_dtype != SA_DTYPE_F16))) {
    return fail(SA_EINVAL, "soft_bias needs strides and an f32/bf16/f16 dtype");
  }
  if (max_count < 0) return fail(SA_EINVAL, "max_count must be >= 0");
  if (static_cast<long long>(Z) * H * N == 0) return SA_OK;    // empty tensors may carry NULL
  if (!q || !k || !v || !out || !counts || (!lists && max_count > 0)) {
    return fail(SA_EINVAL, "NULL tensor argument");
  }

  FwdParams p{};
  p.q = q; p.k = k; p.v = v; p.out = out; p.lse = lse;
  p.lists = lists; p.counts = counts;
  p.sb = soft_bias; p.sb_dtype = soft_bias_dtype;
  if (soft_bias) {
    p.sbs0 = sb_strides[0]; p.sbs1 = sb_strides[1]; p.sbs2 = sb_strides[2]; p.sbs3 = sb_strides[3];
  }
  p.qs0 = q_strides[0]; p.qs1 = q_strides[1]; p.qs2 = q_strides[2]; p.qs3 = q_strides[3];
  p.ks0 = k_strides[0]; p.ks1 = k_strides[1]; p.ks2 = k_strides[2]; p.ks3 = k_strides[3];
  p.vs0 = v_strides[0]; p.vs1 = v_strides[1]; p.vs2 = v_strides[2]; p.vs3 = v_strides[3];
  p.os0 = o_strides[0]; p.os1 = o_strides[1]; p.os2 = o_strides[2]; p.os3 = o_strides[3];
  p.Z = Z; p.H = H; p.Hkv = H_kv; p.N = N; p.RB = route_block;
  p.NB = (N + route_block - 1) / route_block;
  p.max_count = max_count;
  p.group = H / H_kv;
  p.qk_scale = sm_scale * kLog2e;
  p.is_causal = is_causal != 0;
  // Lists longer than a quarter of the grid (dense-ish rows): four heads
  // dealt together, longest query tiles first, as long as their K / V stay
  // within 32 MB (dense causal N = 8192: 519 against 547 us; config 3 at
  // N = 8192: 6-13% faster at every density). Sparse lists keep one head at a
  // time (config 2: 78.0 against 79.2 us), and so do longer sequences (N =
  // 32768, 64 MB of K / V for four heads: 12% slower at rho = 0.5). The fused
  // build's list lengths are not known at launch: one head at a time.
  const long long kv_heads4 = std::max(1, 4 / std::max(p.group, 1));
  const long long kv_bytes4 = kv_heads4 * static_cast<long long>(N) * D * 2 * (dtype == SA_DTYPE_F32 ? 4 : 2);
  p.hgroup = !fz && 4 * static_cast<long long>(max_count) > p.NB && kv_bytes4 <= (32LL << 20) ? 4 : 1;
  hipStream_t s = as_stream(stream);

  // The MFMA path needs unit stride along D and 16-byte aligned rows.
  const bool rows_ok = p.qs3 == 1 && p.ks3 == 1 && p.vs3 == 1 && p.os3 == 1 &&
                       p.qs2 % 8 == 0 && p.ks2 % 8 == 0 && p.vs2 % 8 == 0 && p.os2 % 8 == 0 &&
                       p.qs1 % 8 == 0 && p.ks1 % 8 == 0 && p.vs1 % 8 == 0 && p.os1 % 8 == 0 &&
                       p.qs0 % 8 == 0 && p.ks0 % 8 == 0 && p.vs0 % 8 == 0 && p.os0 % 8 == 0 &&
                       aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
  // 24-bit row index / row stride multiplies and 32-bit per-head byte spans.
  const long long max_rs = std::max({p.qs2, p.ks2, p.vs2}) * 2;
  const bool offs_ok = N < (1 << 24) && max_rs < (1 << 24) &&
                       static_cast<long long>(N) * max_rs < (1LL << 32);
  const bool mfma_ok = dtype != SA_DTYPE_F32 && (D == 32 || D == 64 || D == 128 || (D == 256 && route_block >= 64)) &&
                       route_block >= 32 && rows_ok && offs_ok;
  const long long wg = static_cast<long long>(Z) * H * ((N + 15) / 16);
  if (wg > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");

  if (fz) {
    // The fused build runs inside the MFMA kernel: one key block per thread.
    const int nt = 64 * (route_block % 128 == 0 ? 4 : (route_block == 64 ? 2 : 1));
    if (!mfma_ok || soft_bias || p.NB > nt) {
      return fail(SA_EUNSUPPORTED, "fused list build needs the MFMA path, no soft bias and NB <= " +
                                       std::to_string(nt));
    }
    p.router = fz->router;
    p.rs0 = fz->strides[0]; p.rs1 = fz->strides[1]; p.rs2 = fz->strides[2]; p.rs3 = fz->strides[3];
    p.router_i64 = fz->router_dtype == SA_DTYPE_I64;
    p.TD = fz->TD;
    p.depth_dev = fz->depth_dev;
    p.depth_uniform = fz->depth_uniform;
    p.base = static_cast<uint64_t>(fz->base);
    p.sink = fz->sink_block != 0;
    p.local = fz->local_blocks;
    p.lists_out = lists_out;
    p.counts_out = counts_out;
  }
  if (mfma_ok) {
    return dtype == SA_DTYPE_BF16 ? launch_mfma<bf16_t>(p, D, s) : launch_mfma<f16_t>(p, D, s);
  }
  if (dtype == SA_DTYPE_F32) return launch_generic<float>(p, D, s);
  if (dtype == SA_DTYPE_BF16) return launch_generic<bf16_t>(p, D, s);
  return launch_generic<f16_t>(p, D, s);
}

}  // namespace
}  // namespace sa

extern "C" int sa_block_sparse_fwd(const void* q, const void* k, const void* v, void* out,
                                   float* lse, const int32_t* lists, const int32_t* counts,
                                   const void* soft_bias, int soft_bias_dtype, int Z, int H,
                                   int H_kv, int N, int D, int route_block, int max_count,
                                   const int64_t* q_strides, const int64_t* k_strides,
                                   const int64_t* v_strides, const int64_t* o_strides,
                                   const int64_t* sb_strides, float sm_scale, int dtype,
                                   int is_causal, void* stream) {
  return sa::fwd_impl(q, k, v, out, lse, lists, counts, soft_bias, soft_bias_dtype, Z, H, H_kv, N, D,
                      route_block, max_count, q_strides, k_strides, v_strides, o_strides, sb_strides, sm_scale,
                      dtype, is_causal, stream, nullptr, nullptr, nullptr);
}

extern "C" int sa_routed_block_sparse_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                                          const void* router, int router_dtype, const int64_t* router_strides,
                                          int TD, const int64_t* depth_dev, int depth_uniform, int64_t base,
                                          int sink_block, int local_blocks, int32_t* lists, int32_t* counts,
                                          int Z, int H, int H_kv, int N, int D, int route_block,
                                          const int64_t* q_strides, const int64_t* k_strides,
                                          const int64_t* v_strides, const int64_t* o_strides, float sm_scale,
                                          int dtype, int is_causal, void* stream) {
  using namespace sa;
  if (router_dtype != SA_DTYPE_I32 && router_dtype != SA_DTYPE_I64) {
    return fail(SA_EINVAL, "router ids must be int32 or int64");
  }
  if (TD < 1) return fail(SA_EINVAL, "tree depth must be >= 1");
  if (!depth_dev && (depth_uniform < 0 || depth_uniform > TD)) {
    return fail(SA_EINVAL, "req_depth out of range [0, TD]");
  }
  if (base < 2) return fail(SA_EINVAL, "code base must be >= 2");
  if (local_blocks < 0) return fail(SA_EINVAL, "local_blocks must be >= 0");
  const long long NB = route_block > 0 ? (static_cast<long long>(N) + route_block - 1) / route_block : 0;
  if (static_cast<long long>(Z) * H * N > 0 && (!router || !router_strides || !lists || !counts)) {
    return fail(SA_EINVAL, "NULL router / lists / counts");
  }
  const FusedRouting fz{router, router_dtype, router_strides, TD, depth_dev, depth_uniform, base, sink_block,
                        local_blocks};
  return fwd_impl(q, k, v, out, lse, lists, counts, nullptr, 0, Z, H, H_kv, N, D, route_block,
                  static_cast<int>(NB), q_strides, k_strides, v_strides, o_strides, nullptr, sm_scale, dtype,
                  is_causal, stream, &fz, lists, counts);
}
