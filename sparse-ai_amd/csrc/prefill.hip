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
//  * prefill_mfma_kernel — bf16/fp16, D in {32, 64, 128}, route_block % 32 == 0.
//    A workgroup of NW waves owns BM = 32*NW query rows of one route block.
//    Each wave computes S^T = K Q^T on 32x32x16 MFMA tiles, so lane (i + 32h)
//    holds 16 keys of query i per tile: row max / row sum need one exchange
//    with lane ^ 32, and the O^T = V^T P^T accumulator is rescaled with one
//    per-lane scalar. K/V sub-tiles of BN keys are double-buffered in LDS:
//    K rows with an XOR swizzle on 16-byte chunks, V as 4-key "quads"
//    (entry [quad][d] = the 4 keys' values of column d) so each MFMA operand
//    is two conflict-free 8-byte LDS reads. Workgroup ids are remapped so
//    that each XCD works on a contiguous range of heads (shared K/V blocks
//    hit that XCD's L2).
//  * prefill_generic_kernel — any of fp32/bf16/fp16, D power of two in
//    [16, 256], any route block: 16 lanes per query row, fp32 FMA math, used
//    for fp32 inputs (true fp32, no TF32 shortcut) and shapes the MFMA path
//    does not cover.
#include "sa_internal.h"

namespace sa {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

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

constexpr int kListCache = 1024;  // MFMA path: a row's list (<= 1024 blocks) lives in LDS

// XCD-aware work index: workgroup b runs on XCD b % 8; give each XCD a
// contiguous range of the T work items.
__device__ __forceinline__ int xcd_remap(int b, int T) {
  const int xcd = b & 7, slot = b >> 3;
  const int q8 = T >> 3, r8 = T & 7;
  return xcd < r8 ? xcd * (q8 + 1) + slot : r8 * (q8 + 1) + (xcd - r8) * q8 + slot;
}

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
template <typename T> struct Mma;
template <> struct Mma<bf16_t> {
  typedef bf16x8_t vec;
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(vec, a),
                                                   __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_bf16x2(lo, hi); }
};
template <> struct Mma<f16_t> {
  typedef f16x8_t vec;
  static __device__ __forceinline__ f32x16_t mma(u32x4_t a, u32x4_t b, f32x16_t c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(vec, a),
                                                  __builtin_bit_cast(vec, b), c, 0, 0, 0);
  }
  static __device__ __forceinline__ uint32_t pack(float lo, float hi) { return pack_f16x2(lo, hi); }
};

template <typename T, int D, int NW, int BN, bool CAUSAL>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void prefill_mfma_kernel(FwdParams p) {
  constexpr int NT = NW * 64;
  constexpr int BM = NW * 32;
  constexpr int CPR = D / 8;   // 16-byte chunks per row
  constexpr int KS = D / 16;   // MFMA k-steps of S^T = K Q^T
  constexpr int ST = BN / 32;  // 32-key S^T tiles per sub-tile
  constexpr int DT = D / 32;   // 32-row O^T tiles
  constexpr int PS = BN / 16;  // MFMA k-steps of O^T += V^T P^T
  constexpr int NQ = BN / 4;   // key quads per sub-tile
  constexpr int K_CHUNKS = BN * CPR;
  constexpr int V_PAIRS = NQ * CPR;
  constexpr int KPT = (K_CHUNKS + NT - 1) / NT;
  constexpr int VPT = (V_PAIRS + NT - 1) / NT;

  __shared__ u32x4_t k_lds[2][K_CHUNKS];
  __shared__ u32x2_t v_lds[2][NQ * D];
  // The row's list (and soft biases) staged once: reading them from LDS in
  // the loop keeps global loads out of the way of the K/V prefetch.
  __shared__ int32_t list_lds[kListCache];
  __shared__ float bias_lds[kListCache];

  const int work = xcd_remap(blockIdx.x, p.total_wg);
  const int zh = work / p.mtiles;
  const int mt = p.mtiles - 1 - work % p.mtiles;
  const int z = zh / p.H, h = zh % p.H, kvh = h / p.group;
  const int m0 = mt * BM;
  const int qb = m0 / p.RB;
  const int64_t row = static_cast<int64_t>(zh) * p.NB + qb;
  const int count = min(max(p.counts[row], 0), p.max_count);
  const int32_t* list = p.lists + row * p.max_count;
  const int spb = p.RB / BN;
  const int total = count * spb;

  const int tid = threadIdx.x;
  const int wave = tid >> 6, lane = tid & 63;
  for (int t = tid; t < count; t += NT) {
    list_lds[t] = list[t];
    if (p.sb) bias_lds[t] = load_bias(p, z, h, qb, t);
  }
  __syncthreads();
  const int li = lane & 31, kh = lane >> 5;
  const int qw0 = m0 + wave * 32;
  const int qpos = qw0 + li;
  const int N = p.N;

  const T* qp = static_cast<const T*>(p.q) + z * p.qs0 + h * p.qs1;
  const T* kp = static_cast<const T*>(p.k) + z * p.ks0 + kvh * p.ks1;
  const T* vp = static_cast<const T*>(p.v) + z * p.vs0 + kvh * p.vs1;

  // Q^T operand, resident for the whole row: lane (li + 32 kh) holds
  // Q[qpos][16 s + 8 kh .. +8].
  // Rows past N are clamped to row N-1 (never stored): every load is
  // unconditional, so the compiler can count outstanding loads exactly.
  u32x4_t qf[KS];
  const int qrow = qpos < N ? qpos : N - 1;
#pragma unroll
  for (int s = 0; s < KS; ++s) {
    qf[s] = *reinterpret_cast<const u32x4_t*>(qp + qrow * p.qs2 + 16 * s + 8 * kh);
  }

  f32x16_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16_t{};
  float m_i = -INFINITY, l_i = 0.f;

  u32x4_t kreg[KPT];
  u32x4_t vreg[VPT][4];

  auto tile_key0 = [&](int n) { return list_lds[n / spb] * p.RB + (n % spb) * BN; };

  // Keys outside [0, N) load row 0 instead (branch-free, always in bounds):
  // their scores are masked to -inf, so p = 0 exactly and the finite data
  // they bring never reaches the output.
  auto clamp_key = [&](int key) { return static_cast<unsigned>(key) < static_cast<unsigned>(N) ? key : 0; };
  auto load_tile = [&](int n) {
    const int key0 = tile_key0(n);
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int ci = tid + i * NT;
      if (K_CHUNKS % NT == 0 || ci < K_CHUNKS) {
        const int j = ci / CPR, c = ci % CPR;
        kreg[i] = *reinterpret_cast<const u32x4_t*>(kp + clamp_key(key0 + j) * p.ks2 + 8 * c);
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int pi = tid + i * NT;
      if (V_PAIRS % NT == 0 || pi < V_PAIRS) {
        const int q4 = pi / CPR, c = pi % CPR;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          vreg[i][r] = *reinterpret_cast<const u32x4_t*>(vp + clamp_key(key0 + 4 * q4 + r) * p.vs2 + 8 * c);
        }
      }
    }
  };

  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < KPT; ++i) {
      const int ci = tid + i * NT;
      if (K_CHUNKS % NT == 0 || ci < K_CHUNKS) {
        const int j = ci / CPR, c = ci % CPR;
        k_lds[buf][j * CPR + (c ^ (j & (CPR - 1)))] = kreg[i];
      }
    }
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int pi = tid + i * NT;
      if (V_PAIRS % NT == 0 || pi < V_PAIRS) {
        const int q4 = pi / CPR, c = pi % CPR;
        // Entry for column 8c + e: the four keys' 16-bit values of that column.
        u32x2_t ent[8];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          const uint32_t r0 = vreg[i][0][w], r1 = vreg[i][1][w];
          const uint32_t r2 = vreg[i][2][w], r3 = vreg[i][3][w];
          ent[2 * w] = u32x2_t{(r0 & 0xffffu) | (r1 << 16), (r2 & 0xffffu) | (r3 << 16)};
          ent[2 * w + 1] = u32x2_t{(r0 >> 16) | (r1 & 0xffff0000u), (r2 >> 16) | (r3 & 0xffff0000u)};
        }
        u32x4_t* dst = reinterpret_cast<u32x4_t*>(&v_lds[buf][q4 * D + 8 * c]);
#pragma unroll
        for (int w = 0; w < 4; ++w) {
          dst[w] = u32x4_t{ent[2 * w][0], ent[2 * w][1], ent[2 * w + 1][0], ent[2 * w + 1][1]};
        }
      }
    }
  };

  if (total > 0) {
    load_tile(0);
    store_tile(0);
  }
  // Wait for every outstanding load (Q included) on all paths into the loop,
  // so the loop's waits only ever cover its own prefetch.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  int cur_t = -1;
  float bias = 0.f;
  for (int n = 0; n < total; ++n) {
    const int buf = n & 1;
    // Everything this tile needs from memory other than LDS is read before
    // the next tile's prefetch is issued (loads complete in order).
    const int key0 = tile_key0(n);
    const int t = n / spb;
    if (p.sb && t != cur_t) {
      bias = bias_lds[t];
      cur_t = t;
    }
    if (n + 1 < total) load_tile(n + 1);

    const bool skip = qw0 >= N || static_cast<unsigned>(key0) >= static_cast<unsigned>(N) || (CAUSAL && key0 > qw0 + 31);
    if (!skip) {
      const bool need_mask = key0 + BN > N || (CAUSAL && key0 + BN - 1 > qw0);

      f32x16_t st[ST];
#pragma unroll
      for (int t2 = 0; t2 < ST; ++t2) {
        st[t2] = f32x16_t{};
        const int j = 32 * t2 + li;
#pragma unroll
        for (int s = 0; s < KS; ++s) {
          const u32x4_t a = k_lds[buf][j * CPR + ((2 * s + kh) ^ (j & (CPR - 1)))];
          st[t2] = Mma<T>::mma(a, qf[s], st[t2]);
        }
      }

      float mloc = -INFINITY;
#pragma unroll
      for (int t2 = 0; t2 < ST; ++t2) {
#pragma unroll
        for (int v = 0; v < 16; ++v) {
          float sv = st[t2][v] * p.qk_scale + bias;
          if (need_mask) {
            const int key = key0 + 32 * t2 + 8 * (v >> 2) + 4 * kh + (v & 3);
            if (key >= N || (CAUSAL && key > qpos)) sv = -INFINITY;
          }
          st[t2][v] = sv;
          mloc = fmaxf(mloc, sv);
        }
      }
      mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
      const float m_new = fmaxf(m_i, mloc);
      const float m_ref = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = fast_exp2(m_i - m_ref);
      l_i *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
      m_i = m_new;

      u32x4_t pb[PS];
#pragma unroll
      for (int s2 = 0; s2 < PS; ++s2) {
        float pv[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          pv[e] = fast_exp2(st[s2 >> 1][8 * (s2 & 1) + e] - m_ref);
          l_i += pv[e];
        }
        pb[s2] = u32x4_t{Mma<T>::pack(pv[0], pv[1]), Mma<T>::pack(pv[2], pv[3]),
                         Mma<T>::pack(pv[4], pv[5]), Mma<T>::pack(pv[6], pv[7])};
      }
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int s2 = 0; s2 < PS; ++s2) {
          const u32x2_t lo = v_lds[buf][(4 * s2 + kh) * D + 32 * dt + li];
          const u32x2_t hi = v_lds[buf][(4 * s2 + 2 + kh) * D + 32 * dt + li];
          acc[dt] = Mma<T>::mma(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, pb[s2], acc[dt]);
        }
      }
    }

    if (n + 1 < total) store_tile(buf ^ 1);
    __syncthreads();
  }

  const float l_tot = l_i + __shfl_xor(l_i, 32);
  if (qpos < N) {
    const float l_safe = l_tot == 0.f ? 1.f : l_tot;
    T* op = static_cast<T*>(p.out) + z * p.os0 + h * p.os1 + qpos * p.os2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * kh;
        const u32x2_t val{Mma<T>::pack(acc[dt][4 * g] / l_safe, acc[dt][4 * g + 1] / l_safe),
                          Mma<T>::pack(acc[dt][4 * g + 2] / l_safe, acc[dt][4 * g + 3] / l_safe)};
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

template <typename T, int D, int NW, int BN>
void launch_mfma_shape(FwdParams& p, hipStream_t stream) {
  p.mtiles = (p.N + NW * 32 - 1) / (NW * 32);
  p.total_wg = p.Z * p.H * p.mtiles;
  dim3 g(p.total_wg), b(NW * 64);
  if (p.is_causal)
    hipLaunchKernelGGL((prefill_mfma_kernel<T, D, NW, BN, true>), g, b, 0, stream, p);
  else
    hipLaunchKernelGGL((prefill_mfma_kernel<T, D, NW, BN, false>), g, b, 0, stream, p);
}

template <typename T, int D>
int launch_mfma_d(FwdParams& p, hipStream_t stream) {
  const int RB = p.RB;
  if (RB % 128 == 0) launch_mfma_shape<T, D, 4, 64>(p, stream);
  else if (RB == 64) launch_mfma_shape<T, D, 2, 64>(p, stream);
  else launch_mfma_shape<T, D, 1, 32>(p, stream);  // RB == 32
  return check_launch("block-sparse prefill (MFMA) kernel");
}

template <typename T>
int launch_mfma(FwdParams& p, int D, hipStream_t stream) {
  switch (D) {
    case 32: return launch_mfma_d<T, 32>(p, stream);
    case 64: return launch_mfma_d<T, 64>(p, stream);
    default: return launch_mfma_d<T, 128>(p, stream);
  }
}

bool aligned16(const void* ptr) { return (reinterpret_cast<uintptr_t>(ptr) & 15u) == 0; }

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
  using namespace sa;
  if (!q || !k || !v || !out || !lists || !counts) return fail(SA_EINVAL, "NULL tensor argument");
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
  if (static_cast<long long>(Z) * H * N == 0) return SA_OK;

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
  hipStream_t s = as_stream(stream);

  // The MFMA path needs unit stride along D and 16-byte aligned rows.
  const bool rows_ok = p.qs3 == 1 && p.ks3 == 1 && p.vs3 == 1 && p.os3 == 1 &&
                       p.qs2 % 8 == 0 && p.ks2 % 8 == 0 && p.vs2 % 8 == 0 && p.os2 % 8 == 0 &&
                       p.qs1 % 8 == 0 && p.ks1 % 8 == 0 && p.vs1 % 8 == 0 && p.os1 % 8 == 0 &&
                       p.qs0 % 8 == 0 && p.ks0 % 8 == 0 && p.vs0 % 8 == 0 && p.os0 % 8 == 0 &&
                       aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out);
  const bool mfma_ok = dtype != SA_DTYPE_F32 && (D == 32 || D == 64 || D == 128) &&
                       route_block >= 32 && rows_ok && max_count <= kListCache;
  const long long wg = static_cast<long long>(Z) * H * ((N + 15) / 16);
  if (wg > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");

  if (mfma_ok) {
    return dtype == SA_DTYPE_BF16 ? launch_mfma<bf16_t>(p, D, s) : launch_mfma<f16_t>(p, D, s);
  }
  if (dtype == SA_DTYPE_F32) return launch_generic<float>(p, D, s);
  if (dtype == SA_DTYPE_BF16) return launch_generic<bf16_t>(p, D, s);
  return launch_generic<f16_t>(p, D, s);
}
