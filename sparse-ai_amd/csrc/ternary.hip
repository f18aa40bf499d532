// Ternary (2-bit) packed K/V: quantize + pack, and the causal block-sparse
// prefill over packed K/V (gfx950).
//
// Format (pack_ternary, src/llama_surgery/surgery.py:35-55): 16 values per
// int32 word, value i in bits [2i, 2i + 2), code 0 -> 0, 1 -> +1, 2 -> -1
// (code 3, never written, reads as +3 like the reference kernel's
// k_val.to(float)). A row of D values is D / 16 words plus one scale.
//
// ternary_pack_kernel — TernaryQuantize (surgery.py:15-28): gamma = mean |x|
//   of the row, x > gamma/2 -> +1, x < -gamma/2 -> -1, else 0; scale = gamma.
//   Mode "exact" packs values already in {-1, 0, 1} (scale 1), as
//   pack_ternary does.
// ternary_prefill_kernel — _ternary_ultrametric_fwd_kernel
//   (src/llama_surgery/kernel.py:147-249) over block lists (route block 128):
//   the lists carry the reference's block choice (routing match on the first
//   req_depth levels, sink, local window, causal), built by the block-list
//   compactor. Token masks: causal, tail, and the shift regions (keys and
//   queries on the same side of N - shift_size). The ternary values are exact
//   in fp16, so the MFMA operands hold them unscaled: the key scale multiplies
//   the raw scores and the value scale multiplies P before the PV product
//   (sum_j p_j vs_j V_j). A row with no visible key yet keeps the all-masked
//   guard (where the reference would produce NaN) and rows with no visible key
//   at all give 0.
//   Layout: 4 waves x 32 query rows (one route block), fp16 Q^T in registers,
//   tiles of 32 keys double-buffered in LDS; each stage's packed words (64 B
//   per key) are loaded into registers one stage ahead and unpacked into the
//   bank-conflict-free chunk layout used for both the row-major K reads and
//   the transposing V reads.
#include "mfma_util.h"

#include <type_traits>

namespace sa {
namespace {

struct TernParams {
  const void* q;
  const int32_t* kp;
  const int32_t* vp;
  const void* ks;
  const void* vs;
  int scale_dtype;
  const int32_t* lists;
  const int32_t* counts;
  void* out;
  int64_t qs0, qs1, qs2;
  int64_t kps0, kps1, kps2;
  int64_t vps0, vps1, vps2;
  int64_t kss0, kss1, kss2;
  int64_t vss0, vss1, vss2;
  int64_t os0, os1, os2;
  int Z, H, Hkv, N, NB, max_count, group, shift;
  float qk_scale;   // log2(e) / sqrt(D)
  int mtiles, total_wg;
};

template <int D>
__device__ __forceinline__ int tsw(int r) {
  const int sig = D == 128 ? (r & 3) : (D == 64 ? ((r >> 1) & 1) : 0);
  return 4 * sig + ((r >> 2) & 3);
}

__device__ __forceinline__ float load_scale(const void* base, int dtype, int64_t off) {
  if (dtype == SA_DTYPE_F32) return static_cast<const float*>(base)[off];
  if (dtype == SA_DTYPE_BF16) return Elem<bf16_t>::load(static_cast<const bf16_t*>(base) + off);
  return Elem<f16_t>::load(static_cast<const f16_t*>(base) + off);
}

// Unpacks one word (16 codes) into 8 words of fp16 pairs: out[j] holds values
// 2j (low half) and 2j + 1. The fp16 bits of codes 0..3 (0, +1, -1, +3) differ
// in their high byte only, so a byte permute (v_perm_b32) with the table
// 0x42BC3C00 maps a selector [0x0C, code, 0x0C, code] (0x0C selects a zero
// byte) to one output word. Selectors come from the codes split into bytes:
// E0 / E1 / O0 / O1 hold codes 4b / 4b+2 / 4b+1 / 4b+3 in byte b.
__device__ __forceinline__ void unpack_word(uint32_t w, uint32_t (&out)[8]) {
  const uint32_t E = w & 0x33333333u, O = (w >> 2) & 0x33333333u;
  const uint32_t E0 = E & 0x0F0F0F0Fu, E1 = (E >> 4) & 0x0F0F0F0Fu;
  const uint32_t O0 = O & 0x0F0F0F0Fu, O1 = (O >> 4) & 0x0F0F0F0Fu;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const uint32_t b = static_cast<uint32_t>(j >> 1);
    const uint32_t S = 0x0Cu | (b << 8) | (0x0Cu << 16) | ((4u + b) << 24);
    const uint32_t sel = __builtin_amdgcn_perm(j & 1 ? O1 : O0, j & 1 ? E1 : E0, S) | 0x000C000Cu;
    out[j] = __builtin_amdgcn_perm(0u, 0x42BC3C00u, sel);
  }
}

constexpr int kTernSeg = 256;

template <int D>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3)))
void ternary_prefill_kernel(TernParams p) {
  constexpr int BN = 32, RB = 128, WPR = D / 16;   // packed words per row
  constexpr int ROWB = 2 * D, TILEB = BN * ROWB, STAGEB = 2 * TILEB + 256;
  constexpr int KS = D / 16, DT = D / 32;
  constexpr int WPS = BN * WPR;                              // words per K (or V) tile
  static_assert(2 * WPS <= 2 * 256, "one K and one V word per thread at most");
  __shared__ __attribute__((aligned(1024))) char stage_lds[2 * STAGEB];
  __shared__ int32_t list_lds[kTernSeg];

  const int work = xcd_remap(blockIdx.x, p.total_wg);
  const int zh = work / p.mtiles;
  const int mt = p.mtiles - 1 - work % p.mtiles;
  const int z = zh / p.H, h = zh % p.H, kvh = h / p.group;
  const int m0 = mt * RB, qb = mt;
  const int64_t row = static_cast<int64_t>(zh) * p.NB + qb;
  const int count = min(max(p.counts[row], 0), p.max_count);
  const int32_t* list = p.lists + row * p.max_count;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, li = lane & 31, kh = lane >> 5;
  const int N = p.N;
  const int qw0 = m0 + wave * 32, qpos = qw0 + li, qr = min(qpos, N - 1);
  const int split = N - p.shift;                 // first token of the shifted region
  const bool qtail = qpos >= split;

  u32x4_t qf[KS];
  {
    const char* qrow = reinterpret_cast<const char*>(static_cast<const f16_t*>(p.q) + z * p.qs0 + h * p.qs1 +
                                                     static_cast<int64_t>(qr) * p.qs2);
#pragma unroll
    for (int s = 0; s < KS; ++s) qf[s] = *reinterpret_cast<const u32x4_t*>(qrow + 32 * s + 16 * kh);
  }

  // Tile loader: thread t < WPS takes word t of the K tile and of the V tile
  // (key t / WPR, words t % WPR); threads 0..31 / 32..63 take the key / value
  // scales of the tile's 32 keys.
  const int lr = tid / WPR, lw = tid % WPR;
  const bool loads_word = tid < WPS;
  const int32_t* kp0 = p.kp + z * p.kps0 + kvh * p.kps1;
  const int32_t* vp0 = p.vp + z * p.vps0 + kvh * p.vps1;
  const int64_t ks0 = z * p.kss0 + kvh * p.kss1, vs0 = z * p.vss0 + kvh * p.vss1;
  // Two register sets: the words of a tile are loaded two stages before they
  // are unpacked into LDS.
  uint32_t kw[2] = {0u, 0u}, vw[2] = {0u, 0u};
  float sc[2] = {0.f, 0.f};
  auto load_tile = [&](int key0, int r) {
    const int key = min(max(key0 + lr, 0), N - 1);
    if (loads_word) {
      kw[r] = static_cast<uint32_t>(kp0[key * p.kps2 + lw]);
      vw[r] = static_cast<uint32_t>(vp0[key * p.vps2 + lw]);
    }
    if (tid < 64) {
      const int sk = min(max(key0 + (tid & 31), 0), N - 1);
      sc[r] = tid < 32 ? load_scale(p.ks, p.scale_dtype, ks0 + sk * p.kss2)
                       : load_scale(p.vs, p.scale_dtype, vs0 + sk * p.vss2);
    }
  };
  // Unpacks register set r into stage `stg`: word lw of row lr covers
  // d = 16 lw .. 16 lw + 15, i.e. chunks 2 lw and 2 lw + 1.
  auto store_tile = [&](int stg, int r) {
    char* base = stage_lds + stg * STAGEB;
    if (loads_word) {
#pragma unroll
      for (int t2 = 0; t2 < 2; ++t2) {
        const uint32_t w = t2 == 0 ? kw[r] : vw[r];
        char* tile = base + t2 * TILEB + lr * ROWB;
        uint32_t u[8];
        unpack_word(w, u);
#pragma unroll
        for (int half = 0; half < 2; ++half) {
          *reinterpret_cast<u32x4_t*>(tile + 16 * ((2 * lw + half) ^ tsw<D>(lr))) =
              u32x4_t{u[4 * half], u[4 * half + 1], u[4 * half + 2], u[4 * half + 3]};
        }
      }
    }
    if (tid < 64) reinterpret_cast<float*>(base + 2 * TILEB)[tid] = sc[r];
  };

  uint32_t rm[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) rm[s] = li * ROWB + 16 * ((2 * s + kh) ^ tsw<D>(li));
  uint32_t tr0[DT], tr1[DT];
  {
    const int g = lane >> 4, j = lane & 15;
    const int vr = 4 * kh + (j >> 2);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const int c = 4 * dt + 2 * (g & 1) + ((j & 3) >> 1);
      tr0[dt] = TILEB + vr * ROWB + 16 * (c ^ tsw<D>(vr)) + 8 * (j & 1);
      tr1[dt] = TILEB + (vr + 8) * ROWB + 16 * (c ^ tsw<D>(vr + 8)) + 8 * (j & 1);
    }
  }

  f32x16_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16_t{};
  float m_i = -INFINITY, l_i = 0.f;
  const float c = p.qk_scale;

  auto compute = [&](int key0, int stg) {
    if (qw0 >= N || key0 >= N || key0 > qw0 + 31) return;
    const char* sbase = stage_lds + stg * STAGEB;
    f32x16_t st = f32x16_t{};
#pragma unroll
    for (int s = 0; s < KS; ++s) st = Mma<f16_t>::mma(*reinterpret_cast<const u32x4_t*>(sbase + rm[s]), qf[s], st);
    // register v: key key0 + 8 (v >> 2) + 4 kh + (v & 3)
    // tail keys, the causal diagonal, and (with a shift) tiles or query rows
    // that touch the shifted region
    const bool need_mask = key0 + BN > N || key0 + BN - 1 > qw0 ||
                           (p.shift > 0 && (key0 + BN > split || qw0 + 31 >= split));
    float mx = -INFINITY;
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4_t k4 = *reinterpret_cast<const f32x4_t*>(sbase + 2 * TILEB + 4 * (8 * g4 + 4 * kh));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = 4 * g4 + i;
        float x = st[v] * k4[i] * c;
        if (need_mask) {
          const int key = key0 + 8 * g4 + 4 * kh + i;
          if (key >= N || key > qpos || ((key >= split) != qtail)) x = -INFINITY;
        }
        st[v] = x;
        mx = fmaxf(mx, x);
      }
    }
    {
      const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mx), __float_as_uint(mx), false, false);
      mx = fmaxf(mx, fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1])));
    }
    const float m_new = fmaxf(m_i, mx);
    const float m_ref = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = fast_exp2(m_i - m_ref);
    if (alpha != 1.f) {
      l_i *= alpha;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] *= alpha;
    }
    m_i = m_new;
    float pv[16];
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const f32x4_t v4 = *reinterpret_cast<const f32x4_t*>(sbase + 2 * TILEB + 128 + 4 * (8 * g4 + 4 * kh));
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int v = 4 * g4 + i;
        const float e = fast_exp2(st[v] - m_ref);
        l_i += e;
        pv[v] = e * v4[i];
      }
    }
    u32x4_t pb[2];
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      pb[h2] = u32x4_t{pack_f16x2(pv[8 * h2], pv[8 * h2 + 1]), pack_f16x2(pv[8 * h2 + 2], pv[8 * h2 + 3]),
                       pack_f16x2(pv[8 * h2 + 4], pv[8 * h2 + 5]), pack_f16x2(pv[8 * h2 + 6], pv[8 * h2 + 7])};
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int h2 = 0; h2 < 2; ++h2) {
        SA_LDS s16x4_t* a0 = (SA_LDS s16x4_t*)((SA_LDS char*)sbase + tr0[dt] + 16 * h2 * ROWB);
        SA_LDS s16x4_t* a1 = (SA_LDS s16x4_t*)((SA_LDS char*)sbase + tr1[dt] + 16 * h2 * ROWB);
        const u32x2_t lo = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(a0));
        const u32x2_t hi = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(a1));
        acc[dt] = Mma<f16_t>::mma(u32x4_t{lo[0], lo[1], hi[0], hi[1]}, pb[h2], acc[dt]);
      }
    }
  };

  for (int seg = 0; seg < count; seg += kTernSeg) {
    const int seg_n = min(count - seg, kTernSeg);
    __syncthreads();
    for (int t = tid; t < seg_n; t += 256) list_lds[t] = list[seg + t];
    __syncthreads();
    const int total = seg_n * (RB / BN);
    auto key_of = [&](int n) { return list_lds[n >> 2] * RB + (n & 3) * BN; };
    // register set / LDS stage of tile n: n & 1
    load_tile(key_of(0), 0);
    if (total > 1) load_tile(key_of(1), 1);
    store_tile(0, 0);
    if (total > 2) load_tile(key_of(2), 0);
    __syncthreads();
    auto step = [&](int n, auto par_c) {
      constexpr int par = decltype(par_c)::value;   // n & 1
      compute(key_of(n), par);
      if (n + 1 < total) {
        store_tile(par ^ 1, par ^ 1);
        if (n + 3 < total) load_tile(key_of(n + 3), par ^ 1);
      }
      __syncthreads();
    };
    for (int n = 0; n < total; n += 2) {
      step(n, std::integral_constant<int, 0>{});
      if (n + 1 < total) step(n + 1, std::integral_constant<int, 1>{});
    }
  }

  const float l_tot = l_i + __shfl_xor(l_i, 32);
  if (qpos < N) {
    const float inv = 1.f / (l_tot == 0.f ? 1.f : l_tot);
    f16_t* op = static_cast<f16_t*>(p.out) + z * p.os0 + h * p.os1 + static_cast<int64_t>(qpos) * p.os2;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * kh;
        *reinterpret_cast<u32x2_t*>(op + d) = u32x2_t{pack_f16x2(acc[dt][4 * g] * inv, acc[dt][4 * g + 1] * inv),
                                                      pack_f16x2(acc[dt][4 * g + 2] * inv, acc[dt][4 * g + 3] * inv)};
      }
    }
  }
}

// One wave per row: gamma = mean |x| (mode 0) or 1 (mode 1, values already
// ternary); lane w < D / 16 packs word w.
template <typename T>
__global__ __launch_bounds__(256) void ternary_pack_kernel(const T* x, int64_t xs0, int64_t xs1, int rows, int D,
                                                           int mode, int32_t* packed, float* scale) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= rows) return;
  const T* xr = x + r * xs0;
  float a = 0.f;
  for (int d = lane; d < D; d += 64) a += fabsf(Elem<T>::load(xr + d * xs1));
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) a += __shfl_xor(a, o);
  const float gamma = mode == 0 ? a / static_cast<float>(D) : 1.f;
  const float thr = 0.5f * gamma;
  for (int w = lane; w < D / 16; w += 64) {
    uint32_t word = 0;
    for (int i = 0; i < 16; ++i) {
      const float v = Elem<T>::load(xr + (16 * w + i) * xs1);
      const uint32_t cde = mode == 0 ? (v > thr ? 1u : (v < -thr ? 2u : 0u)) : (v == 1.f ? 1u : (v == -1.f ? 2u : 0u));
      word |= cde << (2 * i);
    }
    packed[static_cast<int64_t>(r) * (D / 16) + w] = static_cast<int32_t>(word);
  }
  if (lane == 0 && scale) scale[r] = gamma;
}

// Rows with D / 16 a power of two <= 64 and unit element stride: lane j of
// the LPR lanes of a row owns word j (16 consecutive values, loaded as
// vectors); gamma is reduced over the row's lanes with shuffles.
template <typename T, int LPR>
__global__ __launch_bounds__(256) void ternary_pack_rows_kernel(const T* x, int64_t xs0, int rows, int mode,
                                                                int32_t* packed, float* scale) {
  constexpr int D = 16 * LPR;
  const int tid = blockIdx.x * 256 + threadIdx.x;
  const int r = tid / LPR, w = tid % LPR;
  const bool ok = r < rows;
  const T* xr = x + static_cast<int64_t>(ok ? r : 0) * xs0 + 16 * w;
  float v[16];
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 f = reinterpret_cast<const float4*>(xr)[i];
      v[4 * i] = f.x; v[4 * i + 1] = f.y; v[4 * i + 2] = f.z; v[4 * i + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const uint4 u = reinterpret_cast<const uint4*>(xr)[i];
      const uint32_t ww[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if constexpr (std::is_same<T, bf16_t>::value) {
          v[8 * i + 2 * e] = bf16_bits_to_float(ww[e] & 0xffffu);
          v[8 * i + 2 * e + 1] = bf16_bits_to_float(ww[e] >> 16);
        } else {
          v[8 * i + 2 * e] = f16_bits_to_float(ww[e] & 0xffffu);
          v[8 * i + 2 * e + 1] = f16_bits_to_float(ww[e] >> 16);
        }
      }
    }
  }
  float a = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) a += fabsf(v[i]);
#pragma unroll
  for (int o = 1; o < LPR; o <<= 1) a += __shfl_xor(a, o);
  const float gamma = mode == 0 ? a / static_cast<float>(D) : 1.f;
  const float thr = 0.5f * gamma;
  uint32_t word = 0;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const uint32_t c = mode == 0 ? (v[i] > thr ? 1u : (v[i] < -thr ? 2u : 0u))
                                 : (v[i] == 1.f ? 1u : (v[i] == -1.f ? 2u : 0u));
    word |= c << (2 * i);
  }
  if (ok) {
    packed[static_cast<int64_t>(r) * LPR + w] = static_cast<int32_t>(word);
    if (w == 0 && scale) scale[r] = gamma;
  }
}

template <typename T>
int launch_pack_rows(const T* x, int64_t xs0, int rows, int D, int mode, int32_t* packed, float* scale,
                     hipStream_t s) {
  const int lpr = D / 16;
  const long long threads = static_cast<long long>(rows) * lpr;
  const unsigned g = static_cast<unsigned>((threads + 255) / 256);
  switch (lpr) {
    case 1: hipLaunchKernelGGL((ternary_pack_rows_kernel<T, 1>), dim3(g), dim3(256), 0, s, x, xs0, rows, mode, packed, scale); break;
    case 2: hipLaunchKernelGGL((ternary_pack_rows_kernel<T, 2>), dim3(g), dim3(256), 0, s, x, xs0, rows, mode, packed, scale); break;
    case 4: hipLaunchKernelGGL((ternary_pack_rows_kernel<T, 4>), dim3(g), dim3(256), 0, s, x, xs0, rows, mode, packed, scale); break;
    case 8: hipLaunchKernelGGL((ternary_pack_rows_kernel<T, 8>), dim3(g), dim3(256), 0, s, x, xs0, rows, mode, packed, scale); break;
    case 16: hipLaunchKernelGGL((ternary_pack_rows_kernel<T, 16>), dim3(g), dim3(256), 0, s, x, xs0, rows, mode, packed, scale); break;
    case 32: hipLaunchKernelGGL((ternary_pack_rows_kernel<T, 32>), dim3(g), dim3(256), 0, s, x, xs0, rows, mode, packed, scale); break;
    default: hipLaunchKernelGGL((ternary_pack_rows_kernel<T, 64>), dim3(g), dim3(256), 0, s, x, xs0, rows, mode, packed, scale); break;
  }
  return check_launch("ternary pack kernel");
}

}  // namespace
}  // namespace sa

extern "C" int sa_ternary_pack(const void* x, int dtype, const int64_t* strides, int rows, int D, int mode,
                               int32_t* packed, float* scale, void* stream) {
  using namespace sa;
  if (rows < 0 || D <= 0 || D % 16 != 0) return fail(SA_EINVAL, "D must be a positive multiple of 16");
  if (mode != 0 && mode != 1) return fail(SA_EINVAL, "mode must be 0 (quantize) or 1 (exact)");
  if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16) {
    return fail(SA_EINVAL, "dtype must be f32, bf16 or f16");
  }
  if (rows == 0) return SA_OK;
  if (!x || !strides || !packed) return fail(SA_EINVAL, "NULL argument");
  hipStream_t s = as_stream(stream);
  // Vector path: D / 16 a power of two <= 64, unit element stride, 16-byte aligned rows.
  const int lpr = D / 16;
  const int64_t esz = dtype == SA_DTYPE_F32 ? 4 : 2;
  if ((lpr & (lpr - 1)) == 0 && lpr <= 64 && strides[1] == 1 && (strides[0] * esz) % 16 == 0 &&
      (reinterpret_cast<uintptr_t>(x) & 15u) == 0 && static_cast<long long>(rows) * lpr < (1LL << 31)) {
    if (dtype == SA_DTYPE_F32) return launch_pack_rows(static_cast<const float*>(x), strides[0], rows, D, mode, packed, scale, s);
    if (dtype == SA_DTYPE_BF16) return launch_pack_rows(static_cast<const bf16_t*>(x), strides[0], rows, D, mode, packed, scale, s);
    return launch_pack_rows(static_cast<const f16_t*>(x), strides[0], rows, D, mode, packed, scale, s);
  }
  const unsigned g = static_cast<unsigned>((static_cast<long long>(rows) + 3) / 4);
  if (dtype == SA_DTYPE_F32)
    hipLaunchKernelGGL((ternary_pack_kernel<float>), dim3(g), dim3(256), 0, s, static_cast<const float*>(x),
                       strides[0], strides[1], rows, D, mode, packed, scale);
  else if (dtype == SA_DTYPE_BF16)
    hipLaunchKernelGGL((ternary_pack_kernel<bf16_t>), dim3(g), dim3(256), 0, s, static_cast<const bf16_t*>(x),
                       strides[0], strides[1], rows, D, mode, packed, scale);
  else
    hipLaunchKernelGGL((ternary_pack_kernel<f16_t>), dim3(g), dim3(256), 0, s, static_cast<const f16_t*>(x),
                       strides[0], strides[1], rows, D, mode, packed, scale);
  return check_launch("ternary pack kernel");
}

extern "C" int sa_ternary_prefill_fwd(const void* q, const int32_t* k_packed, const int32_t* v_packed,
                                      const void* k_scale, const void* v_scale, int scale_dtype,
                                      const int32_t* lists, const int32_t* counts, int max_count, void* out,
                                      int Z, int H, int H_kv, int N, int D, int shift_size,
                                      const int64_t* q_strides, const int64_t* kp_strides,
                                      const int64_t* vp_strides, const int64_t* ks_strides,
                                      const int64_t* vs_strides, const int64_t* o_strides, void* stream) {
  using namespace sa;
  if (Z < 0 || H < 0 || N < 0 || H_kv <= 0 || (H > 0 && H % H_kv != 0)) return fail(SA_EINVAL, "bad Z/H/H_kv/N");
  if (D != 32 && D != 64 && D != 128) return fail(SA_EUNSUPPORTED, "ternary prefill supports D in {32, 64, 128}");
  if (shift_size < 0 || shift_size > N) return fail(SA_EINVAL, "shift_size must lie in [0, N]");
  if (scale_dtype != SA_DTYPE_F32 && scale_dtype != SA_DTYPE_BF16 && scale_dtype != SA_DTYPE_F16) {
    return fail(SA_EINVAL, "scale dtype must be f32, bf16 or f16");
  }
  if (max_count < 0) return fail(SA_EINVAL, "max_count must be >= 0");
  if (static_cast<long long>(Z) * H * N == 0) return SA_OK;
  if (!q || !k_packed || !v_packed || !k_scale || !v_scale || !counts || !out || (!lists && max_count > 0)) {
    return fail(SA_EINVAL, "NULL tensor argument");
  }
  const int64_t* st[6] = {q_strides, kp_strides, vp_strides, ks_strides, vs_strides, o_strides};
  for (const int64_t* x : st) {
    if (!x) return fail(SA_EINVAL, "NULL strides");
  }
  if (q_strides[3] != 1 || o_strides[3] != 1 || kp_strides[3] != 1 || vp_strides[3] != 1) {
    return fail(SA_EUNSUPPORTED, "q / out / packed K / packed V need unit stride along the last dimension");
  }
  for (int i = 0; i < 3; ++i) {
    if (q_strides[i] % 8 != 0 || o_strides[i] % 8 != 0) {
      return fail(SA_EUNSUPPORTED, "q / out rows must be 16-byte aligned");
    }
  }
  if ((reinterpret_cast<uintptr_t>(q) & 15u) || (reinterpret_cast<uintptr_t>(out) & 15u)) {
    return fail(SA_EUNSUPPORTED, "q / out base pointers must be 16-byte aligned");
  }
  TernParams p{};
  p.q = q; p.kp = k_packed; p.vp = v_packed; p.ks = k_scale; p.vs = v_scale; p.scale_dtype = scale_dtype;
  p.lists = lists; p.counts = counts; p.out = out;
  p.qs0 = q_strides[0]; p.qs1 = q_strides[1]; p.qs2 = q_strides[2];
  p.kps0 = kp_strides[0]; p.kps1 = kp_strides[1]; p.kps2 = kp_strides[2];
  p.vps0 = vp_strides[0]; p.vps1 = vp_strides[1]; p.vps2 = vp_strides[2];
  p.kss0 = ks_strides[0]; p.kss1 = ks_strides[1]; p.kss2 = ks_strides[2];
  p.vss0 = vs_strides[0]; p.vss1 = vs_strides[1]; p.vss2 = vs_strides[2];
  p.os0 = o_strides[0]; p.os1 = o_strides[1]; p.os2 = o_strides[2];
  p.Z = Z; p.H = H; p.Hkv = H_kv; p.N = N; p.NB = (N + 127) / 128; p.max_count = max_count;
  p.group = H / H_kv; p.shift = shift_size;
  p.qk_scale = kLog2e / sqrtf(static_cast<float>(D));
  p.mtiles = p.NB;
  const long long wg = static_cast<long long>(Z) * H * p.mtiles;
  if (wg > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  p.total_wg = static_cast<int>(wg);
  hipStream_t s = as_stream(stream);
  if (D == 32) hipLaunchKernelGGL((ternary_prefill_kernel<32>), dim3(p.total_wg), dim3(256), 0, s, p);
  else if (D == 64) hipLaunchKernelGGL((ternary_prefill_kernel<64>), dim3(p.total_wg), dim3(256), 0, s, p);
  else hipLaunchKernelGGL((ternary_prefill_kernel<128>), dim3(p.total_wg), dim3(256), 0, s, p);
  return check_launch("ternary prefill kernel");
}
