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
// Kernel 1 (decode_split_kernel): one workgroup per (b, kv head, range of
// kPagesPerSplit logical pages). Phase A: one thread per page reads the block
// table entry and the G routing vectors, builds a G-bit head mask, and the
// selected pages are compacted in ascending order into LDS (wave ballot +
// per-wave prefix). Phase B: the 4 waves take selected pages round-robin;
// within a wave, 16 lanes cover one token row of D elements with one vector
// load each and the 4 lane groups take tokens g, g+4, ... of the page; every
// lane group keeps its own online-softmax state per head (base-2), so no
// cross-group traffic happens per page. Phase C: lane groups and waves are
// merged; the (m, l, acc[D]) partial of each head is written to the
// workspace. Kernel 2 (decode_merge_kernel) combines the partials of the
// splits of each (b, h) and writes out.
#include "sa_internal.h"

namespace sa {
namespace {

constexpr int kDecWaves = 4;
constexpr int kDecThreads = kDecWaves * 64;
constexpr int kPagesPerSplit = kDecThreads;  // phase A: one page per thread
constexpr int kMaxTD = 64;
constexpr int kMaxG = 8;

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
  int64_t qs0, qs1, qs2;
  int64_t ks0, ks1, ks2;
  int64_t vs0, vs1, vs2;
  int64_t bts0, bts1;
  int64_t rs0, rs1, rs2;
  int64_t qrs0, qrs1, qrs2;
  int64_t os0, os1, os2;
  float qk_scale;
};

// Load DPL consecutive elements (unit stride, DPL*sizeof(T) aligned) as floats.
template <typename T, int DPL>
__device__ __forceinline__ void load_row(const T* ptr, float (&x)[DPL]) {
  if constexpr (sizeof(T) == 2 && DPL == 8) {
    const uint4 u = *reinterpret_cast<const uint4*>(ptr);
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[2 * i] = Elem<T>::load(reinterpret_cast<const T*>(&w[i]));
      x[2 * i + 1] = Elem<T>::load(reinterpret_cast<const T*>(&w[i]) + 1);
    }
  } else if constexpr (sizeof(T) == 2 && DPL == 4) {
    const uint2 u = *reinterpret_cast<const uint2*>(ptr);
    const uint32_t w[2] = {u.x, u.y};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      x[2 * i] = Elem<T>::load(reinterpret_cast<const T*>(&w[i]));
      x[2 * i + 1] = Elem<T>::load(reinterpret_cast<const T*>(&w[i]) + 1);
    }
  } else if constexpr (sizeof(T) == 4 && DPL % 4 == 0) {
#pragma unroll
    for (int i = 0; i < DPL / 4; ++i) {
      const float4 u = *reinterpret_cast<const float4*>(ptr + 4 * i);
      x[4 * i] = u.x;
      x[4 * i + 1] = u.y;
      x[4 * i + 2] = u.z;
      x[4 * i + 3] = u.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < DPL; ++i) x[i] = Elem<T>::load(ptr + i);
  }
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t ballot) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(ballot >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(ballot), 0u));
}

template <typename T, int D, int G>
__global__ __launch_bounds__(kDecThreads) void decode_split_kernel(DecParams p) {
  constexpr int DPL = D / 16;
  __shared__ int32_t sel_phys[kPagesPerSplit];
  __shared__ int32_t sel_meta[kPagesPerSplit];
  __shared__ int32_t qroute[G][kMaxTD];
  __shared__ int32_t wave_count[kDecWaves];
  __shared__ float red_m[kDecWaves][G];
  __shared__ float red_l[kDecWaves][G];
  __shared__ float red_acc[kDecWaves][G][D];

  const int split = blockIdx.x % p.splits;
  const int bk = blockIdx.x / p.splits;
  const int kvh = bk % p.Hkv;
  const int b = bk / p.Hkv;
  const int ctx = p.ctx[b];
  if (ctx <= 0) return;
  int n = (ctx + p.PS - 1) / p.PS;
  if (n > p.max_pages) n = p.max_pages;  // block table bound (memory safety)
  const int l0 = split * kPagesPerSplit;
  if (l0 >= n) return;
  const int l1 = min(n, l0 + kPagesPerSplit);

  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
  const int h0 = kvh * G;

  for (int i = tid; i < G * p.r; i += kDecThreads) {
    const int g = i / p.r, lev = i % p.r;
    qroute[g][lev] = p.qr[b * p.qrs0 + (h0 + g) * p.qrs1 + lev * p.qrs2];
  }
  __syncthreads();

  // ---- phase A: select and compact ------------------------------------------
  const int l = l0 + tid;
  int mask = 0, phys = 0;
  if (l < l1) {
    phys = p.bt[b * p.bts0 + l * p.bts1];
    if (phys >= 0 && phys < p.P) {
      const bool forced = (p.sink && l == 0) || (p.local > 0 && l >= n - p.local);
#pragma unroll
      for (int g = 0; g < G; ++g) {
        bool m = true;
        if (!forced) {
          const int32_t* rv = p.router + phys * p.rs0 + (h0 + g) * p.rs1;
          for (int lev = 0; lev < p.r; ++lev) {
            if (rv[lev * p.rs2] != qroute[g][lev]) {
              m = false;
              break;
            }
          }
        }
        if (m) mask |= 1 << g;
      }
    }
  }
  const uint64_t bal = __ballot(mask != 0);
  if (lane == 0) wave_count[wave] = __popcll(bal);
  __syncthreads();
  int base = 0, nsel = 0;
#pragma unroll
  for (int w = 0; w < kDecWaves; ++w) {
    if (w < wave) base += wave_count[w];
    nsel += wave_count[w];
  }
  if (mask != 0) {
    const int pos = base + static_cast<int>(lanes_below(bal));
    sel_phys[pos] = phys;
    sel_meta[pos] = (l - l0) | (mask << 16);
  }
  __syncthreads();

  // ---- phase B: gather + attend ---------------------------------------------
  const int grp = lane >> 4, sub = lane & 15;
  float qv[G][DPL];
  float m_s[G], l_s[G], acc[G][DPL];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const T* qp = static_cast<const T*>(p.q) + b * p.qs0 + (h0 + g) * p.qs1 + sub * DPL * p.qs2;
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      qv[g][e] = Elem<T>::load(qp + e * p.qs2);
      acc[g][e] = 0.f;
    }
    m_s[g] = -INFINITY;
    l_s[g] = 0.f;
  }

  for (int i = wave; i < nsel; i += kDecWaves) {
    const int ph = sel_phys[i];
    const int meta = sel_meta[i];
    const int lp = l0 + (meta & 0xffff);
    const int hmask = meta >> 16;
    const int valid = min(p.PS, ctx - lp * p.PS);
    const T* kpage = static_cast<const T*>(p.kc) + ph * p.ks0 + kvh * p.ks1 + sub * DPL;
    const T* vpage = static_cast<const T*>(p.vc) + ph * p.vs0 + kvh * p.vs1 + sub * DPL;
    for (int tc = 0; tc < p.PS; tc += 16) {
      float kx[4][DPL], vx[4][DPL];
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int tok = tc + 4 * it + grp;
        if (tok < valid) {
          load_row<T, DPL>(kpage + tok * p.ks2, kx[it]);
          load_row<T, DPL>(vpage + tok * p.vs2, vx[it]);
        } else {
#pragma unroll
          for (int e = 0; e < DPL; ++e) kx[it][e] = vx[it][e] = 0.f;
        }
      }
#pragma unroll
      for (int g = 0; g < G; ++g) {
        if (!((hmask >> g) & 1)) continue;
        float s[4];
        float mloc = -INFINITY;
#pragma unroll
        for (int it = 0; it < 4; ++it) {
          float part = 0.f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) part = fmaf(qv[g][e], kx[it][e], part);
          const float sc = row16_sum(part) * p.qk_scale;
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
          for (int e = 0; e < DPL; ++e) acc[g][e] = fmaf(pv, vx[it][e], acc[g][e]);
        }
        l_s[g] = lsum;
        m_s[g] = m_new;
      }
    }
  }

  // ---- phase C: merge lane groups, then waves ----------------------------------
#pragma unroll
  for (int g = 0; g < G; ++g) {
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
    float* dst = p.part + ((static_cast<int64_t>(b) * p.H + h0 + g) * p.splits + split) * (D + 2);
    dst[2 + d] = a;
    if (d == 0) {
      dst[0] = mx;
      dst[1] = lsum;
    }
  }
}

template <typename T>
__global__ __launch_bounds__(256) void decode_merge_kernel(DecParams p) {
  const int bh = blockIdx.x;
  const int b = bh / p.H, h = bh % p.H;
  const int D = p.D;
  T* op = static_cast<T*>(p.out) + b * p.os0 + h * p.os1;
  const int ctx = p.ctx[b];
  int n = ctx > 0 ? (ctx + p.PS - 1) / p.PS : 0;
  if (n > p.max_pages) n = p.max_pages;
  const int nsplit = (n + kPagesPerSplit - 1) / kPagesPerSplit;
  const float* src = p.part + static_cast<int64_t>(bh) * p.splits * (D + 2);
  float mx = -INFINITY;
  for (int s = 0; s < nsplit; ++s) mx = fmaxf(mx, src[s * (D + 2)]);
  const float mref = mx == -INFINITY ? 0.f : mx;
  float lsum = 0.f;
  for (int s = 0; s < nsplit; ++s) lsum += src[s * (D + 2) + 1] * fast_exp2(src[s * (D + 2)] - mref);
  for (int d = threadIdx.x; d < D; d += blockDim.x) {
    float a = 0.f;
    for (int s = 0; s < nsplit; ++s) a += src[s * (D + 2) + 2 + d] * fast_exp2(src[s * (D + 2)] - mref);
    Elem<T>::store(op + d * p.os2, lsum > 0.f ? a / lsum : 0.f);
  }
}

template <typename T, int D>
void launch_split_d(DecParams& p, dim3 g, hipStream_t s) {
  switch (p.G) {
    case 1: hipLaunchKernelGGL((decode_split_kernel<T, D, 1>), g, dim3(kDecThreads), 0, s, p); break;
    case 2: hipLaunchKernelGGL((decode_split_kernel<T, D, 2>), g, dim3(kDecThreads), 0, s, p); break;
    case 4: hipLaunchKernelGGL((decode_split_kernel<T, D, 4>), g, dim3(kDecThreads), 0, s, p); break;
    default: hipLaunchKernelGGL((decode_split_kernel<T, D, 8>), g, dim3(kDecThreads), 0, s, p); break;
  }
}

template <typename T>
int launch_decode(DecParams& p, hipStream_t s) {
  const long long wg = static_cast<long long>(p.B) * p.Hkv * p.splits;
  if (wg > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  dim3 g(static_cast<unsigned>(wg));
  if (wg > 0) {
    switch (p.D) {
      case 16: launch_split_d<T, 16>(p, g, s); break;
      case 32: launch_split_d<T, 32>(p, g, s); break;
      case 64: launch_split_d<T, 64>(p, g, s); break;
      case 128: launch_split_d<T, 128>(p, g, s); break;
      default: launch_split_d<T, 256>(p, g, s); break;
    }
    int rc = check_launch("sparse paged decode kernel");
    if (rc != SA_OK) return rc;
  }
  hipLaunchKernelGGL((decode_merge_kernel<T>), dim3(p.B * p.H), dim3(64), 0, s, p);
  return check_launch("sparse paged decode merge kernel");
}

int splits_for(int max_pages) { return max_pages <= 0 ? 1 : (max_pages + kPagesPerSplit - 1) / kPagesPerSplit; }

}  // namespace
}  // namespace sa

extern "C" size_t sa_decode_workspace_bytes(int B, int H, int D, int max_pages) {
  if (B <= 0 || H <= 0 || D <= 0) return 0;
  return static_cast<size_t>(B) * H * sa::splits_for(max_pages) * (D + 2) * sizeof(float);
}

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
  using namespace sa;
  if (B < 0 || H < 0 || H_kv <= 0 || (H > 0 && H % H_kv != 0)) return fail(SA_EINVAL, "bad B/H/H_kv");
  const int G = H > 0 ? H / H_kv : 1;
  if (G != 1 && G != 2 && G != 4 && G != 8) {
    return fail(SA_EUNSUPPORTED, "query heads per kv head must be 1, 2, 4 or 8");
  }
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
  if (!q || !k_cache || !v_cache || !block_tables || !context_lens || !router || !q_router || !out) {
    return fail(SA_EINVAL, "NULL tensor argument");
  }
  if (!q_strides || !k_strides || !v_strides || !bt_strides || !r_strides || !qr_strides || !o_strides) {
    return fail(SA_EINVAL, "NULL strides");
  }
  if (k_strides[3] != 1 || v_strides[3] != 1) {
    return fail(SA_EUNSUPPORTED, "k_cache / v_cache need unit stride along head_dim");
  }
  // Each lane loads D/16 consecutive elements with one vector load (at most
  // 16 bytes), so rows and base pointers must be aligned to that size.
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
  const size_t need = sa_decode_workspace_bytes(B, H, D, max_pages);
  if (!workspace || workspace_bytes < need) {
    return fail(SA_EINVAL, "workspace too small: need " + std::to_string(need) + " bytes");
  }

  DecParams p{};
  p.q = q; p.kc = k_cache; p.vc = v_cache; p.bt = block_tables; p.ctx = context_lens;
  p.router = router; p.qr = q_router; p.out = out; p.part = static_cast<float*>(workspace);
  p.B = B; p.H = H; p.Hkv = H_kv; p.D = D; p.PS = page_size; p.TD = TD;
  p.max_pages = max_pages; p.P = num_phys_pages;
  p.r = req_depth < 0 ? 0 : (req_depth > TD ? TD : req_depth);
  p.local = local_blocks; p.sink = sink_block != 0; p.G = G;
  p.splits = splits_for(max_pages);
  p.qs0 = q_strides[0]; p.qs1 = q_strides[1]; p.qs2 = q_strides[2];
  p.ks0 = k_strides[0]; p.ks1 = k_strides[1]; p.ks2 = k_strides[2];
  p.vs0 = v_strides[0]; p.vs1 = v_strides[1]; p.vs2 = v_strides[2];
  p.bts0 = bt_strides[0]; p.bts1 = bt_strides[1];
  p.rs0 = r_strides[0]; p.rs1 = r_strides[1]; p.rs2 = r_strides[2];
  p.qrs0 = qr_strides[0]; p.qrs1 = qr_strides[1]; p.qrs2 = qr_strides[2];
  p.os0 = o_strides[0]; p.os1 = o_strides[1]; p.os2 = o_strides[2];
  p.qk_scale = (1.0f / sqrtf(static_cast<float>(D))) * kLog2e;
  hipStream_t s = as_stream(stream);
  if (dtype == SA_DTYPE_F32) return launch_decode<float>(p, s);
  if (dtype == SA_DTYPE_BF16) return launch_decode<bf16_t>(p, s);
  return launch_decode<f16_t>(p, s);
}
