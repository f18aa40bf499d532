// Block-sparse attention backward over block lists (gfx950).
//
// Semantics follow _block_list_attention_bwd and its two Triton kernels
// (src/ultrametric/block_list.py:494-681, :758-880):
//   delta_i = sum_d dO[i,d] O[i,d]                        (fp32)
//   p_ij    = exp2(s_ij - lse_i log2 e)  over visible pairs, s_ij the scaled
//             score (+ the listed block's soft bias) in log2 units, lse the
//             forward's natural-log LSE (rows with lse = -inf use 0)
//   ds_ij   = p_ij (dO_i . V_j - delta_i)
//   dQ_i   += sm_scale ds_ij K_j          (over the row's listed key blocks)
//   dK_j   += sm_scale ds_ij Q_i, dV_j += p_ij dO_i
//             (over the query blocks that list j's key block: transposed lists)
//   dbias[qb, t] = sum over the rows of qb and the keys of block list[qb][t]
//             of ds_ij (the straight-through gradient of the soft block bias).
// GQA: a kv head accumulates dK / dV over the H / H_kv query heads that read it.
//
// Kernels (fp32 arithmetic for every element type; 16 lanes per row, D/16
// elements per lane, tiles of 16 rows staged in LDS as fp32):
//   bwd_delta_kernel — one 16-lane group per row.
//   bwd_dq_kernel    — one workgroup per 16 query rows; walks the row block's
//                      list, 16 keys at a time; per (row block, list slot)
//                      the soft-bias gradient is summed over the workgroup
//                      and added with one float atomic per wave.
//   bwd_dkdv_kernel  — one workgroup per 16 key rows of one kv head; walks the
//                      transposed list of each query head of the group, 16
//                      query rows at a time.
#include "sa_internal.h"

namespace sa {
namespace {

struct BwdParams {
  const void* q;
  const void* k;
  const void* v;
  const void* o;
  const void* dout;
  const float* lse;
  const int32_t* lists;
  const int32_t* counts;
  const int32_t* tlists;
  const int32_t* tcounts;
  const void* sb;
  int sb_dtype;
  float* delta;
  void* dq;
  void* dk;
  void* dv;
  float* dsb;
  int64_t sbs[4];
  int64_t qs[4], ks[4], vs[4], os[4], dos[4], dqs[4], dks[4], dvs[4];
  int Z, H, Hkv, N, RB, NB, max_count, t_max, group;
  float qk_scale;   // sm_scale * log2(e)
  float sm_scale;
  int is_causal;
  int tiles;        // 16-row tiles per (z, head)
};

__device__ __forceinline__ float bias_at(const BwdParams& p, int z, int h, int qb, int t) {
  const int64_t off = z * p.sbs[0] + h * p.sbs[1] + qb * p.sbs[2] + t * p.sbs[3];
  if (p.sb_dtype == SA_DTYPE_F32) return static_cast<const float*>(p.sb)[off] * kLog2e;
  if (p.sb_dtype == SA_DTYPE_BF16) return Elem<bf16_t>::load(static_cast<const bf16_t*>(p.sb) + off) * kLog2e;
  return Elem<f16_t>::load(static_cast<const f16_t*>(p.sb) + off) * kLog2e;
}

template <typename T>
__device__ __forceinline__ const T* at(const void* base, const int64_t* st, int z, int h, int row) {
  return static_cast<const T*>(base) + z * st[0] + h * st[1] + row * st[2];
}

template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_delta_kernel(BwdParams p) {
  constexpr int DPL = D / 16;
  const int tid = threadIdx.x, ri = tid / 16, sub = tid % 16;
  const int64_t grow = static_cast<int64_t>(blockIdx.x) * 16 + ri;   // (z, h, row) flattened
  const int64_t rows = static_cast<int64_t>(p.Z) * p.H * p.N;
  if (grow >= rows) return;
  const int i = static_cast<int>(grow % p.N);
  const int zh = static_cast<int>(grow / p.N);
  const int z = zh / p.H, h = zh % p.H;
  const T* op = at<T>(p.o, p.os, z, h, i);
  const T* dp = at<T>(p.dout, p.dos, z, h, i);
  float acc = 0.f;
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = e * 16 + sub;
    acc = fmaf(Elem<T>::load(op + d * p.os[3]), Elem<T>::load(dp + d * p.dos[3]), acc);
  }
  acc = row16_sum(acc);
  if (sub == 0) p.delta[grow] = acc;
}

template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_dq_kernel(BwdParams p) {
  constexpr int DPL = D / 16;
  __shared__ float kt[16][D];
  __shared__ float vt[16][D];
  const int work = xcd_remap(blockIdx.x, p.Z * p.H * p.tiles);
  const int zh = work / p.tiles;
  const int mt = p.tiles - 1 - work % p.tiles;
  const int z = zh / p.H, h = zh % p.H, kvh = h / p.group;
  const int tid = threadIdx.x, qi = tid / 16, sub = tid % 16;
  const int lane = tid & 63;
  const int m0 = mt * 16, qpos = m0 + qi;
  const bool qvalid = qpos < p.N;
  const int qb = m0 / p.RB;
  const int64_t row = static_cast<int64_t>(zh) * p.NB + qb;
  const int count = min(max(p.counts[row], 0), p.max_count);
  const int32_t* list = p.lists + row * p.max_count;

  float qv[DPL], dov[DPL], dq[DPL];
  const int qr = qvalid ? qpos : 0;
  const T* qp = at<T>(p.q, p.qs, z, h, qr);
  const T* dop = at<T>(p.dout, p.dos, z, h, qr);
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = e * 16 + sub;
    qv[e] = qvalid ? Elem<T>::load(qp + d * p.qs[3]) : 0.f;
    dov[e] = qvalid ? Elem<T>::load(dop + d * p.dos[3]) : 0.f;
    dq[e] = 0.f;
  }
  const float lse = qvalid ? p.lse[static_cast<int64_t>(zh) * p.N + qpos] : -INFINITY;
  const float lse2 = lse == -INFINITY ? 0.f : lse * kLog2e;
  const float delta = qvalid ? p.delta[static_cast<int64_t>(zh) * p.N + qpos] : 0.f;
  const T* kb0 = at<T>(p.k, p.ks, z, kvh, 0);
  const T* vb0 = at<T>(p.v, p.vs, z, kvh, 0);
  const int q_last = m0 + 15;

  for (int t = 0; t < count; ++t) {
    const int kb = list[t];
    const float bias = p.sb ? bias_at(p, z, h, qb, t) : 0.f;
    float db = 0.f;
    for (int s0 = 0; s0 < p.RB; s0 += 16) {
      const int key0 = kb * p.RB + s0;
      if (static_cast<unsigned>(key0) >= static_cast<unsigned>(p.N)) break;
      if (p.is_causal && key0 > q_last) break;
      __syncthreads();
      for (int idx = tid; idx < 16 * D; idx += 256) {
        const int j = idx / D, d = idx % D, key = key0 + j;
        const bool ok = key < p.N;
        kt[j][d] = ok ? Elem<T>::load(kb0 + key * p.ks[2] + d * p.ks[3]) : 0.f;
        vt[j][d] = ok ? Elem<T>::load(vb0 + key * p.vs[2] + d * p.vs[3]) : 0.f;
      }
      __syncthreads();
#pragma unroll 4
      for (int j = 0; j < 16; ++j) {
        float sd = 0.f, pd = 0.f;
#pragma unroll
        for (int e = 0; e < DPL; ++e) {
          sd = fmaf(qv[e], kt[j][e * 16 + sub], sd);
          pd = fmaf(dov[e], vt[j][e * 16 + sub], pd);
        }
        sd = row16_sum(sd);
        pd = row16_sum(pd);
        const int key = key0 + j;
        const bool keep = qvalid && key < p.N && (!p.is_causal || key <= qpos);
        const float pij = keep ? fast_exp2(sd * p.qk_scale + bias - lse2) : 0.f;
        const float ds = pij * (pd - delta);
        db += ds;
        const float dss = ds * p.sm_scale;
#pragma unroll
        for (int e = 0; e < DPL; ++e) dq[e] = fmaf(dss, kt[j][e * 16 + sub], dq[e]);
      }
    }
    if (p.sb && p.dsb) {
      // db is the same on the 16 lanes of a row: sum the wave's 4 rows.
      float w = db;
      w += __shfl_xor(w, 16);
      w += __shfl_xor(w, 32);
      if (lane == 0 && w != 0.f) atomicAdd(p.dsb + row * p.max_count + t, w);
    }
  }
  if (qvalid) {
    T* out = static_cast<T*>(p.dq) + z * p.dqs[0] + h * p.dqs[1] + qpos * p.dqs[2];
#pragma unroll
    for (int e = 0; e < DPL; ++e) Elem<T>::store(out + (e * 16 + sub) * p.dqs[3], dq[e]);
  }
}

template <typename T, int D>
__global__ __launch_bounds__(256) void bwd_dkdv_kernel(BwdParams p) {
  constexpr int DPL = D / 16;
  __shared__ float qt[16][D];
  __shared__ float dot[16][D];
  __shared__ float lse2s[16];
  __shared__ float dels[16];
  const int work = xcd_remap(blockIdx.x, p.Z * p.Hkv * p.tiles);
  const int zk = work / p.tiles;
  const int nt = work % p.tiles;
  const int z = zk / p.Hkv, kvh = zk % p.Hkv;
  const int tid = threadIdx.x, ki = tid / 16, sub = tid % 16;
  const int n0 = nt * 16, kpos = n0 + ki;
  const bool kvalid = kpos < p.N;
  const int kb = n0 / p.RB;
  const int kr = kvalid ? kpos : 0;
  float kv[DPL], vv[DPL], dk[DPL], dv[DPL];
  const T* kp = at<T>(p.k, p.ks, z, kvh, kr);
  const T* vp = at<T>(p.v, p.vs, z, kvh, kr);
#pragma unroll
  for (int e = 0; e < DPL; ++e) {
    const int d = e * 16 + sub;
    kv[e] = kvalid ? Elem<T>::load(kp + d * p.ks[3]) : 0.f;
    vv[e] = kvalid ? Elem<T>::load(vp + d * p.vs[3]) : 0.f;
    dk[e] = 0.f;
    dv[e] = 0.f;
  }

  for (int g = 0; g < p.group; ++g) {
    const int h = kvh * p.group + g;
    const int zh = z * p.H + h;
    const int64_t trow = static_cast<int64_t>(zh) * p.NB + kb;
    const int qcount = min(max(p.tcounts[trow], 0), p.t_max);
    const int32_t* tl = p.tlists + trow * p.t_max;
    const T* qb0 = at<T>(p.q, p.qs, z, h, 0);
    const T* db0 = at<T>(p.dout, p.dos, z, h, 0);
    for (int tq = 0; tq < qcount; ++tq) {
      const int qb = tl[tq];
      float bias = 0.f;
      if (p.sb) {
        // The bias of the pair (qb, kb) sits at kb's slot in qb's forward list.
        const int64_t frow = static_cast<int64_t>(zh) * p.NB + qb;
        const int fc = min(max(p.counts[frow], 0), p.max_count);
        const int32_t* fl = p.lists + frow * p.max_count;
        for (int ft = 0; ft < fc; ++ft) {
          if (fl[ft] == kb) {
            bias = bias_at(p, z, h, qb, ft);
            break;
          }
        }
      }
      for (int r0 = 0; r0 < p.RB; r0 += 16) {
        const int row0 = qb * p.RB + r0;
        if (static_cast<unsigned>(row0) >= static_cast<unsigned>(p.N)) break;
        if (p.is_causal && row0 + 15 < n0) continue;   // every row precedes every key of the tile
        __syncthreads();
        for (int idx = tid; idx < 16 * D; idx += 256) {
          const int i = idx / D, d = idx % D, r = row0 + i;
          const bool ok = r < p.N;
          qt[i][d] = ok ? Elem<T>::load(qb0 + r * p.qs[2] + d * p.qs[3]) : 0.f;
          dot[i][d] = ok ? Elem<T>::load(db0 + r * p.dos[2] + d * p.dos[3]) : 0.f;
        }
        if (tid < 16) {
          const int r = row0 + tid;
          const float l = r < p.N ? p.lse[static_cast<int64_t>(zh) * p.N + r] : -INFINITY;
          lse2s[tid] = l == -INFINITY ? 0.f : l * kLog2e;
          dels[tid] = r < p.N ? p.delta[static_cast<int64_t>(zh) * p.N + r] : 0.f;
        }
        __syncthreads();
#pragma unroll 4
        for (int i = 0; i < 16; ++i) {
          float sd = 0.f, pd = 0.f;
#pragma unroll
          for (int e = 0; e < DPL; ++e) {
            sd = fmaf(qt[i][e * 16 + sub], kv[e], sd);
            pd = fmaf(dot[i][e * 16 + sub], vv[e], pd);
          }
          sd = row16_sum(sd);
          pd = row16_sum(pd);
          const int r = row0 + i;
          const bool keep = kvalid && r < p.N && (!p.is_causal || r >= kpos);
          const float pij = keep ? fast_exp2(sd * p.qk_scale + bias - lse2s[i]) : 0.f;
          const float ds = pij * (pd - dels[i]) * p.sm_scale;
#pragma unroll
          for (int e = 0; e < DPL; ++e) {
            dv[e] = fmaf(pij, dot[i][e * 16 + sub], dv[e]);
            dk[e] = fmaf(ds, qt[i][e * 16 + sub], dk[e]);
          }
        }
      }
    }
  }
  if (kvalid) {
    T* kout = static_cast<T*>(p.dk) + z * p.dks[0] + kvh * p.dks[1] + kpos * p.dks[2];
    T* vout = static_cast<T*>(p.dv) + z * p.dvs[0] + kvh * p.dvs[1] + kpos * p.dvs[2];
#pragma unroll
    for (int e = 0; e < DPL; ++e) {
      Elem<T>::store(kout + (e * 16 + sub) * p.dks[3], dk[e]);
      Elem<T>::store(vout + (e * 16 + sub) * p.dvs[3], dv[e]);
    }
  }
}

template <typename T, int D>
int launch_bwd_d(BwdParams& p, hipStream_t s) {
  const long long rows = static_cast<long long>(p.Z) * p.H * p.N;
  const long long g_delta = (rows + 15) / 16;
  const long long g_dq = static_cast<long long>(p.Z) * p.H * p.tiles;
  const long long g_dkdv = static_cast<long long>(p.Z) * p.Hkv * p.tiles;
  if (g_delta > 0x7fffffffLL || g_dq > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  hipLaunchKernelGGL((bwd_delta_kernel<T, D>), dim3(static_cast<unsigned>(g_delta)), dim3(256), 0, s, p);
  int rc = check_launch("block-sparse backward delta kernel");
  if (rc != SA_OK) return rc;
  hipLaunchKernelGGL((bwd_dq_kernel<T, D>), dim3(static_cast<unsigned>(g_dq)), dim3(256), 0, s, p);
  rc = check_launch("block-sparse backward dQ kernel");
  if (rc != SA_OK) return rc;
  hipLaunchKernelGGL((bwd_dkdv_kernel<T, D>), dim3(static_cast<unsigned>(g_dkdv)), dim3(256), 0, s, p);
  return check_launch("block-sparse backward dK/dV kernel");
}

template <typename T>
int launch_bwd(BwdParams& p, int D, hipStream_t s) {
  switch (D) {
    case 16: return launch_bwd_d<T, 16>(p, s);
    case 32: return launch_bwd_d<T, 32>(p, s);
    case 64: return launch_bwd_d<T, 64>(p, s);
    case 128: return launch_bwd_d<T, 128>(p, s);
    default: return launch_bwd_d<T, 256>(p, s);
  }
}

}  // namespace
}  // namespace sa

extern "C" int sa_block_sparse_bwd(const void* q, const void* k, const void* v, const void* out,
                                   const void* dout, const float* lse, const int32_t* lists,
                                   const int32_t* counts, int max_count, const int32_t* t_lists,
                                   const int32_t* t_counts, int t_max_count, const void* soft_bias,
                                   int soft_bias_dtype, const int64_t* sb_strides, float* delta,
                                   void* dq, void* dk, void* dv, float* d_soft_bias, int Z, int H,
                                   int H_kv, int N, int D, int route_block,
                                   const int64_t* q_strides, const int64_t* k_strides,
                                   const int64_t* v_strides, const int64_t* o_strides,
                                   const int64_t* do_strides, const int64_t* dq_strides,
                                   const int64_t* dk_strides, const int64_t* dv_strides,
                                   float sm_scale, int dtype, int is_causal, void* stream) {
  using namespace sa;
  if (Z < 0 || H < 0 || N < 0 || H_kv <= 0 || (H > 0 && H % H_kv != 0)) return fail(SA_EINVAL, "bad Z/H/H_kv/N");
  if (!is_pow2(D) || D < 16) return fail(SA_EINVAL, "head_dim must be a power of two >= 16");
  if (D > 256) return fail(SA_EUNSUPPORTED, "head_dim > 256 is not supported");
  if (!is_pow2(route_block) || route_block < 16) return fail(SA_EINVAL, "route_block must be a power of two >= 16");
  if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16) {
    return fail(SA_EINVAL, "dtype must be f32, bf16 or f16");
  }
  if (max_count < 0 || t_max_count < 0) return fail(SA_EINVAL, "negative list widths");
  if (soft_bias && (!sb_strides || (soft_bias_dtype != SA_DTYPE_F32 && soft_bias_dtype != SA_DTYPE_BF16 &&
                                    soft_bias_dtype != SA_DTYPE_F16))) {
    return fail(SA_EINVAL, "soft_bias needs strides and an f32/bf16/f16 dtype");
  }
  if (static_cast<long long>(Z) * H * N == 0) return SA_OK;
  if (!q || !k || !v || !out || !dout || !lse || !counts || !t_counts || !delta || !dq || !dk || !dv ||
      (!lists && max_count > 0) || (!t_lists && t_max_count > 0)) {
    return fail(SA_EINVAL, "NULL tensor argument");
  }
  const int64_t* st[8] = {q_strides, k_strides, v_strides, o_strides, do_strides, dq_strides, dk_strides, dv_strides};
  for (const int64_t* x : st) {
    if (!x) return fail(SA_EINVAL, "NULL strides");
  }
  BwdParams p{};
  p.q = q; p.k = k; p.v = v; p.o = out; p.dout = dout; p.lse = lse;
  p.lists = lists; p.counts = counts; p.tlists = t_lists; p.tcounts = t_counts;
  p.sb = soft_bias; p.sb_dtype = soft_bias_dtype; p.delta = delta;
  p.dq = dq; p.dk = dk; p.dv = dv; p.dsb = d_soft_bias;
  for (int i = 0; i < 4; ++i) {
    p.sbs[i] = soft_bias ? sb_strides[i] : 0;
    p.qs[i] = q_strides[i]; p.ks[i] = k_strides[i]; p.vs[i] = v_strides[i]; p.os[i] = o_strides[i];
    p.dos[i] = do_strides[i]; p.dqs[i] = dq_strides[i]; p.dks[i] = dk_strides[i]; p.dvs[i] = dv_strides[i];
  }
  p.Z = Z; p.H = H; p.Hkv = H_kv; p.N = N; p.RB = route_block;
  p.NB = (N + route_block - 1) / route_block;
  p.max_count = max_count; p.t_max = t_max_count; p.group = H / H_kv;
  p.qk_scale = sm_scale * kLog2e; p.sm_scale = sm_scale;
  p.is_causal = is_causal != 0;
  p.tiles = (N + 15) / 16;
  hipStream_t s = as_stream(stream);
  if (dtype == SA_DTYPE_F32) return launch_bwd<float>(p, D, s);
  if (dtype == SA_DTYPE_BF16) return launch_bwd<bf16_t>(p, D, s);
  return launch_bwd<f16_t>(p, D, s);
}
