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
#include "mfma_util.h"

#include <algorithm>
#include <type_traits>

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
  // MFMA path
  const int4* work;        // dK/dV work items {tile, chunk, partial slot or -1, entries}
  const int4* multi;       // split tiles {tile, first item, items, 0}
  const float* t_bias;     // soft bias per transposed entry (log2 units) or NULL
  int2* ent_rh;            // per work item, `chunk` entries {first query row, head}
  float* ent_b;            // per work item, `chunk` entries: soft bias (log2 units)
  float* partials;         // fp32 dK / dV partials of the items of split tiles
  int n_work, n_multi;
  int ktiles;              // key tiles per (z, kv head)
  int key_tile;            // keys per key tile
  int chunk;               // transposed entries per work item
  int mtiles;              // query tiles per (z, head) of the dQ kernel
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

// ============================================================================
// MFMA kernels (bf16 / fp16, D in {32, 64, 128}, route_block % 32 == 0).
//   bwd_dq_mfma_kernel   — NW waves own 32 query rows each (one route block
//       slice, as the forward); K / V tiles of 32 keys stream through a
//       3-stage direct-to-LDS ring. S^T = K Q^T and dP^T = V dO^T (lane =
//       query, 16 keys per lane), dS^T in registers, dQ^T += K^T dS^T with K^T
//       from transposing LDS reads.
//   bwd_dkdv_mfma_kernel — one work item: NW waves own 32 keys each of one
//       key tile; K and V stay in registers as MFMA operands; Q / dO tiles of
//       32 query rows (+ their lse and delta) stream through the ring.
//       S = Q K^T and dP = dO V^T (lane = key, 16 queries per lane),
//       dV^T += dO^T P and dK^T += Q^T dS. A work item covers at most
//       `chunk` transposed-list entries; the items of a key tile with more
//       entries write fp32 partials that bwd_finalize_kernel sums.
//   bwd_plan_kernel      — builds the work list (split tiles first, then the
//       others by decreasing entry count) from the transposed counts;
//       bwd_items_kernel then resolves each item's entries.
// ============================================================================
constexpr int kBwdSeg = 256;        // dQ: list entries staged in LDS at a time
constexpr int kChunkStages = 64;    // dK/dV: 32-row query stages per work item
constexpr int kMaxChunk = 64;       // entries per work item (route_block 32); one wave resolves them

// Chunk c of row r of a stage tile is stored at position c ^ bsw(r). Row-major
// operand reads (lanes 0..15 read rows 0..15, one 16-byte chunk each) and
// transposing reads (ds_read_b64_tr_b16: 32 lanes read 4 rows x 64 bytes)
// both fall on distinct banks of the 256-byte bank window. bsw(r + 16) =
// bsw(r); bsw(r + 8) = bsw(r) ^ 2.
template <int D>
__device__ __forceinline__ int bsw(int r) {
  const int sig = D == 128 ? (r & 3) : (D == 64 ? ((r >> 1) & 1) : 0);
  return 4 * sig + ((r >> 2) & 3);
}

// Per-lane direct-to-LDS loads of a pair of 32-row tiles (X, then Y) whose
// rows are stored with bsw. Load i of wave w fills 1-KB block `blk` of X or Y:
// lane L writes slot 64 blk + L = (row, position) and fetches the chunk that
// belongs there.
template <int D, int NW>
struct TilePair {
  static constexpr int ROWB = 2 * D, TILEB = 32 * ROWB, CPR = D / 8, NKI = TILEB / 1024;
  static constexpr int LPW = 2 * NKI / NW;
  static_assert((2 * NKI) % NW == 0 && LPW >= 1, "loads must split evenly over waves");
  uint32_t goff[LPW];

  // Row of the tile that load i of this wave fills (lane dependent).
  static __device__ __forceinline__ int row_of(int wave, int lane, int i) {
    const int q = wave * LPW + i;
    return ((q < NKI ? q : q - NKI) * 64 + lane) / CPR;
  }
  __device__ __forceinline__ void init(int wave, int lane, uint32_t xsb, uint32_t ysb) {
#pragma unroll
    for (int i = 0; i < LPW; ++i) {
      const int q = wave * LPW + i;
      const bool isx = q < NKI;
      const int slot = (isx ? q : q - NKI) * 64 + lane;
      const int r = slot / CPR, pos = slot % CPR;
      goff[i] = __umul24(static_cast<uint32_t>(r), isx ? xsb : ysb) + 16u * (pos ^ bsw<D>(r));
    }
  }
  // Issues rows row0 .. row0 + 31 of X and Y into LDS at dst (X) / dst + TILEB (Y).
  // Rows outside [0, N) read row N - 1 (or 0); the kernels mask them.
  __device__ __forceinline__ void issue(const char* xb, const char* yb, uint32_t xsb, uint32_t ysb, int row0,
                                        int N, uint32_t dst, int wave, int lane) const {
    if (row0 >= 0 && row0 + 32 <= N) {
      const char* xt = xb + static_cast<size_t>(row0) * xsb;
      const char* yt = yb + static_cast<size_t>(row0) * ysb;
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int q = wave * LPW + i;
        const bool isx = q < NKI;
        const uint32_t d = __builtin_amdgcn_readfirstlane(dst + (isx ? 0 : TILEB) + (isx ? q : q - NKI) * 1024);
        dma16_s(isx ? xt : yt, goff[i], d);
      }
    } else {
#pragma unroll
      for (int i = 0; i < LPW; ++i) {
        const int q = wave * LPW + i;
        const bool isx = q < NKI;
        const char* gb = isx ? xb : yb;
        const uint32_t rs = isx ? xsb : ysb;
        const int gr = row_of(wave, lane, i);
        const uint32_t rr = static_cast<uint32_t>(min(max(row0 + gr, 0), N - 1));
        const char* src = gb + __umul24(rr, rs) + (goff[i] - __umul24(static_cast<uint32_t>(gr), rs));
        const uint32_t d = __builtin_amdgcn_readfirstlane(dst + (isx ? 0 : TILEB) + (isx ? q : q - NKI) * 1024);
        dma16(src, d);
      }
    }
  }
};

// Lane byte offsets of the transposing reads that build the A operand
// X^T[d][row] (k index over 32 rows) of tile dt: rows 4 kh + (j >> 2)
// (r0) and 8 + 4 kh + (j >> 2) (r1); the second half of the 32 rows adds 16
// rows (an immediate). MFMA k index 8 kh + e of half s2 is row 16 s2 + 4 kh + e
// (e < 4, r0) or 16 s2 + 8 + 4 kh + e - 4 (r1).
template <int D>
__device__ __forceinline__ void tr_offsets(int lane, uint32_t (&r0)[D / 32], uint32_t (&r1)[D / 32]) {
  constexpr int ROWB = 2 * D;
  const int g = lane >> 4, j = lane & 15, kh = lane >> 5;
  const int vr = 4 * kh + (j >> 2);
#pragma unroll
  for (int dt = 0; dt < D / 32; ++dt) {
    const int c = 4 * dt + 2 * (g & 1) + ((j & 3) >> 1);
    r0[dt] = vr * ROWB + 16 * (c ^ bsw<D>(vr)) + 8 * (j & 1);
    r1[dt] = (vr + 8) * ROWB + 16 * (c ^ bsw<D>(vr + 8)) + 8 * (j & 1);
  }
}

template <typename T, int D>
__device__ __forceinline__ u32x4_t tr_operand(const char* base, uint32_t r0, uint32_t r1, int s2) {
  constexpr int ROWB = 2 * D;
  SA_LDS s16x4_t* a0 = (SA_LDS s16x4_t*)((SA_LDS char*)base + r0 + 16 * s2 * ROWB);
  SA_LDS s16x4_t* a1 = (SA_LDS s16x4_t*)((SA_LDS char*)base + r1 + 16 * s2 * ROWB);
  const u32x2_t lo = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(a0));
  const u32x2_t hi = __builtin_bit_cast(u32x2_t, __builtin_amdgcn_ds_read_tr16_b64_v4i16(a1));
  return u32x4_t{lo[0], lo[1], hi[0], hi[1]};
}

template <typename T> __device__ __forceinline__ float lo_elem(uint32_t w);
template <typename T> __device__ __forceinline__ float hi_elem(uint32_t w);
template <> __device__ __forceinline__ float lo_elem<bf16_t>(uint32_t w) { return bf16_bits_to_float(w & 0xffffu); }
template <> __device__ __forceinline__ float hi_elem<bf16_t>(uint32_t w) { return bf16_bits_to_float(w >> 16); }
template <> __device__ __forceinline__ float lo_elem<f16_t>(uint32_t w) { return f16_bits_to_float(w & 0xffffu); }
template <> __device__ __forceinline__ float hi_elem<f16_t>(uint32_t w) { return f16_bits_to_float(w >> 16); }

template <typename T>
__device__ __forceinline__ u32x4_t pack8(const float* x) {
  return u32x4_t{Mma<T>::pack(x[0], x[1]), Mma<T>::pack(x[2], x[3]), Mma<T>::pack(x[4], x[5]),
                 Mma<T>::pack(x[6], x[7])};
}

__device__ __forceinline__ float wave_sum(float x) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) x += __shfl_xor(x, o);
  return x;
}

template <typename T, int D, int NW, bool CAUSAL>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(2)))
void bwd_dq_mfma_kernel(BwdParams p) {
  using TP = TilePair<D, NW>;
  constexpr int S = 3, BN = 32, NT = NW * 64, BM = NW * 32;
  constexpr int ROWB = 2 * D, TILEB = TP::TILEB, STAGEB = 2 * TILEB;
  constexpr int KS = D / 16, DT = D / 32, LPW = TP::LPW;
  __shared__ __attribute__((aligned(1024))) char stage_lds[S * STAGEB];
  __shared__ int32_t list_lds[kBwdSeg];
  __shared__ float bias_lds[kBwdSeg];
  __shared__ float db_lds[NW][kBwdSeg];   // per-wave soft-bias gradient of each staged entry

  const int work = xcd_remap(blockIdx.x, p.Z * p.H * p.mtiles);
  const int zh = work / p.mtiles;
  const int mt = p.mtiles - 1 - work % p.mtiles;
  const int z = zh / p.H, h = zh % p.H, kvh = h / p.group;
  const int m0 = mt * BM, qb = m0 / p.RB;
  const int64_t row = static_cast<int64_t>(zh) * p.NB + qb;
  const int count = min(max(p.counts[row], 0), p.max_count);
  const int32_t* list = p.lists + row * p.max_count;
  const int spb = p.RB / BN, lspb = __builtin_ctz(spb);
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, li = lane & 31, kh = lane >> 5;
  const int N = p.N;
  const int qw0 = m0 + wave * 32, qpos = qw0 + li, qr = min(qpos, N - 1);
  const bool qok = qpos < N;

  const char* kbase = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + z * p.ks[0] + kvh * p.ks[1]);
  const char* vbase = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + z * p.vs[0] + kvh * p.vs[1]);
  const uint32_t ksb = static_cast<uint32_t>(p.ks[2]) * 2u, vsb = static_cast<uint32_t>(p.vs[2]) * 2u;

  // Q^T and dO^T as B operands: lane (li + 32 kh) holds X[qr][16 s + 8 kh .. +8].
  u32x4_t qf[KS], dof[KS];
  {
    const char* qrow = reinterpret_cast<const char*>(static_cast<const T*>(p.q) + z * p.qs[0] + h * p.qs[1] +
                                                     static_cast<int64_t>(qr) * p.qs[2]);
    const char* drow = reinterpret_cast<const char*>(static_cast<const T*>(p.dout) + z * p.dos[0] +
                                                     h * p.dos[1] + static_cast<int64_t>(qr) * p.dos[2]);
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      qf[s] = *reinterpret_cast<const u32x4_t*>(qrow + 32 * s + 16 * kh);
      dof[s] = *reinterpret_cast<const u32x4_t*>(drow + 32 * s + 16 * kh);
    }
  }
  const float lse = p.lse[static_cast<int64_t>(zh) * N + qr];
  const float lse2 = lse == -INFINITY ? 0.f : lse * kLog2e;
  // delta = rowsum(dO * O) in fp32 (lanes kh = 0 / 1 hold the two halves of
  // the row); stored for the dK / dV kernels.
  float delta;
  {
    const char* orow = reinterpret_cast<const char*>(static_cast<const T*>(p.o) + z * p.os[0] + h * p.os[1] +
                                                     static_cast<int64_t>(qr) * p.os[2]);
    float part = 0.f;
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4_t ov = *reinterpret_cast<const u32x4_t*>(orow + 32 * s + 16 * kh);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        part = fmaf(lo_elem<T>(ov[e]), lo_elem<T>(dof[s][e]), part);
        part = fmaf(hi_elem<T>(ov[e]), hi_elem<T>(dof[s][e]), part);
      }
    }
    delta = part + __shfl_xor(part, 32);
    if (qok && kh == 0) p.delta[static_cast<int64_t>(zh) * N + qpos] = delta;
  }
  const bool want_db = p.sb != nullptr && p.dsb != nullptr;

  TP tp;
  tp.init(wave, lane, ksb, vsb);
  uint32_t rm[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) rm[s] = li * ROWB + 16 * ((2 * s + kh) ^ bsw<D>(li));
  uint32_t tr0[DT], tr1[DT];
  tr_offsets<D>(lane, tr0, tr1);
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SA_LDS char*)stage_lds));

  f32x16_t acc[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16_t{};
  float dbw = 0.f;

  auto compute = [&](int n, int key0, int stg) {
    const bool skip = qw0 >= N || static_cast<unsigned>(key0) >= static_cast<unsigned>(N) ||
                      (CAUSAL && key0 > qw0 + 31);
    if (skip) return;
    const char* sbase = stage_lds + stg * STAGEB;
    f32x16_t st = f32x16_t{}, dp = f32x16_t{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4_t ka = *reinterpret_cast<const u32x4_t*>(sbase + rm[s]);
      st = Mma<T>::mma(ka, qf[s], st);
    }
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4_t va = *reinterpret_cast<const u32x4_t*>(sbase + TILEB + rm[s]);
      dp = Mma<T>::mma(va, dof[s], dp);
    }
    const bool need_mask = !qok || key0 + BN > N || (CAUSAL && key0 + BN - 1 > qw0);
    int lim = 0;
    if (need_mask) {
      lim = qok ? N - 1 - key0 : -1;
      if (CAUSAL && qok) lim = min(lim, qpos - key0);
      lim -= 4 * kh;
    }
    const float nb = bias_lds[n >> lspb] - lse2;
    float ds[16];
#pragma unroll
    for (int v = 0; v < 16; ++v) {
      float pv = fast_exp2(fmaf(st[v], p.qk_scale, nb));
      if (need_mask && 8 * (v >> 2) + (v & 3) > lim) pv = 0.f;
      ds[v] = pv * (dp[v] - delta);
    }
    if (want_db) {
#pragma unroll
      for (int v = 0; v < 16; ++v) dbw += ds[v];
    }
    const u32x4_t pb0 = pack8<T>(ds), pb1 = pack8<T>(ds + 8);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      acc[dt] = Mma<T>::mma(tr_operand<T, D>(sbase, tr0[dt], tr1[dt], 0), pb0, acc[dt]);
      acc[dt] = Mma<T>::mma(tr_operand<T, D>(sbase, tr0[dt], tr1[dt], 1), pb1, acc[dt]);
    }
  };

  for (int seg = 0; seg < count; seg += kBwdSeg) {
    const int seg_n = min(count - seg, kBwdSeg);
    if (seg > 0) __syncthreads();
    for (int t = tid; t < seg_n; t += NT) {
      list_lds[t] = list[seg + t];
      bias_lds[t] = p.sb ? bias_at(p, z, h, qb, seg + t) : 0.f;
    }
    __syncthreads();
    __builtin_amdgcn_s_waitcnt(0);
    const int total = seg_n * spb;
    auto tile_key0 = [&](int m) { return list_lds[m >> lspb] * p.RB + (m & (spb - 1)) * BN; };
    int key_of[S];
#pragma unroll
    for (int st0 = 0; st0 < S - 1; ++st0) {
      key_of[st0] = st0 < total ? tile_key0(st0) : 0;
      if (st0 < total) tp.issue(kbase, vbase, ksb, vsb, key_of[st0], N, lds_base + st0 * STAGEB, wave, lane);
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
        tp.issue(kbase, vbase, ksb, vsb, next_key, N, lds_base + nst * STAGEB, wave, lane);
        if (n + S < total) next_key = tile_key0(n + S);
      }
      compute(n, key_of[stg], stg);
      if (want_db && (n & (spb - 1)) == spb - 1) {
        // LDS only: no vector-memory operation may join the pipeline's loads.
        const float w = wave_sum(dbw);
        if (lane == 0) db_lds[wave][n >> lspb] = w;
        dbw = 0.f;
      }
      ++n;
    };
    while (n < total) {
      step(std::integral_constant<int, 0>{});
      step(std::integral_constant<int, 1>{});
      step(std::integral_constant<int, 2>{});
    }
    if (want_db) {
      wait_vmcnt<0>();
      __syncthreads();
      for (int t = tid; t < seg_n; t += NT) {
        float w = 0.f;
#pragma unroll
        for (int i = 0; i < NW; ++i) w += db_lds[i][t];
        if (w != 0.f) atomicAdd(p.dsb + row * p.max_count + seg + t, w);
      }
    }
  }

  wait_vmcnt<0>();
  if (qok) {
    T* op = static_cast<T*>(p.dq) + z * p.dqs[0] + h * p.dqs[1] + static_cast<int64_t>(qpos) * p.dqs[2];
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * dt + 8 * g + 4 * kh;
        const float sc = p.sm_scale;
        const u32x2_t val{Mma<T>::pack(acc[dt][4 * g] * sc, acc[dt][4 * g + 1] * sc),
                          Mma<T>::pack(acc[dt][4 * g + 2] * sc, acc[dt][4 * g + 3] * sc)};
        *reinterpret_cast<u32x2_t*>(op + d) = val;
      }
    }
  }
}

__global__ void fill_i32_kernel(int32_t* x, int n, int v) {
  if (static_cast<int>(threadIdx.x) < n) x[threadIdx.x] = v;
}

// Transposed entries of key tile `tile` (all query heads of its kv head).
__device__ __forceinline__ int tile_entries(const BwdParams& p, int tile, int BK) {
  const int zk = tile / p.ktiles, nt = tile % p.ktiles;
  const int z = zk / p.Hkv, kvh = zk % p.Hkv;
  const int kb = nt * BK / p.RB;
  int e = 0;
  for (int g = 0; g < p.group; ++g) {
    const int64_t trow = (static_cast<int64_t>(z) * p.H + kvh * p.group + g) * p.NB + kb;
    e += min(max(p.tcounts[trow], 0), p.t_max);
  }
  return e;
}

// One workgroup: split tiles get ceil(E / chunk) items (placed first; each
// writes fp32 partials into slot = its item index), other tiles one item,
// grouped by decreasing entry count. info = {items, split tiles, items of
// split tiles}.
__global__ __launch_bounds__(1024) void bwd_plan_kernel(BwdParams p, int BK, int4* work, int4* multi,
                                                        int32_t* info) {
  __shared__ int hist[kMaxChunk + 1];
  __shared__ int cur[kMaxChunk + 1];
  __shared__ int n_items_multi, n_multi, mcur, scur;
  const int tid = threadIdx.x;
  const int T = p.Z * p.Hkv * p.ktiles;
  const int C = p.chunk;
  if (tid <= C) hist[tid] = 0;
  if (tid == 0) { n_items_multi = 0; n_multi = 0; mcur = 0; scur = 0; }
  __syncthreads();
  for (int t = tid; t < T; t += 1024) {
    const int e = tile_entries(p, t, BK);
    if (e > C) {
      atomicAdd(&n_items_multi, (e + C - 1) / C);
      atomicAdd(&n_multi, 1);
    } else {
      atomicAdd(&hist[e], 1);
    }
  }
  __syncthreads();
  if (tid == 0) {
    int pos = n_items_multi;
    for (int e = C; e >= 0; --e) {
      cur[e] = pos;
      pos += hist[e];
    }
    info[0] = pos;
    info[1] = n_multi;
    info[2] = n_items_multi;
  }
  __syncthreads();
  for (int t = tid; t < T; t += 1024) {
    const int e = tile_entries(p, t, BK);
    if (e > C) {
      const int nc = (e + C - 1) / C;
      const int first = atomicAdd(&mcur, nc);
      const int slot = atomicAdd(&scur, 1);
      for (int c = 0; c < nc; ++c) work[first + c] = int4{t, c, first + c, e};
      multi[slot] = int4{t, first, nc, 0};
    } else {
      const int pos = atomicAdd(&cur[e], 1);
      work[pos] = int4{t, 0, -1, e};
    }
  }
}

// Soft bias of each transposed entry: forward pair (qb, slot t) with key block
// kb lands at qb's position in kb's (ascending) transposed list.
__global__ __launch_bounds__(256) void bwd_tbias_kernel(BwdParams p, float* t_bias) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int64_t total = static_cast<int64_t>(p.Z) * p.H * p.NB * p.max_count;
  if (i >= total) return;
  const int64_t row = i / p.max_count;
  const int t = static_cast<int>(i % p.max_count);
  if (t >= min(max(p.counts[row], 0), p.max_count)) return;
  const int kb = p.lists[i];
  if (kb < 0 || kb >= p.NB) return;
  const int zh = static_cast<int>(row / p.NB), qb = static_cast<int>(row % p.NB);
  const int64_t trow = static_cast<int64_t>(zh) * p.NB + kb;
  const int tc = min(max(p.tcounts[trow], 0), p.t_max);
  const int32_t* tl = p.tlists + trow * p.t_max;
  int lo = 0, hi = tc;
  while (lo < hi) {
    const int mid = (lo + hi) >> 1;
    if (tl[mid] < qb) lo = mid + 1;
    else hi = mid;
  }
  if (lo < tc && tl[lo] == qb) t_bias[trow * p.t_max + lo] = bias_at(p, zh / p.H, zh % p.H, qb, t);
}

// Resolves the transposed entries of each work item once (lane e: entry
// chunk * C + e, walked over the G query heads of the kv head), so that the
// dK / dV workgroups load them with one read. Part of the plan: it runs
// before the item count is read back, so it walks the items up to info[0]
// with a fixed grid, one wave per item.
__device__ __forceinline__ void resolve_entry(const BwdParams& p, int4 item, int w, int e) {
  const int zk = item.x / p.ktiles, nt = item.x % p.ktiles;
  const int z = zk / p.Hkv, kvh = zk % p.Hkv;
  const int kb = nt * p.key_tile / p.RB;
  const int ge = item.y * p.chunk + e;
  int g = 0, acc = 0;
  for (; g < p.group - 1; ++g) {
    const int c = min(max(p.tcounts[(static_cast<int64_t>(z) * p.H + kvh * p.group + g) * p.NB + kb], 0), p.t_max);
    if (ge < acc + c) break;
    acc += c;
  }
  const int h = kvh * p.group + g;
  const int64_t trow = (static_cast<int64_t>(z) * p.H + h) * p.NB + kb;
  const int u = min(max(ge - acc, 0), max(p.t_max - 1, 0));
  const int64_t slot = static_cast<int64_t>(w) * p.chunk + e;
  p.ent_rh[slot] = int2{p.tlists[trow * p.t_max + u] * p.RB, h};
  p.ent_b[slot] = p.t_bias ? p.t_bias[trow * p.t_max + u] : 0.f;
}

__global__ __launch_bounds__(256) void bwd_items_kernel(BwdParams p, const int32_t* info, int max_items) {
  const int n_items = min(info[0], max_items), e = threadIdx.x & 63;
  for (int w = blockIdx.x * 4 + (threadIdx.x >> 6); w < n_items; w += gridDim.x * 4) {
    const int4 item = p.work[w];
    const int ne = max(0, min(item.w - item.y * p.chunk, p.chunk));
    if (e < ne) resolve_entry(p, item, w, e);
  }
}

// PASS 0 accumulates dV (S, P, dV^T += dO^T P; K in registers), PASS 1 dK
// (S, dP, dS, dK^T += Q^T dS; K and V in registers): one pass holding K, V
// and both fp32 accumulators would not fit two waves per SIMD at D = 128.
template <typename T, int D, int NW, bool CAUSAL, int PASS>
__global__ __launch_bounds__(NW * 64) __attribute__((amdgpu_waves_per_eu(PASS == 0 ? 3 : 2)))
void bwd_dkdv_mfma_kernel(BwdParams p) {
  using TP = TilePair<D, NW>;
  constexpr int S = 3, BK = NW * 32;
  constexpr int ROWB = 2 * D, TILEB = TP::TILEB, STAGEB = 2 * TILEB + 256;
  constexpr int KS = D / 16, DT = D / 32, LPW = TP::LPW + 1;   // + the lse / delta load
  constexpr int LL = 64 / NW;                                   // lanes per wave loading lse / delta
  __shared__ __attribute__((aligned(1024))) char stage_lds[S * STAGEB];
  __shared__ int32_t ent_row[kMaxChunk];
  __shared__ int32_t ent_h[kMaxChunk];
  __shared__ float ent_bias[kMaxChunk];

  const int4 item = p.work[blockIdx.x];
  const int tile = item.x, chunk = item.y, part = item.z, E = item.w;
  const int zk = tile / p.ktiles, nt = tile % p.ktiles;
  const int z = zk / p.Hkv, kvh = zk % p.Hkv;
  const int n0 = nt * BK, kb = n0 / p.RB;
  const int tid = threadIdx.x;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int lane = tid & 63, li = lane & 31, kh = lane >> 5;
  const int N = p.N;
  const int key0w = n0 + wave * 32, kpos = key0w + li, kr = min(kpos, N - 1);
  const bool kok = kpos < N;

  // K^T (and V^T in pass 1) as B operands: lane (li + 32 kh) holds X[kr][16 s + 8 kh .. +8].
  u32x4_t kf[KS], vf[PASS == 1 ? KS : 1];
  {
    const char* krow = reinterpret_cast<const char*>(static_cast<const T*>(p.k) + z * p.ks[0] + kvh * p.ks[1] +
                                                     static_cast<int64_t>(kr) * p.ks[2]);
#pragma unroll
    for (int s = 0; s < KS; ++s) kf[s] = *reinterpret_cast<const u32x4_t*>(krow + 32 * s + 16 * kh);
    if constexpr (PASS == 1) {
      const char* vrow = reinterpret_cast<const char*>(static_cast<const T*>(p.v) + z * p.vs[0] + kvh * p.vs[1] +
                                                       static_cast<int64_t>(kr) * p.vs[2]);
#pragma unroll
      for (int s = 0; s < KS; ++s) vf[s] = *reinterpret_cast<const u32x4_t*>(vrow + 32 * s + 16 * kh);
    }
  }
  const int spq = p.RB >> 5, lspq = __builtin_ctz(spq);
  const int ne = max(0, min(E - chunk * p.chunk, p.chunk));
  if (tid < p.chunk) {
    // all `chunk` slots are read (those past ne are never used), so these
    // loads do not wait for the item header
    const int64_t slot = static_cast<int64_t>(blockIdx.x) * p.chunk + tid;
    const int2 rh = p.ent_rh[slot];
    ent_row[tid] = rh.x;
    ent_h[tid] = rh.y;
    ent_bias[tid] = p.ent_b[slot];
  }
  __syncthreads();
  __builtin_amdgcn_s_waitcnt(0);

  const uint32_t qsb = static_cast<uint32_t>(p.qs[2]) * 2u, dsb = static_cast<uint32_t>(p.dos[2]) * 2u;
  TP tp;
  tp.init(wave, lane, qsb, dsb);
  uint32_t rm[KS];
#pragma unroll
  for (int s = 0; s < KS; ++s) rm[s] = li * ROWB + 16 * ((2 * s + kh) ^ bsw<D>(li));
  uint32_t tr0[DT], tr1[DT];
  tr_offsets<D>(lane, tr0, tr1);
  const uint32_t lds_base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((SA_LDS char*)stage_lds));

  auto stage_row = [&](int m) { return ent_row[m >> lspq] + ((m & (spq - 1)) << 5); };
  auto issue = [&](int m, int stg) {
    const int h = __builtin_amdgcn_readfirstlane(ent_h[m >> lspq]);
    const int row0 = __builtin_amdgcn_readfirstlane(stage_row(m));
    const char* qb0 = reinterpret_cast<const char*>(static_cast<const T*>(p.q) + z * p.qs[0] + h * p.qs[1]);
    const char* db0 = reinterpret_cast<const char*>(static_cast<const T*>(p.dout) + z * p.dos[0] + h * p.dos[1]);
    const uint32_t dst = lds_base + stg * STAGEB;
    tp.issue(qb0, db0, qsb, dsb, row0, N, dst, wave, lane);
    if (lane < LL) {
      const int gl = wave * LL + lane;   // 0..31: lse rows, 32..63: delta rows
      const int r = min(max(row0 + (gl & 31), 0), N - 1);
      const float* src = (gl < 32 ? p.lse : p.delta) + (static_cast<int64_t>(z) * p.H + h) * N + r;
      dma4(src, __builtin_amdgcn_readfirstlane(dst + 2 * TILEB + wave * LL * 4));
    }
  };

  f32x16_t acc[DT];   // dV^T (pass 0) or dK^T (pass 1)
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) acc[dt] = f32x16_t{};

  auto compute = [&](int m, int stg) {
    const int q0 = stage_row(m);
    const bool skip = key0w >= N || q0 >= N || (CAUSAL && q0 + 31 < key0w);
    if (skip) return;
    const char* sbase = stage_lds + stg * STAGEB;
    f32x16_t st = f32x16_t{}, dp = f32x16_t{};
#pragma unroll
    for (int s = 0; s < KS; ++s) {
      const u32x4_t qa = *reinterpret_cast<const u32x4_t*>(sbase + rm[s]);
      st = Mma<T>::mma(qa, kf[s], st);
    }
    if constexpr (PASS == 1) {
#pragma unroll
      for (int s = 0; s < KS; ++s) {
        const u32x4_t da = *reinterpret_cast<const u32x4_t*>(sbase + TILEB + rm[s]);
        dp = Mma<T>::mma(da, vf[s], dp);
      }
    }
    const float bias = ent_bias[m >> lspq];
    const bool need_mask = !kok || q0 + 32 > N || (CAUSAL && q0 < key0w + 31);
    // Register v holds query q0 + 8 (v >> 2) + 4 kh + (v & 3); one half s2
    // (v = 8 s2 .. 8 s2 + 7) at a time feeds the B operand of step s2.
#pragma unroll
    for (int s2 = 0; s2 < 2; ++s2) {
      float x[8];
#pragma unroll
      for (int gg = 0; gg < 2; ++gg) {
        const int g4 = 2 * s2 + gg;
        const f32x4_t l4 = *reinterpret_cast<const f32x4_t*>(sbase + 2 * TILEB + 4 * (8 * g4 + 4 * kh));
        f32x4_t d4 = f32x4_t{0.f, 0.f, 0.f, 0.f};
        if constexpr (PASS == 1) d4 = *reinterpret_cast<const f32x4_t*>(sbase + 2 * TILEB + 128 + 4 * (8 * g4 + 4 * kh));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int v = 4 * g4 + i;
          const float l2 = l4[i] == -INFINITY ? 0.f : l4[i] * kLog2e;
          float e = fast_exp2(fmaf(st[v], p.qk_scale, bias - l2));
          if (need_mask) {
            const int qq = q0 + 8 * g4 + 4 * kh + i;
            if (!(kok && qq < N && (!CAUSAL || qq >= kpos))) e = 0.f;
          }
          if constexpr (PASS == 1) e *= dp[v] - d4[i];
          x[4 * gg + i] = e;
        }
      }
      const u32x4_t b = pack8<T>(x);
      // pass 0: dV^T += dO^T P (dO tile); pass 1: dK^T += Q^T dS (Q tile)
      const char* abase = PASS == 0 ? sbase + TILEB : sbase;
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) acc[dt] = Mma<T>::mma(tr_operand<T, D>(abase, tr0[dt], tr1[dt], s2), b, acc[dt]);
    }
  };

  const int total = ne << lspq;
#pragma unroll
  for (int st0 = 0; st0 < S - 1; ++st0) {
    if (st0 < total) issue(st0, st0);
  }
  int n = 0;
  auto step = [&](auto stg_c) {
    constexpr int stg = decltype(stg_c)::value;
    if (n >= total) return;
    wait_tiles<LPW, S - 2>(total - 1 - n);
    barrier_only();
    if (n + S - 1 < total) issue(n + S - 1, (stg + S - 1) % S);
    compute(n, stg);
    ++n;
  };
  while (n < total) {
    step(std::integral_constant<int, 0>{});
    step(std::integral_constant<int, 1>{});
    step(std::integral_constant<int, 2>{});
  }
  wait_vmcnt<0>();

  const float sc = PASS == 1 ? p.sm_scale : 1.f;
  if (part < 0) {
    if (kok) {
      T* o = PASS == 1
                 ? static_cast<T*>(p.dk) + z * p.dks[0] + kvh * p.dks[1] + static_cast<int64_t>(kpos) * p.dks[2]
                 : static_cast<T*>(p.dv) + z * p.dvs[0] + kvh * p.dvs[1] + static_cast<int64_t>(kpos) * p.dvs[2];
#pragma unroll
      for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int d = 32 * dt + 8 * g + 4 * kh;
          *reinterpret_cast<u32x2_t*>(o + d) = u32x2_t{Mma<T>::pack(acc[dt][4 * g] * sc, acc[dt][4 * g + 1] * sc),
                                                       Mma<T>::pack(acc[dt][4 * g + 2] * sc, acc[dt][4 * g + 3] * sc)};
        }
      }
    }
  } else {
    // Partial of a split tile: float4 j = (K|V, dt, g) of lane L of wave w at
    // ((part * NW + w) * 8 DT + j) * 64 + L (coalesced 1-KB stores).
    f32x4_t* out = reinterpret_cast<f32x4_t*>(p.partials) +
                   (static_cast<int64_t>(part) * NW + wave) * 8 * DT * 64 + (PASS == 1 ? 0 : 4 * DT * 64) + lane;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        out[(4 * dt + g) * 64] = f32x4_t{acc[dt][4 * g] * sc, acc[dt][4 * g + 1] * sc, acc[dt][4 * g + 2] * sc,
                                         acc[dt][4 * g + 3] * sc};
      }
    }
  }
}

// Sums the partials of each split tile's items and writes its dK / dV rows:
// workgroup (slot, j) handles float4 column j = (K|V, dt, g) of every lane of
// the tile's NW waves (coalesced 1-KB reads per wave and item).
template <typename T, int D, int NW>
__global__ __launch_bounds__(NW * 64) void bwd_finalize_kernel(BwdParams p) {
  constexpr int BK = NW * 32, DT = D / 32, J = 8 * DT;
  const int slot = blockIdx.x / J, j = blockIdx.x % J;
  const int4 m = p.multi[slot];
  const int tile = m.x, first = m.y, nc = m.z;
  const int zk = tile / p.ktiles, nt = tile % p.ktiles;
  const int z = zk / p.Hkv, kvh = zk % p.Hkv;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, li = lane & 31, kh = lane >> 5;
  const int kpos = nt * BK + wave * 32 + li;
  const f32x4_t* in = reinterpret_cast<const f32x4_t*>(p.partials) + (static_cast<int64_t>(wave) * J + j) * 64 + lane;
  f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int c = 0; c < nc; ++c) acc += in[static_cast<int64_t>(first + c) * NW * J * 64];
  if (kpos >= p.N) return;
  const int jj = j % (4 * DT), dt = jj >> 2, g = jj & 3;
  const int d = 32 * dt + 8 * g + 4 * kh;
  T* o = j < 4 * DT
             ? static_cast<T*>(p.dk) + z * p.dks[0] + kvh * p.dks[1] + static_cast<int64_t>(kpos) * p.dks[2]
             : static_cast<T*>(p.dv) + z * p.dvs[0] + kvh * p.dvs[1] + static_cast<int64_t>(kpos) * p.dvs[2];
  *reinterpret_cast<u32x2_t*>(o + d) = u32x2_t{Mma<T>::pack(acc[0], acc[1]), Mma<T>::pack(acc[2], acc[3])};
}

// Phase 1: dQ (with delta and the soft-bias gradient); phase 2: dK / dV.
template <typename T, int D, int NW>
int launch_dq_mfma_nw(BwdParams& p, hipStream_t s) {
  constexpr int BM = NW * 32;
  p.mtiles = (p.N + BM - 1) / BM;
  const long long g_dq = static_cast<long long>(p.Z) * p.H * p.mtiles;
  if (g_dq > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  if (p.is_causal) {
    hipLaunchKernelGGL((bwd_dq_mfma_kernel<T, D, NW, true>), dim3(static_cast<unsigned>(g_dq)), dim3(NW * 64), 0, s, p);
  } else {
    hipLaunchKernelGGL((bwd_dq_mfma_kernel<T, D, NW, false>), dim3(static_cast<unsigned>(g_dq)), dim3(NW * 64), 0, s, p);
  }
  return check_launch("block-sparse backward dQ (MFMA) kernel");
}

template <typename T, int D, int NW>
int launch_dkdv_mfma_nw(BwdParams& p, hipStream_t s) {
  if (p.n_work == 0) return SA_OK;
  if (p.is_causal) {
    hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, NW, true, 0>), dim3(p.n_work), dim3(NW * 64), 0, s, p);
    hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, NW, true, 1>), dim3(p.n_work), dim3(NW * 64), 0, s, p);
  } else {
    hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, NW, false, 0>), dim3(p.n_work), dim3(NW * 64), 0, s, p);
    hipLaunchKernelGGL((bwd_dkdv_mfma_kernel<T, D, NW, false, 1>), dim3(p.n_work), dim3(NW * 64), 0, s, p);
  }
  int rc = check_launch("block-sparse backward dK/dV (MFMA) kernels");
  if (rc != SA_OK || p.n_multi == 0) return rc;
  hipLaunchKernelGGL((bwd_finalize_kernel<T, D, NW>), dim3(p.n_multi * 8 * (D / 32)), dim3(NW * 64), 0, s, p);
  return check_launch("block-sparse backward dK/dV finalize kernel");
}

template <typename T, int D>
int launch_bwd_mfma_d(BwdParams& p, int phase, hipStream_t s) {
  if (p.RB >= 128) return phase == 1 ? launch_dq_mfma_nw<T, D, 4>(p, s) : launch_dkdv_mfma_nw<T, D, 4>(p, s);
  if (p.RB == 64) return phase == 1 ? launch_dq_mfma_nw<T, D, 2>(p, s) : launch_dkdv_mfma_nw<T, D, 2>(p, s);
  return phase == 1 ? launch_dq_mfma_nw<T, D, 1>(p, s) : launch_dkdv_mfma_nw<T, D, 1>(p, s);
}

template <typename T>
int launch_bwd_mfma(BwdParams& p, int D, int phase, hipStream_t s) {
  if (D == 32) return launch_bwd_mfma_d<T, 32>(p, phase, s);
  if (D == 64) return launch_bwd_mfma_d<T, 64>(p, phase, s);
  return launch_bwd_mfma_d<T, 128>(p, phase, s);
}

// Keys per dK/dV work item and transposed entries per item.
inline int bwd_key_tile(int route_block) { return route_block >= 128 ? 128 : route_block; }
inline int bwd_chunk(int route_block) {
  return std::min(kMaxChunk, std::max(1, kChunkStages / std::max(1, route_block / 32)));
}

// Plan buffer: work items (int4, at most one per key tile plus one per `chunk`
// transposed entries), split tiles (int4, at most one per key tile), then the
// transposed soft-bias values (float, Z * H * NB * t_max).
inline size_t bwd_plan_work_bytes(int Z, int H, int H_kv, int N, int route_block, int t_max) {
  const int BK = bwd_key_tile(route_block);
  const long long NB = (N + route_block - 1) / route_block;
  const long long T = static_cast<long long>(Z) * H_kv * ((N + BK - 1) / BK);
  const long long entries = static_cast<long long>(route_block / BK) * Z * H * NB * t_max;
  const long long C = bwd_chunk(route_block);
  return static_cast<size_t>(T + (entries + C - 1) / C) * sizeof(int4);
}
inline size_t bwd_plan_tbias_bytes(int Z, int H, int N, int route_block, int t_max) {
  const long long NB = (N + route_block - 1) / route_block;
  return (static_cast<size_t>(Z) * H * NB * t_max * sizeof(float) + 15) / 16 * 16;
}
// + the resolved entries of every work item: `chunk` {row, head} pairs and biases.
inline size_t bwd_plan_bytes(int Z, int H, int H_kv, int N, int route_block, int t_max) {
  const int BK = bwd_key_tile(route_block);
  const long long T = static_cast<long long>(Z) * H_kv * ((N + BK - 1) / BK);
  const size_t wb = bwd_plan_work_bytes(Z, H, H_kv, N, route_block, t_max);
  const size_t items = wb / sizeof(int4);
  return wb + static_cast<size_t>(T) * sizeof(int4) + bwd_plan_tbias_bytes(Z, H, N, route_block, t_max) +
         items * bwd_chunk(route_block) * (sizeof(int2) + sizeof(float));
}
// Points p's plan fields into the plan buffer (layout of bwd_plan_bytes).
inline void bwd_plan_layout(BwdParams& p, char* pl, int Z, int H, int H_kv, int N, int route_block, int t_max,
                            bool soft_bias) {
  const int BK = bwd_key_tile(route_block);
  const long long T = static_cast<long long>(Z) * H_kv * ((N + BK - 1) / BK);
  const size_t wb = bwd_plan_work_bytes(Z, H, H_kv, N, route_block, t_max);
  const size_t items = wb / sizeof(int4);
  const size_t C = bwd_chunk(route_block);
  char* tb = pl + wb + static_cast<size_t>(T) * sizeof(int4);
  char* rec = tb + bwd_plan_tbias_bytes(Z, H, N, route_block, t_max);
  p.work = reinterpret_cast<const int4*>(pl);
  p.multi = reinterpret_cast<const int4*>(pl + wb);
  p.t_bias = soft_bias ? reinterpret_cast<const float*>(tb) : nullptr;
  p.ent_rh = reinterpret_cast<int2*>(rec);
  p.ent_b = reinterpret_cast<float*>(rec + items * C * sizeof(int2));
}

template <typename T, int D>
int launch_bwd_d(BwdParams& p, int phase, hipStream_t s) {
  const long long rows = static_cast<long long>(p.Z) * p.H * p.N;
  const long long g_delta = (rows + 15) / 16;
  const long long g_dq = static_cast<long long>(p.Z) * p.H * p.tiles;
  const long long g_dkdv = static_cast<long long>(p.Z) * p.Hkv * p.tiles;
  if (g_delta > 0x7fffffffLL || g_dq > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  if (phase == 1) {
    hipLaunchKernelGGL((bwd_delta_kernel<T, D>), dim3(static_cast<unsigned>(g_delta)), dim3(256), 0, s, p);
    int rc = check_launch("block-sparse backward delta kernel");
    if (rc != SA_OK) return rc;
    hipLaunchKernelGGL((bwd_dq_kernel<T, D>), dim3(static_cast<unsigned>(g_dq)), dim3(256), 0, s, p);
    return check_launch("block-sparse backward dQ kernel");
  }
  hipLaunchKernelGGL((bwd_dkdv_kernel<T, D>), dim3(static_cast<unsigned>(g_dkdv)), dim3(256), 0, s, p);
  return check_launch("block-sparse backward dK/dV kernel");
}

template <typename T>
int launch_bwd(BwdParams& p, int D, int phase, hipStream_t s) {
  switch (D) {
    case 16: return launch_bwd_d<T, 16>(p, phase, s);
    case 32: return launch_bwd_d<T, 32>(p, phase, s);
    case 64: return launch_bwd_d<T, 64>(p, phase, s);
    case 128: return launch_bwd_d<T, 128>(p, phase, s);
    default: return launch_bwd_d<T, 256>(p, phase, s);
  }
}

}  // namespace
}  // namespace sa

extern "C" int sa_block_sparse_bwd(const void* q, const void* k, const void* v, const void* out,
                                   const void* dout, const float* lse, const int32_t* lists,
                                   const int32_t* counts, int max_count, const int32_t* t_lists,
                                   const int32_t* t_counts, int t_max_count, const void* soft_bias,
                                   int soft_bias_dtype, const int64_t* sb_strides, float* delta,
                                   void* dq, void* dk, void* dv, float* d_soft_bias,
                                   const void* plan, int n_work, int n_multi, float* dkv_partials,
                                   int phases, int Z, int H, int H_kv, int N, int D, int route_block,
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

  // MFMA kernels: unit stride along D and 16-byte aligned rows; dK / dV also
  // need a work plan.
  bool rows_ok = true;
  for (const int64_t* x : st) rows_ok = rows_ok && x[3] == 1 && x[2] % 8 == 0 && x[1] % 8 == 0 && x[0] % 8 == 0;
  const void* ptrs[8] = {q, k, v, out, dout, dq, dk, dv};
  for (const void* x : ptrs) rows_ok = rows_ok && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
  long long max_rs = 0;
  for (const int64_t* x : st) max_rs = std::max<long long>(max_rs, x[2] * 2);
  const bool offs_ok = N < (1 << 24) && max_rs < (1 << 24) && static_cast<long long>(N) * max_rs < (1LL << 32);
  const bool mfma_shapes = dtype != SA_DTYPE_F32 && (D == 32 || D == 64 || D == 128) && route_block >= 32 &&
                           rows_ok && offs_ok;
  if (phases < 1 || phases > 3) return fail(SA_EINVAL, "phases must be 1 (dQ), 2 (dK/dV) or 3 (both)");
  int rc = SA_OK;
  if (phases & 1) {
    if (mfma_shapes) {
      rc = dtype == SA_DTYPE_BF16 ? launch_bwd_mfma<bf16_t>(p, D, 1, s) : launch_bwd_mfma<f16_t>(p, D, 1, s);
    } else if (dtype == SA_DTYPE_F32) {
      rc = launch_bwd<float>(p, D, 1, s);
    } else {
      rc = dtype == SA_DTYPE_BF16 ? launch_bwd<bf16_t>(p, D, 1, s) : launch_bwd<f16_t>(p, D, 1, s);
    }
    if (rc != SA_OK) return rc;
  }
  if (!(phases & 2)) return SA_OK;
  if (mfma_shapes && plan) {
    const int BK = bwd_key_tile(route_block);
    const long long T = static_cast<long long>(Z) * H_kv * ((N + BK - 1) / BK);
    if (n_work < 0 || n_multi < 0 || n_work > T + static_cast<long long>(Z) * H * p.NB * t_max_count) {
      return fail(SA_EINVAL, "n_work / n_multi do not come from sa_block_sparse_bwd_plan");
    }
    if (n_multi > 0 && !dkv_partials) return fail(SA_EINVAL, "dkv_partials is NULL but the plan has split tiles");
    bwd_plan_layout(p, const_cast<char*>(static_cast<const char*>(plan)), Z, H, H_kv, N, route_block, t_max_count,
                    soft_bias != nullptr);
    p.key_tile = BK;
    p.partials = dkv_partials;
    p.n_work = n_work;
    p.n_multi = n_multi;
    p.ktiles = static_cast<int>((N + BK - 1) / BK);
    p.chunk = bwd_chunk(route_block);
    return dtype == SA_DTYPE_BF16 ? launch_bwd_mfma<bf16_t>(p, D, 2, s) : launch_bwd_mfma<f16_t>(p, D, 2, s);
  }
  if (dtype == SA_DTYPE_F32) return launch_bwd<float>(p, D, 2, s);
  if (dtype == SA_DTYPE_BF16) return launch_bwd<bf16_t>(p, D, 2, s);
  return launch_bwd<f16_t>(p, D, 2, s);
}

extern "C" size_t sa_block_sparse_bwd_plan_bytes(int Z, int H, int H_kv, int N, int route_block, int t_max_count) {
  if (Z <= 0 || H <= 0 || H_kv <= 0 || N <= 0 || route_block < 32 || t_max_count < 0) return 0;
  return sa::bwd_plan_bytes(Z, H, H_kv, N, route_block, t_max_count);
}

extern "C" int sa_block_sparse_bwd_plan(const int32_t* lists, const int32_t* counts, int max_count,
                                        const int32_t* t_lists, const int32_t* t_counts, int t_max_count,
                                        const void* soft_bias, int soft_bias_dtype, const int64_t* sb_strides,
                                        int Z, int H, int H_kv, int N, int route_block, void* plan,
                                        size_t plan_bytes, int32_t* plan_info, void* stream) {
  using namespace sa;
  if (Z < 0 || H < 0 || N < 0 || H_kv <= 0 || (H > 0 && H % H_kv != 0)) return fail(SA_EINVAL, "bad Z/H/H_kv/N");
  if (!is_pow2(route_block) || route_block < 32) return fail(SA_EINVAL, "route_block must be a power of two >= 32");
  if (max_count < 0 || t_max_count < 0) return fail(SA_EINVAL, "negative list widths");
  if (!plan_info) return fail(SA_EINVAL, "NULL plan_info");
  if (static_cast<long long>(Z) * H * N == 0) {
    hipLaunchKernelGGL(fill_i32_kernel, dim3(1), dim3(64), 0, as_stream(stream), plan_info, 3, 0);
    return check_launch("plan info fill");
  }
  if (!counts || !t_counts || (!lists && max_count > 0) || (!t_lists && t_max_count > 0) || !plan) {
    return fail(SA_EINVAL, "NULL tensor argument");
  }
  if (soft_bias && (!sb_strides || (soft_bias_dtype != SA_DTYPE_F32 && soft_bias_dtype != SA_DTYPE_BF16 &&
                                    soft_bias_dtype != SA_DTYPE_F16))) {
    return fail(SA_EINVAL, "soft_bias needs strides and an f32/bf16/f16 dtype");
  }
  const size_t need = bwd_plan_bytes(Z, H, H_kv, N, route_block, t_max_count);
  if (plan_bytes < need) return fail(SA_EINVAL, "plan buffer too small: need " + std::to_string(need) + " bytes");
  BwdParams p{};
  p.lists = lists; p.counts = counts; p.tlists = t_lists; p.tcounts = t_counts;
  p.sb = soft_bias; p.sb_dtype = soft_bias_dtype;
  for (int i = 0; i < 4; ++i) p.sbs[i] = soft_bias ? sb_strides[i] : 0;
  p.Z = Z; p.H = H; p.Hkv = H_kv; p.N = N; p.RB = route_block;
  p.NB = (N + route_block - 1) / route_block;
  p.max_count = max_count; p.t_max = t_max_count; p.group = H / H_kv;
  const int BK = bwd_key_tile(route_block);
  p.ktiles = (N + BK - 1) / BK;
  p.chunk = bwd_chunk(route_block);
  hipStream_t s = as_stream(stream);
  char* pl = static_cast<char*>(plan);
  const size_t wb = bwd_plan_work_bytes(Z, H, H_kv, N, route_block, t_max_count);
  const long long T = static_cast<long long>(Z) * H_kv * p.ktiles;
  if (T > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large");
  bwd_plan_layout(p, pl, Z, H, H_kv, N, route_block, t_max_count, soft_bias != nullptr);
  p.key_tile = BK;
  hipLaunchKernelGGL(bwd_plan_kernel, dim3(1), dim3(1024), 0, s, p, BK, reinterpret_cast<int4*>(pl),
                     reinterpret_cast<int4*>(pl + wb), plan_info);
  int rc = check_launch("block-sparse backward plan kernel");
  if (rc != SA_OK) return rc;
  if (soft_bias && max_count > 0 && t_max_count > 0) {
    const long long pairs = static_cast<long long>(Z) * H * p.NB * max_count;
    const long long g = (pairs + 255) / 256;
    if (g > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
    hipLaunchKernelGGL(bwd_tbias_kernel, dim3(static_cast<unsigned>(g)), dim3(256), 0, s, p,
                       const_cast<float*>(p.t_bias));
    rc = check_launch("block-sparse backward soft-bias transpose kernel");
    if (rc != SA_OK) return rc;
  }
  // entries of each work item, up to the item count the plan kernel wrote
  const long long items = static_cast<long long>(wb / sizeof(int4));
  const unsigned g_items = static_cast<unsigned>(std::min<long long>((items + 3) / 4, 2048));
  hipLaunchKernelGGL(bwd_items_kernel, dim3(g_items), dim3(256), 0, s, p, plan_info,
                     static_cast<int>(std::min<long long>(items, 0x7fffffffLL)));
  return check_launch("block-sparse backward work-item kernel");
}
