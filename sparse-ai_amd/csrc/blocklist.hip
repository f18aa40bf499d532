// Block-list compaction: routing vectors (or an explicit block mask) -> per
// (z, h, query block) ascending list of active key blocks + count.
//
// Semantics follow build_block_lists / _build_block_lists_kernel in the
// reference (src/ultrametric/block_list.py:127-278):
//   * match(i, j): mixed-radix codes equal (block_list.py:224-229), or the
//     first depth[h] levels equal element-wise (block_list.py:256-258);
//   * then local band OR, sink column OR, causal AND (block_list.py:107-118);
//   * the k-th active key block of a row goes to slot k, slots >= count are 0
//     (block_list.py:263-278).
//
// Design: one workgroup = 4 waves handles 4*R consecutive query-block rows of
// one (z, h), R = rows per wave (1..16, as few as keeps ~4096 waves busy).
// The NB key codes of that head are computed into LDS; each wave then walks
// its rows 64 key blocks at a time: one predicate per lane,
// a wave ballot, and mbcnt (popcount of the ballot below the lane) gives
// every active lane its output slot. Padding zeros are written by the same
// kernel, so the output needs no memset.
#include "sa_internal.h"

#include <algorithm>

namespace sa {
namespace {

constexpr int kWaves = 4;
constexpr int kMaxRowsPerWave = 16;
constexpr long long kTargetWaves = 4096;  // enough waves to fill 256 CUs
constexpr int kMaxNB = 8192;  // codes of one head live in LDS: 8192 * 8 B = 64 KB

enum MatchMode { kCodes = 0, kElementwise = 1, kMask = 2 };

struct BLParams {
  const void* router;
  int64_t rs0, rs1, rs2, rs3;
  const uint8_t* mask;
  int64_t ms0, ms1, ms2, ms3;
  const int64_t* depth_dev;
  int depth_uniform;
  uint64_t base;
  int Z, H, NB, TD;
  int is_causal, sink_block, local_blocks;
  int32_t* lists;
  int cols;
  int32_t* counts;
  int groups_per_head;
  int rows_per_wave;
};

template <typename IdT>
__device__ __forceinline__ int64_t load_id(const BLParams& p, int z, int h, int b, int l) {
  const IdT* r = static_cast<const IdT*>(p.router);
  return static_cast<int64_t>(r[z * p.rs0 + h * p.rs1 + b * p.rs2 + l * p.rs3]);
}

__device__ __forceinline__ uint32_t lanes_below(uint64_t ballot) {
  return __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(ballot >> 32),
                                   __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(ballot), 0u));
}

template <typename IdT, int MODE>
__global__ __launch_bounds__(kWaves * 64) void blocklist_kernel(BLParams p) {
  extern __shared__ uint64_t codes[];  // NB entries (kCodes mode only)

  const int group = blockIdx.x % p.groups_per_head;
  const int zh = blockIdx.x / p.groups_per_head;
  const int z = zh / p.H;
  const int h = zh % p.H;
  const int NB = p.NB;
  const int depth = p.depth_dev ? static_cast<int>(p.depth_dev[h]) : p.depth_uniform;

  if (MODE == kCodes) {
    // code = sum_l id_l * [l < depth] * base^l, in wrapping 64-bit arithmetic
    // like the reference's int64 torch ops.
    for (int kb = threadIdx.x; kb < NB; kb += blockDim.x) {
      uint64_t code = 0, pw = 1;
      for (int l = 0; l < p.TD; ++l) {
        if (l < depth) code += static_cast<uint64_t>(load_id<IdT>(p, z, h, kb, l)) * pw;
        pw *= p.base;
      }
      codes[kb] = code;
    }
    __syncthreads();
  }

  const int wave = threadIdx.x / 64;
  const int lane = threadIdx.x % 64;
  const int row0 = (group * kWaves + wave) * p.rows_per_wave;
  for (int r = 0; r < p.rows_per_wave; ++r) {
    const int qb = row0 + r;
    if (qb >= NB) break;
    const int64_t row = static_cast<int64_t>(zh) * NB + qb;
    int32_t* out_row = p.lists ? p.lists + row * p.cols : nullptr;
    uint64_t qcode = 0;
    if (MODE == kCodes) qcode = codes[qb];
    // Under causal masking no key block past qb can survive.
    const int kb_end = p.is_causal ? qb + 1 : NB;
    int written = 0;
    for (int c0 = 0; c0 < kb_end; c0 += 64) {
      const int kb = c0 + lane;
      bool m = false;
      if (kb < NB) {
        if (MODE == kCodes) {
          m = codes[kb] == qcode;
        } else if (MODE == kElementwise) {
          m = true;
          for (int l = 0; l < depth && l < p.TD; ++l) {
            if (load_id<IdT>(p, z, h, qb, l) != load_id<IdT>(p, z, h, kb, l)) {
              m = false;
              break;
            }
          }
        } else {
          m = p.mask[z * p.ms0 + h * p.ms1 + qb * p.ms2 + kb * p.ms3] != 0;
        }
        const int diff = qb > kb ? qb - kb : kb - qb;
        if (p.local_blocks > 0 && diff <= p.local_blocks) m = true;
        if (p.sink_block && kb == 0) m = true;
        if (p.is_causal && kb > qb) m = false;
      }
      const uint64_t bal = __ballot(m);
      if (m && out_row) {
        const int pos = written + static_cast<int>(lanes_below(bal));
        if (pos < p.cols) out_row[pos] = kb;
      }
      written += __popcll(bal);
    }
    if (lane == 0) p.counts[row] = written;
    if (out_row) {
      for (int t = written + lane; t < p.cols; t += 64) out_row[t] = 0;
    }
  }
}

int launch(BLParams& p, int mode, int id_dtype, hipStream_t stream) {
  if (p.Z < 0 || p.H < 0 || p.NB < 0) return fail(SA_EINVAL, "negative dimension");
  if (p.NB > kMaxNB) {
    return fail(SA_EUNSUPPORTED, "block-list builder supports NB <= 8192, got " + std::to_string(p.NB));
  }
  if (p.lists && p.cols < 0) return fail(SA_EINVAL, "lists_cols must be >= 0");
  const long long rows_total = static_cast<long long>(p.Z) * p.H * p.NB;
  if (rows_total == 0) return SA_OK;                     // empty tensors may carry NULL
  if (!p.counts) return fail(SA_EINVAL, "counts must not be NULL");
  // Rows per wave: as few as keeps ~kTargetWaves waves busy (each workgroup
  // recomputes its head's NB codes, a cached read of NB * TD ids).
  long long rpw = (rows_total + kTargetWaves - 1) / kTargetWaves;
  p.rows_per_wave = static_cast<int>(rpw < 1 ? 1 : (rpw > kMaxRowsPerWave ? kMaxRowsPerWave : rpw));
  const int rows_per_group = kWaves * p.rows_per_wave;
  p.groups_per_head = (p.NB + rows_per_group - 1) / rows_per_group;
  const long long grid = static_cast<long long>(p.Z) * p.H * p.groups_per_head;
  if (grid > 0x7fffffffLL) return fail(SA_EINVAL, "too many rows");
  const size_t lds = mode == kCodes ? static_cast<size_t>(p.NB) * sizeof(uint64_t) : 0;
  dim3 g(static_cast<unsigned>(grid)), b(kWaves * 64);
  if (mode == kMask) {
    hipLaunchKernelGGL((blocklist_kernel<int32_t, kMask>), g, b, lds, stream, p);
  } else if (id_dtype == SA_DTYPE_I32) {
    if (mode == kCodes)
      hipLaunchKernelGGL((blocklist_kernel<int32_t, kCodes>), g, b, lds, stream, p);
    else
      hipLaunchKernelGGL((blocklist_kernel<int32_t, kElementwise>), g, b, lds, stream, p);
  } else {
    if (mode == kCodes)
      hipLaunchKernelGGL((blocklist_kernel<int64_t, kCodes>), g, b, lds, stream, p);
    else
      hipLaunchKernelGGL((blocklist_kernel<int64_t, kElementwise>), g, b, lds, stream, p);
  }
  return check_launch("block-list compaction kernel");
}

}  // namespace
}  // namespace sa

extern "C" int sa_build_block_lists(const void* router, int router_dtype,
                                    const int64_t* router_strides, int Z, int H, int NB, int TD,
                                    const int64_t* depth_dev, int depth_uniform, int64_t base,
                                    int use_codes, int is_causal, int sink_block,
                                    int local_blocks, int32_t* lists, int lists_cols,
                                    int32_t* counts, void* stream) {
  using namespace sa;
  if (router_dtype != SA_DTYPE_I32 && router_dtype != SA_DTYPE_I64) {
    return fail(SA_EINVAL, "router ids must be int32 or int64");
  }
  if (TD < 1) return fail(SA_EINVAL, "tree depth must be >= 1");
  if (!depth_dev && (depth_uniform < 0 || depth_uniform > TD)) {
    return fail(SA_EINVAL, "req_depth out of range [0, TD]");
  }
  if (use_codes && base < 2) return fail(SA_EINVAL, "code base must be >= 2");
  if (!router_strides || (!router && static_cast<long long>(Z) * H * NB > 0)) {
    return fail(SA_EINVAL, "router must not be NULL");
  }
  BLParams p{};
  p.router = router;
  p.rs0 = router_strides[0];
  p.rs1 = router_strides[1];
  p.rs2 = router_strides[2];
  p.rs3 = router_strides[3];
  p.depth_dev = depth_dev;
  p.depth_uniform = depth_uniform;
  p.base = static_cast<uint64_t>(base);
  p.Z = Z;
  p.H = H;
  p.NB = NB;
  p.TD = TD;
  p.is_causal = is_causal != 0;
  p.sink_block = sink_block != 0;
  p.local_blocks = local_blocks;
  p.lists = lists;
  p.cols = lists_cols;
  p.counts = counts;
  return launch(p, use_codes ? kCodes : kElementwise, router_dtype, as_stream(stream));
}

extern "C" int sa_build_block_lists_mask(const uint8_t* mask, const int64_t* mask_strides, int Z,
                                         int H, int NB, int is_causal, int sink_block,
                                         int local_blocks, int32_t* lists, int lists_cols,
                                         int32_t* counts, void* stream) {
  using namespace sa;
  if (!mask_strides || (!mask && static_cast<long long>(Z) * H * NB > 0)) {
    return fail(SA_EINVAL, "mask must not be NULL");
  }
  BLParams p{};
  p.mask = mask;
  p.ms0 = mask_strides[0];
  p.ms1 = mask_strides[1];
  p.ms2 = mask_strides[2];
  p.ms3 = mask_strides[3];
  p.Z = Z;
  p.H = H;
  p.NB = NB;
  p.TD = 1;
  p.is_causal = is_causal != 0;
  p.sink_block = sink_block != 0;
  p.local_blocks = local_blocks;
  p.lists = lists;
  p.cols = lists_cols;
  p.counts = counts;
  return launch(p, kMask, SA_DTYPE_I32, as_stream(stream));
}

namespace sa {
namespace {

// Bit matrix of the transpose: CK key-block rows of NB query-block bits (odd
// row stride in words, so that the row scans below do not share banks), at
// most 64 KB of dynamic LDS; NB up to kMaxNB.
constexpr int kTransLdsWords = 16384;

// One workgroup per (z, h, chunk of CK key blocks): every listed pair
// (qb, kb) with kb in the chunk sets bit qb of row kb - k0; thread j then
// writes row k0 + j's query blocks in ascending order, zero-padded to t_cols,
// and its count. Every chunk scans all of the head's list entries, so a grid
// of NB <= 512 is one chunk per head.
__global__ __launch_bounds__(1024) void transpose_lists_kernel(const int32_t* lists, const int32_t* counts,
                                                               int max_count, int NB, int CK, int chunks,
                                                               int32_t* t_lists, int t_cols, int32_t* t_counts) {
  extern __shared__ uint32_t bits[];
  const int zh = blockIdx.x / chunks, k0 = (blockIdx.x % chunks) * CK, tid = threadIdx.x;
  const int nk = min(CK, NB - k0);
  const int W = (NB + 31) / 32, WS = W | 1;
  for (int i = tid; i < nk * WS; i += 1024) bits[i] = 0u;
  __syncthreads();
  const int32_t* L = lists + static_cast<int64_t>(zh) * NB * max_count;
  const int32_t* C = counts + static_cast<int64_t>(zh) * NB;
  for (int64_t i = tid; i < static_cast<int64_t>(NB) * max_count; i += 1024) {
    const int qb = static_cast<int>(i / max_count), t = static_cast<int>(i % max_count);
    if (t < min(max(C[qb], 0), max_count)) {
      const int kb = L[i] - k0;
      if (kb >= 0 && kb < nk) atomicOr(&bits[kb * WS + (qb >> 5)], 1u << (qb & 31));
    }
  }
  __syncthreads();
  for (int j = tid; j < nk; j += 1024) {
    const int kb = k0 + j;
    int n = 0;
    int32_t* out = t_lists ? t_lists + (static_cast<int64_t>(zh) * NB + kb) * t_cols : nullptr;
    for (int w = 0; w < W; ++w) {
      uint32_t x = bits[j * WS + w];
      while (x) {
        const int b = __builtin_ctz(x);
        x &= x - 1u;
        if (out && n < t_cols) out[n] = w * 32 + b;
        ++n;
      }
    }
    if (out) {
      for (int c = n; c < t_cols; ++c) out[c] = 0;
    }
    t_counts[static_cast<int64_t>(zh) * NB + kb] = n;
  }
}

}  // namespace
}  // namespace sa

extern "C" int sa_transpose_block_lists(const int32_t* lists, const int32_t* counts, int max_count, int Z, int H,
                                        int NB, int32_t* t_lists, int t_cols, int32_t* t_counts, void* stream) {
  using namespace sa;
  if (Z < 0 || H < 0 || NB < 0 || max_count < 0 || t_cols < 0) return fail(SA_EINVAL, "negative size");
  if (NB > kMaxNB) return fail(SA_EUNSUPPORTED, "transposed lists need NB <= " + std::to_string(kMaxNB));
  const long long zh = static_cast<long long>(Z) * H;
  if (zh == 0 || NB == 0) return SA_OK;
  if (!counts || !t_counts || (max_count > 0 && !lists)) return fail(SA_EINVAL, "NULL tensor argument");
  if (t_lists && t_cols < 1) return fail(SA_EINVAL, "t_cols must be >= 1 when t_lists is given");
  const int WS = ((NB + 31) / 32) | 1;
  const int CK = std::min(NB, kTransLdsWords / WS);
  const int chunks = (NB + CK - 1) / CK;
  if (zh * chunks > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  hipLaunchKernelGGL(transpose_lists_kernel, dim3(static_cast<unsigned>(zh * chunks)), dim3(1024),
                     static_cast<size_t>(CK) * WS * sizeof(uint32_t), as_stream(stream), lists, counts, max_count,
                     NB, CK, chunks, t_lists, t_cols, t_counts);
  return check_launch("block-list transpose kernel");
}
