// Route-block majority vote of the surgery caller (gfx950).
//
// Semantics follow SurgicalLlamaAttention._block_list_prefill
// (src/llama_surgery/surgery.py:543-547): for every (b, h, route block i,
// level l < r), each token t of the block votes for argmax_j assign[b,h,t,l,j]
// (first maximum on ties, as torch.argmax), and the block's routing id for
// level l is the branch with the most votes (lowest id on ties). Tokens past
// S do not vote (the reference pads its one-hot votes with zeros). With
// route_block = 1 this is the direct block routing of surgery.py:536-541
// (one row of assignments per block).
//
// route_vote_kernel: one 256-thread workgroup per (b, h, block). Each thread
// takes (token, level) pairs of the block, reads the p branch scores of the
// pair, and adds its vote to a per-(level, branch) LDS counter; the first r
// threads then pick each level's winner. The scores are read once, so the
// kernel is HBM-bound: B H S L p element reads for the whole batch.
#include "sa_internal.h"

#include <type_traits>

namespace sa {
namespace {

constexpr int kVoteThreads = 256;
constexpr int kMaxP = 64;
constexpr int kMaxR = 32;

struct VoteParams {
  const void* a;
  int64_t s0, s1, s2, s3, s4;
  int B, H, S, L, P, R, RB, NB;
  int32_t* out;
};

// Four consecutive scores, 4 * sizeof(T)-aligned, as floats.
template <typename T>
__device__ __forceinline__ void load4(const T* src, float (&x)[4]) {
  if constexpr (sizeof(T) == 4) {
    const float4 v = *reinterpret_cast<const float4*>(src);
    x[0] = v.x; x[1] = v.y; x[2] = v.z; x[3] = v.w;
  } else {
    const uint2 u = *reinterpret_cast<const uint2*>(src);
    const uint32_t h[4] = {u.x & 0xffffu, u.x >> 16, u.y & 0xffffu, u.y >> 16};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      if constexpr (std::is_same<T, bf16_t>::value) x[c] = bf16_bits_to_float(h[c]);
      else x[c] = f16_bits_to_float(h[c]);
    }
  }
}

// Argmax order of torch.argmax: the first maximum wins ties, and a NaN counts
// as the maximum (the first NaN wins).
__device__ __forceinline__ bool beats(float y, float best) {
  return y > best || (y != y && best == best);
}

template <typename T>
__global__ __launch_bounds__(kVoteThreads) void route_vote_kernel(VoteParams p) {
  __shared__ int votes[kMaxR][kMaxP];
  const int blk = blockIdx.x;
  const int i = blk % p.NB;
  const int bh = blk / p.NB;
  const int h = bh % p.H, b = bh / p.H;
  for (int j = threadIdx.x; j < p.R * p.P; j += kVoteThreads) votes[j / p.P][j % p.P] = 0;
  __syncthreads();
  const int t0 = i * p.RB;
  const int len = min(p.RB, p.S - t0);
  const T* base = static_cast<const T*>(p.a) + b * p.s0 + h * p.s1;
  // Four contiguous, aligned branch scores: one vector read per (token, level).
  constexpr int kVec4 = 4 * static_cast<int>(sizeof(T));
  const bool vec4 = p.P == 4 && p.s4 == 1 && (p.s0 * sizeof(T)) % kVec4 == 0 && (p.s1 * sizeof(T)) % kVec4 == 0 &&
                    (p.s2 * sizeof(T)) % kVec4 == 0 && (p.s3 * sizeof(T)) % kVec4 == 0 &&
                    (reinterpret_cast<uintptr_t>(p.a) % kVec4) == 0;
  for (int j = threadIdx.x; j < len * p.R; j += kVoteThreads) {
    const int t = t0 + j / p.R, l = j % p.R;
    const T* row = base + t * p.s2 + l * p.s3;
    float x[4];
    int arg = 0;
    if (vec4) {
      load4<T>(row, x);
#pragma unroll
      for (int c = 1; c < 4; ++c) {
        if (beats(x[c], x[arg])) arg = c;
      }
    } else {
      float best = Elem<T>::load(row);
      for (int c = 1; c < p.P; ++c) {
        const float y = Elem<T>::load(row + c * p.s4);
        if (beats(y, best)) {
          best = y;
          arg = c;
        }
      }
    }
    atomicAdd(&votes[l][arg], 1);
  }
  __syncthreads();
  if (threadIdx.x < p.R) {
    const int l = threadIdx.x;
    int best = votes[l][0], arg = 0;
    for (int c = 1; c < p.P; ++c) {
      if (votes[l][c] > best) {   // lowest id wins ties
        best = votes[l][c];
        arg = c;
      }
    }
    p.out[(static_cast<int64_t>(bh) * p.NB + i) * p.R + l] = arg;
  }
}

}  // namespace
}  // namespace sa

extern "C" int sa_route_block_vote(const void* assign, int dtype, const int64_t* strides, int B, int H,
                                   int S, int L, int P, int r, int route_block, int32_t* out,
                                   void* stream) {
  using namespace sa;
  if (B < 0 || H < 0 || S < 0 || L < 1 || P < 1) return fail(SA_EINVAL, "bad B/H/S/L/p");
  if (r < 0 || r > L) return fail(SA_EINVAL, "r must lie in [0, levels]");
  if (route_block < 1) return fail(SA_EINVAL, "route_block must be >= 1");
  if (P > kMaxP) return fail(SA_EUNSUPPORTED, "more than 64 branches per level is not supported");
  if (r > kMaxR) return fail(SA_EUNSUPPORTED, "more than 32 voted levels is not supported");
  if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16) {
    return fail(SA_EINVAL, "dtype must be f32, bf16 or f16");
  }
  const long long NB = (static_cast<long long>(S) + route_block - 1) / route_block;
  const long long wg = static_cast<long long>(B) * H * NB;
  if (wg == 0 || r == 0) return SA_OK;
  if (!assign || !strides || !out) return fail(SA_EINVAL, "NULL argument");
  if (wg > 0x7fffffffLL) return fail(SA_EINVAL, "problem too large for one launch");
  VoteParams p{};
  p.a = assign;
  p.s0 = strides[0]; p.s1 = strides[1]; p.s2 = strides[2]; p.s3 = strides[3]; p.s4 = strides[4];
  p.B = B; p.H = H; p.S = S; p.L = L; p.P = P; p.R = r; p.RB = route_block; p.NB = static_cast<int>(NB);
  p.out = out;
  const dim3 g(static_cast<unsigned>(wg)), blk(kVoteThreads);
  hipStream_t s = as_stream(stream);
  if (dtype == SA_DTYPE_F32) hipLaunchKernelGGL((route_vote_kernel<float>), g, blk, 0, s, p);
  else if (dtype == SA_DTYPE_BF16) hipLaunchKernelGGL((route_vote_kernel<bf16_t>), g, blk, 0, s, p);
  else hipLaunchKernelGGL((route_vote_kernel<f16_t>), g, blk, 0, s, p);
  return check_launch("route-block vote kernel");
}
