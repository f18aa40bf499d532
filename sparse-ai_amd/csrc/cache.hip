// Paged KV cache writes for serving: new tokens' K / V rows into their pages,
// and each new page's routing code into the per-sequence code array that
// sa_sparse_paged_decode_seq_codes reads.
//
// Layout (the sparse paged decode's): k_cache / v_cache (P, H_kv, PS, D),
// block_tables (B, max_pages) int32 physical page per logical page,
// context_lens (B,) int32, seq_codes (B, H, max_pages) codes of 1, 2 or 4
// bytes. A sequence's step first advances its length (sa_paged_advance), then
// every layer writes the new tokens at the last n positions of that length
// (sa_paged_kv_write) and decodes over it: the two launches keep the length
// read-only while the writes run, so no workgroup reads a length another one
// is updating.
//
// One workgroup writes TOK_PER_WG tokens of one sequence; each thread moves
// 16-byte vectors (8 bf16 / fp16 or 4 fp32 elements) when every row is
// 16-byte aligned and contiguous, element by element otherwise. HBM-bound
// byte copy: 2 * H_kv * D * elem bytes read and written per token.
#include "sa_internal.h"

namespace sa {
namespace {

constexpr int kWriteThreads = 256;
constexpr int kTokPerWg = 4;

struct WriteParams {
  const char* k_new;
  const char* v_new;
  int64_t kn_s[4], vn_s[4];       // (B, H_kv, T, D) strides, elements
  const uint32_t* token_codes;     // (B, H, T) or null
  int64_t tc_s[3];
  const int32_t* n_new;            // (B,) or null (T each)
  char* k_cache;
  char* v_cache;
  int64_t kc_s[4], vc_s[4];        // (P, H_kv, PS, D)
  const int32_t* block_tables;
  int64_t bt_s[2];
  const int32_t* context_lens;
  char* seq_codes;                 // (B, H, max_pages) or null
  int64_t sc_s[3];
  int code_bytes;
  int B, H_kv, T, D, H, max_pages, num_pages, page_size, elem_bytes;
  int vec;                         // 16-byte vector path
  int32_t* status;                 // or null: bit 0 set on a token whose page slot is invalid
};

__device__ __forceinline__ void copy_row(const char* src, char* dst, int D, int eb, int vec, int lane,
                                         int lanes) {
  if (vec) {
    const int nv = D * eb / 16;
    for (int i = lane; i < nv; i += lanes) {
      reinterpret_cast<uint4*>(dst)[i] = reinterpret_cast<const uint4*>(src)[i];
    }
  } else if (eb == 4) {
    for (int i = lane; i < D; i += lanes) {
      reinterpret_cast<uint32_t*>(dst)[i] = reinterpret_cast<const uint32_t*>(src)[i];
    }
  } else {
    for (int i = lane; i < D; i += lanes) {
      reinterpret_cast<uint16_t*>(dst)[i] = reinterpret_cast<const uint16_t*>(src)[i];
    }
  }
}

__global__ void __launch_bounds__(kWriteThreads) paged_kv_write_kernel(WriteParams p) {
  const int b = blockIdx.y;
  const int n = p.n_new ? p.n_new[b] : p.T;
  const int t0 = blockIdx.x * kTokPerWg;
  if (n <= 0 || t0 >= n || t0 >= p.T) return;
  const int ctx = p.context_lens[b];
  // threads split over (token of the workgroup, K or V, kv head)
  const int rows = kTokPerWg * 2 * p.H_kv;
  const int lanes = rows >= kWriteThreads ? 1 : kWriteThreads / rows;
  const int eb = p.elem_bytes;
  for (int r = threadIdx.x / lanes; r < rows; r += kWriteThreads / lanes) {
    const int tt = r / (2 * p.H_kv);
    const int t = t0 + tt;
    if (t >= n || t >= p.T) continue;
    const int which = (r / p.H_kv) & 1;
    const int kh = r % p.H_kv;
    const long long pos = static_cast<long long>(ctx) - n + t;
    const long long slot = pos / p.page_size;
    int page = -1;
    if (pos >= 0 && slot < p.max_pages) page = p.block_tables[b * p.bt_s[0] + slot * p.bt_s[1]];
    if (page < 0 || page >= p.num_pages) {
      if (p.status && threadIdx.x % lanes == 0) atomicOr(p.status, 1);
      continue;
    }
    const int row = static_cast<int>(pos - slot * p.page_size);
    const int64_t* ss = which ? p.vn_s : p.kn_s;
    const int64_t* ds = which ? p.vc_s : p.kc_s;
    const char* src = (which ? p.v_new : p.k_new) +
                      (b * ss[0] + kh * ss[1] + static_cast<int64_t>(t) * ss[2]) * eb;
    char* dst = (which ? p.v_cache : p.k_cache) +
                (static_cast<int64_t>(page) * ds[0] + kh * ds[1] + static_cast<int64_t>(row) * ds[2]) * eb;
    copy_row(src, dst, p.D, eb, p.vec, threadIdx.x % lanes, lanes);
  }
  if (!p.seq_codes || !p.token_codes) return;
  // a page's routing code is the code of its first token
  for (int i = threadIdx.x; i < kTokPerWg * p.H; i += kWriteThreads) {
    const int t = t0 + i / p.H;
    const int h = i % p.H;
    if (t >= n || t >= p.T) continue;
    const long long pos = static_cast<long long>(ctx) - n + t;
    if (pos < 0 || pos % p.page_size != 0) continue;
    const long long slot = pos / p.page_size;
    if (slot >= p.max_pages) continue;
    const uint32_t c = p.token_codes[b * p.tc_s[0] + h * p.tc_s[1] + t * p.tc_s[2]];
    char* dst = p.seq_codes + (b * p.sc_s[0] + h * p.sc_s[1] + slot * p.sc_s[2]) * p.code_bytes;
    if (p.code_bytes == 1) {
      *reinterpret_cast<uint8_t*>(dst) = static_cast<uint8_t>(c);
    } else if (p.code_bytes == 2) {
      *reinterpret_cast<uint16_t*>(dst) = static_cast<uint16_t>(c);
    } else {
      *reinterpret_cast<uint32_t*>(dst) = c;
    }
  }
}

__global__ void paged_advance_kernel(int32_t* context_lens, const int32_t* n_new, int B, int T) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b < B) context_lens[b] += n_new ? n_new[b] : T;
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace sa

using namespace sa;

extern "C" int sa_paged_kv_write(const void* k_new, const void* v_new, const int64_t* kn_strides,
                                 const int64_t* vn_strides, const uint32_t* token_codes,
                                 const int64_t* tc_strides, const int32_t* n_new, int B, int H_kv, int T, int D,
                                 int H, void* k_cache, void* v_cache, const int64_t* kc_strides,
                                 const int64_t* vc_strides, const int32_t* block_tables,
                                 const int64_t* bt_strides, const int32_t* context_lens, int max_pages,
                                 int num_pages, int page_size, void* seq_codes, int code_bytes,
                                 const int64_t* sc_strides, int dtype, int32_t* status, void* stream) {
  if (B < 0 || H_kv < 1 || T < 0 || D < 1 || page_size < 1 || max_pages < 0 || num_pages < 0) {
    return fail(SA_EINVAL, "sa_paged_kv_write: bad sizes");
  }
  if (dtype != SA_DTYPE_F32 && dtype != SA_DTYPE_BF16 && dtype != SA_DTYPE_F16) {
    return fail(SA_EINVAL, "sa_paged_kv_write: dtype must be f32, bf16 or f16");
  }
  if (!kn_strides || !vn_strides || !kc_strides || !vc_strides || !bt_strides) {
    return fail(SA_EINVAL, "sa_paged_kv_write: strides missing");
  }
  if (seq_codes && token_codes) {
    if (H < 1 || !tc_strides || !sc_strides) return fail(SA_EINVAL, "sa_paged_kv_write: code arguments");
    if (code_bytes != 1 && code_bytes != 2 && code_bytes != 4) {
      return fail(SA_EINVAL, "sa_paged_kv_write: code_bytes must be 1, 2 or 4");
    }
  }
  if (B == 0 || T == 0) return SA_OK;
  if (!k_new || !v_new || !k_cache || !v_cache || !block_tables || !context_lens) {
    return fail(SA_EINVAL, "sa_paged_kv_write: null tensor");
  }
  WriteParams p{};
  p.k_new = static_cast<const char*>(k_new);
  p.v_new = static_cast<const char*>(v_new);
  for (int i = 0; i < 4; ++i) {
    p.kn_s[i] = kn_strides[i];
    p.vn_s[i] = vn_strides[i];
    p.kc_s[i] = kc_strides[i];
    p.vc_s[i] = vc_strides[i];
  }
  p.token_codes = (seq_codes && token_codes) ? token_codes : nullptr;
  if (p.token_codes) {
    for (int i = 0; i < 3; ++i) {
      p.tc_s[i] = tc_strides[i];
      p.sc_s[i] = sc_strides[i];
    }
  }
  p.n_new = n_new;
  p.k_cache = static_cast<char*>(k_cache);
  p.v_cache = static_cast<char*>(v_cache);
  p.block_tables = block_tables;
  p.bt_s[0] = bt_strides[0];
  p.bt_s[1] = bt_strides[1];
  p.context_lens = context_lens;
  p.seq_codes = p.token_codes ? static_cast<char*>(seq_codes) : nullptr;
  p.code_bytes = code_bytes;
  p.B = B;
  p.H_kv = H_kv;
  p.T = T;
  p.D = D;
  p.H = H;
  p.max_pages = max_pages;
  p.num_pages = num_pages;
  p.page_size = page_size;
  p.elem_bytes = dtype == SA_DTYPE_F32 ? 4 : 2;
  p.status = status;
  const int eb = p.elem_bytes;
  bool vec = (static_cast<long long>(D) * eb) % 16 == 0 && p.kn_s[3] == 1 && p.vn_s[3] == 1 &&
             p.kc_s[3] == 1 && p.vc_s[3] == 1 && aligned16(k_new) && aligned16(v_new) && aligned16(k_cache) &&
             aligned16(v_cache);
  for (int i = 0; i < 3 && vec; ++i) {
    vec = (p.kn_s[i] * eb) % 16 == 0 && (p.vn_s[i] * eb) % 16 == 0 && (p.kc_s[i] * eb) % 16 == 0 &&
          (p.vc_s[i] * eb) % 16 == 0;
  }
  if (!vec && (p.kn_s[3] != 1 || p.vn_s[3] != 1 || p.kc_s[3] != 1 || p.vc_s[3] != 1)) {
    return fail(SA_EINVAL, "sa_paged_kv_write: the head dimension must be contiguous");
  }
  p.vec = vec ? 1 : 0;
  dim3 grid((T + kTokPerWg - 1) / kTokPerWg, B);
  if (grid.y > 65535) return fail(SA_EINVAL, "sa_paged_kv_write: too many sequences");
  hipLaunchKernelGGL(paged_kv_write_kernel, grid, dim3(kWriteThreads), 0, as_stream(stream), p);
  return check_launch("paged_kv_write_kernel");
}

extern "C" int sa_paged_advance(int32_t* context_lens, const int32_t* n_new, int B, int T, void* stream) {
  if (B < 0 || T < 0) return fail(SA_EINVAL, "sa_paged_advance: bad sizes");
  if (B == 0) return SA_OK;
  if (!context_lens) return fail(SA_EINVAL, "sa_paged_advance: null context_lens");
  hipLaunchKernelGGL(paged_advance_kernel, dim3((B + 255) / 256), dim3(256), 0, as_stream(stream), context_lens,
                     n_new, B, T);
  return check_launch("paged_advance_kernel");
}
