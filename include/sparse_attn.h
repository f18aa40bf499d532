/*
 * sparse_attn.h — C ABI of libsparseattn.so, the MI355X (gfx950) block-sparse
 * attention hot path: block-list compaction, block-sparse prefill forward and
 * sparse paged decode.
 *
 * The reference (sparse-ai, src/ultrametric) has no C ABI: its boundary is a
 * Python function API backed by Triton kernels. Each entry point below names
 * the Python function / Triton kernel it replaces; the Python package
 * `ultrametric` in this repository keeps those Python names and calls these
 * functions through ctypes.
 *
 * Conventions shared by every entry point:
 *   - All tensor arguments are DEVICE pointers (HIP, gfx950). Strides are in
 *     elements, not bytes. Nothing here allocates device memory; callers pass
 *     outputs and any workspace.
 *   - Every call is asynchronous on `stream` (a hipStream_t passed as void*;
 *     NULL = the legacy default stream) and performs no host<->device sync.
 *   - Return value: SA_OK (0) on success, a negative SA_E* code otherwise;
 *     sa_last_error() then returns a thread-local message. Argument errors are
 *     detected on the host before any launch.
 *   - Calls are reentrant; the library keeps no global mutable state apart
 *     from the thread-local error string and, for
 *     sa_sparse_paged_decode_seq_codes_noalloc only, one 8 MiB device array
 *     per GPU (the split-KV partials of that entry point) with its per-device
 *     address.
 */
#ifndef SPARSE_ATTN_H
#define SPARSE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define SA_ABI_VERSION 1

/* Status codes. */
#define SA_OK 0
#define SA_EINVAL (-1)        /* bad shape / stride / parameter (Python: ValueError) */
#define SA_EUNSUPPORTED (-2)  /* valid but not implemented here (Python: RuntimeError) */
#define SA_ELAUNCH (-3)       /* HIP launch or runtime error (Python: RuntimeError) */

/* Element types. */
#define SA_DTYPE_F32 0
#define SA_DTYPE_BF16 1
#define SA_DTYPE_F16 2
#define SA_DTYPE_I32 3
#define SA_DTYPE_I64 4
#define SA_DTYPE_U8 5  /* bool masks */

/* ABI version of the loaded library (SA_ABI_VERSION it was built with). */
int sa_abi_version(void);

/* Thread-local message describing the last failed call on this thread. */
const char* sa_last_error(void);

/*
 * Block-list compaction from per-block routing vectors.
 * Replaces: build_block_lists() and _build_block_lists_kernel
 *   (src/ultrametric/block_list.py:170-278 and :127-167).
 *
 * router      (Z, H, NB, TD) integer branch ids, element type router_dtype
 *             (SA_DTYPE_I32 or SA_DTYPE_I64), strides router_strides[4].
 * depth_dev   optional (H,) int64 device array of per-head required depths;
 *             when NULL every head uses depth_uniform. Depths must already be
 *             validated to lie in [0, TD] (block_list.py:93-104).
 * base        mixed-radix base (block_list.py:211-215): max(2, arity) in the
 *             sync-free mode, max(2, max(id)+1) otherwise.
 * use_codes   1: blocks match iff their mixed-radix codes
 *             sum_l id_l * [l < depth] * base^l (int64, wrapping) are equal
 *             (block_list.py:224-229); 0: element-wise equality on the first
 *             depth levels (block_list.py:256-258). The reference picks 1 iff
 *             TD * log2(base) < 62.
 * is_causal / sink_block / local_blocks: structural masks applied in the
 *             reference order: local band OR, sink column OR, causal AND
 *             (block_list.py:107-118).
 * lists       (Z, H, NB, lists_cols) int32 contiguous output, or NULL to
 *             compute counts only. Row (z,h,i) receives its active key blocks
 *             in ascending order, then zeros up to lists_cols. lists_cols must
 *             be >= the largest count (NB in the sync-free mode).
 * counts      (Z, H, NB) int32 contiguous output.
 * Limits: NB <= 8192.
 */
int sa_build_block_lists(const void* router, int router_dtype, const int64_t* router_strides,
                         int Z, int H, int NB, int TD, const int64_t* depth_dev, int depth_uniform,
                         int64_t base, int use_codes, int is_causal, int sink_block,
                         int local_blocks, int32_t* lists, int lists_cols, int32_t* counts,
                         void* stream);

/*
 * Block-list compaction from an explicit per-head block mask.
 * Replaces: the compaction step of build_block_lists applied to a given
 *   `match` (src/ultrametric/block_list.py:263-278); extension named by the
 *   hot-path scope (block mask -> block list).
 *
 * mask        (Z, H, NB, NB) uint8 (non-zero = active), strides mask_strides[4].
 * The structural masks are applied on top, in the same order as above.
 * lists / lists_cols / counts as for sa_build_block_lists.
 */
int sa_build_block_lists_mask(const uint8_t* mask, const int64_t* mask_strides, int Z, int H,
                              int NB, int is_causal, int sink_block, int local_blocks,
                              int32_t* lists, int lists_cols, int32_t* counts, void* stream);

/*
 * Block-sparse attention forward over block lists.
 * Replaces: _block_list_attention_fwd / _block_list_fwd_kernel
 *   (src/ultrametric/block_list.py:688-757 and :387-470).
 *
 * q, out      (Z, H, N, D); k, v (Z, H_kv, N, D) with H % H_kv == 0 (GQA:
 *             query head h reads kv head h / (H / H_kv)). Element type dtype
 *             (SA_DTYPE_F32 / SA_DTYPE_BF16 / SA_DTYPE_F16) for all four.
 *             Strides q_strides[4], k_strides[4], v_strides[4], o_strides[4].
 * lse         optional (Z, H, N) fp32 contiguous output: natural-log
 *             log-sum-exp of the scaled scores, -inf for rows with no key.
 * lists       (Z, H, NB, max_count) int32 contiguous, NB = ceil(N/route_block);
 * counts      (Z, H, NB) int32 contiguous. Only the first counts[row] entries
 *             of a row are read; each must lie in [0, NB).
 * soft_bias   optional (Z, H, NB, max_count) additive logit bias per listed
 *             block, element type soft_bias_dtype (F32/BF16/F16), strides
 *             sb_strides[4].
 * route_block power of two >= 16; D power of two in [16, 256].
 * Rows of out with index >= N are never written; out = 0 for rows with no
 * visible key.
 */
int sa_block_sparse_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                        const int32_t* lists, const int32_t* counts, const void* soft_bias,
                        int soft_bias_dtype, int Z, int H, int H_kv, int N, int D,
                        int route_block, int max_count, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides,
                        const int64_t* o_strides, const int64_t* sb_strides, float sm_scale,
                        int dtype, int is_causal, void* stream);

/*
 * Routed block-sparse prefill with the list build fused into the forward.
 * Replaces: routed_block_attention (src/ultrametric/block_list.py:1064-1083)
 * when the caller knows the branch arity, i.e. build_block_lists(...,
 * arity=base) (block_list.py:170-278, sync-free) followed by
 * block_list_attention (block_list.py:968-1061), in one launch.
 * Each workgroup builds its row's list from the routing ids (code matching,
 * then local band, sink column and causal mask, as sa_build_block_lists) and
 * writes it to lists (Z, H, NB, NB) int32 contiguous, zero padded, and
 * counts (Z, H, NB): the sync-free BlockLists, usable by the backward.
 * router, router_dtype, router_strides, TD, depth_dev, depth_uniform, base:
 * as sa_build_block_lists with use_codes = 1 (TD * log2(base) < 62 is the
 * caller's condition for that, as in the reference).
 * Supported: bf16 / f16, D in {32, 64, 128}, route block >= 32, no soft
 * bias, NB <= 256 (route block >= 128), 128 (64) or 64 (32). Otherwise
 * SA_EUNSUPPORTED: build the lists and call sa_block_sparse_fwd instead.
 */
int sa_routed_block_sparse_fwd(const void* q, const void* k, const void* v, void* out, float* lse,
                               const void* router, int router_dtype, const int64_t* router_strides, int TD,
                               const int64_t* depth_dev, int depth_uniform, int64_t base, int sink_block,
                               int local_blocks, int32_t* lists, int32_t* counts, int Z, int H, int H_kv,
                               int N, int D, int route_block, const int64_t* q_strides,
                               const int64_t* k_strides, const int64_t* v_strides,
                               const int64_t* o_strides, float sm_scale, int dtype, int is_causal,
                               void* stream);

/*
 * Transposed block lists: per (z, h, key block), the ascending query blocks
 * whose lists hold it.
 * Replaces: build_transposed_block_lists (src/ultrametric/block_list.py:281-327),
 *   whose scatter / transpose / cumsum steps become one kernel.
 *
 * lists / counts / max_count: forward lists (Z, H, NB, max_count) and counts
 *             (Z, H, NB), int32 contiguous; entries outside [0, NB) are ignored.
 * t_lists     (Z, H, NB, t_cols) int32 contiguous output, zero-padded; or NULL
 *             to compute t_counts only (then read max(t_counts) and call again,
 *             as the reference's max_q_count). Rows longer than t_cols are cut.
 * t_counts    (Z, H, NB) int32 contiguous output.
 * Limits: NB <= 512.
 */
int sa_transpose_block_lists(const int32_t* lists, const int32_t* counts, int max_count, int Z, int H, int NB,
                             int32_t* t_lists, int t_cols, int32_t* t_counts, void* stream);

/*
 * Block-sparse attention backward over block lists.
 * Replaces: _block_list_attention_bwd with _block_list_bwd_dq_kernel and
 *   _block_list_bwd_dkdv_kernel (src/ultrametric/block_list.py:758-880,
 *   :494-681), GQA added (dk / dv sum over the H / H_kv query heads of a kv
 *   head).
 *
 * q, out, dout, dq  (Z, H, N, D); k, v, dk, dv (Z, H_kv, N, D); element type
 *             dtype for all; strides *_strides[4].
 * lse         (Z, H, N) fp32 contiguous: the forward's natural-log LSE.
 * lists / counts / max_count: the forward's block lists.
 * t_lists / t_counts / t_max_count: the transposed lists
 *             (build_transposed_block_lists, block_list.py:281-327): per
 *             (z, h, key block), the ascending query blocks that list it;
 *             (Z, H, NB, t_max_count) / (Z, H, NB) int32 contiguous.
 * soft_bias   optional (Z, H, NB, max_count) per-listed-block logit bias, as in
 *             the forward; d_soft_bias (Z, H, NB, max_count) fp32 contiguous
 *             receives its gradient (sum of dL/dlogit over the block pair) and
 *             must be zero-filled by the caller (the kernel accumulates with
 *             float atomics, so its low bits depend on the order of the adds).
 * delta       (Z, H, N) fp32 contiguous workspace (rowsum(dout * out)).
 * plan / n_work / n_multi: the work plan of sa_block_sparse_bwd_plan (same
 *             lists, shapes and soft bias) and the first two values of its
 *             plan_info. With a plan, bf16/fp16 inputs with D in {32, 64, 128},
 *             route_block >= 32, unit stride along D and 16-byte aligned rows
 *             run on MFMA kernels; otherwise (plan NULL, fp32, other shapes)
 *             on fp32 FMA kernels.
 * dkv_partials fp32 workspace of plan_info[2] * 2 * BK * D floats (BK = 128
 *             when route_block >= 128, else route_block), no initialisation
 *             needed; NULL when plan_info[1] == 0.
 * phases      1: delta, dQ and d_soft_bias (the reference's
 *             _block_list_bwd_dq_kernel); 2: dK and dV (its
 *             _block_list_bwd_dkdv_kernel), which reads the delta of phase 1;
 *             3: both. Phase 1 needs no plan, so a caller can queue it before
 *             reading plan_info back.
 * dq, dk, dv are fully written (zeros where no pair is visible).
 */
int sa_block_sparse_bwd(const void* q, const void* k, const void* v, const void* out, const void* dout,
                        const float* lse, const int32_t* lists, const int32_t* counts, int max_count,
                        const int32_t* t_lists, const int32_t* t_counts, int t_max_count,
                        const void* soft_bias, int soft_bias_dtype, const int64_t* sb_strides,
                        float* delta, void* dq, void* dk, void* dv, float* d_soft_bias,
                        const void* plan, int n_work, int n_multi, float* dkv_partials, int phases,
                        int Z, int H, int H_kv, int N, int D, int route_block, const int64_t* q_strides,
                        const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides,
                        const int64_t* do_strides, const int64_t* dq_strides, const int64_t* dk_strides,
                        const int64_t* dv_strides, float sm_scale, int dtype, int is_causal,
                        void* stream);

/*
 * Work plan of the MFMA dK/dV kernel.
 * Replaces: the grid of _block_list_bwd_dkdv_kernel (one program per key
 *   block, block_list.py:834-866) and the host read of max(q_counts) in
 *   build_transposed_block_lists (block_list.py:320): key tiles whose
 *   transposed lists are long (the sink column is listed by every query
 *   block) are split into items of a bounded number of entries, placed
 *   first; the other tiles follow by decreasing entry count.
 *
 * Inputs as for sa_block_sparse_bwd. plan: device buffer of at least
 * sa_block_sparse_bwd_plan_bytes(...) bytes. plan_info: device int32[3]
 * receiving {work items, split tiles, work items of split tiles}; the caller
 * reads it back (one device-to-host copy, at the point where the reference
 * reads max(q_counts)) to size the launch and dkv_partials.
 * With soft_bias the plan also holds each transposed entry's bias. The plan
 * also resolves every work item's entries (first query row, head, bias), so
 * the work that follows the read-back is the dK / dV kernels alone.
 */
size_t sa_block_sparse_bwd_plan_bytes(int Z, int H, int H_kv, int N, int route_block, int t_max_count);
int sa_block_sparse_bwd_plan(const int32_t* lists, const int32_t* counts, int max_count,
                             const int32_t* t_lists, const int32_t* t_counts, int t_max_count,
                             const void* soft_bias, int soft_bias_dtype, const int64_t* sb_strides,
                             int Z, int H, int H_kv, int N, int route_block, void* plan,
                             size_t plan_bytes, int32_t* plan_info, void* stream);

/*
 * Workspace bytes needed by sa_sparse_paged_decode for B sequences of H query
 * heads (H_kv kv heads) of dimension D with at most max_pages logical pages
 * each. 0 when the work items already fill the GPU, so that each is handled
 * by one workgroup and no split-KV partials are kept; otherwise room for the
 * per-split (max, sum, acc[D]) partials. A work item is a (sequence, kv head)
 * when the group size H / H_kv is 1, 2, 4 or 8, else a (sequence, query head).
 * No reference counterpart (the reference decode keeps no split-KV partials).
 */
size_t sa_decode_workspace_bytes(int B, int H, int H_kv, int D, int max_pages);

/*
 * Sparse paged decode with tree-routed page selection.
 * Replaces: ultrametric_decode / _ultrametric_decode_kernel
 *   (src/ultrametric/kernel_decode.py:188-247 and :22-124), with the CPU
 *   reference semantics for ctx_len <= 0 (zeros, kernel_decode.py:145-152)
 *   and GQA added (k/v caches carry H_kv heads, H % H_kv == 0; query head h
 *   reads kv head h / (H / H_kv); with a group of 1, 2, 4 or 8 heads a K/V page
 *   is loaded once per group, other group sizes load it per query head).
 *
 * q           (B, H, D); out (B, H, D) — dtype, strides q_strides[3] / o_strides[3].
 * k_cache, v_cache (P, H_kv, page, D) — dtype, strides k_strides[4] / v_strides[4].
 * block_tables (B, max_pages) int32, strides bt_strides[2]: logical -> physical page.
 * context_lens (B,) int32 contiguous.
 * router      (P, H, TD) int32, strides r_strides[3]: routing vector per
 *             (physical page, query head).
 * q_router    (B, H, TD) int32, strides qr_strides[3].
 * req_depth   levels that must agree (clamped to [0, TD]).
 * A logical page l of sequence b is attended by head h iff its routing
 * vector matches on the first req_depth levels, or (sink_block and l == 0),
 * or (local_blocks > 0 and l >= n_pages - local_blocks). Tokens >= ctx_len
 * are masked; scale = 1/sqrt(D); heads with no selected page get zeros.
 * workspace   device buffer of at least sa_decode_workspace_bytes(...) bytes.
 */
int sa_sparse_paged_decode(const void* q, const void* k_cache, const void* v_cache,
                           const int32_t* block_tables, const int32_t* context_lens,
                           const int32_t* router, const int32_t* q_router, void* out, int B,
                           int H, int H_kv, int D, int page_size, int TD, int max_pages,
                           int num_phys_pages, int req_depth, int local_blocks, int sink_block,
                           const int64_t* q_strides, const int64_t* k_strides,
                           const int64_t* v_strides, const int64_t* bt_strides,
                           const int64_t* r_strides, const int64_t* qr_strides,
                           const int64_t* o_strides, void* workspace, size_t workspace_bytes,
                           int dtype, void* stream);

/*
 * Sparse paged decode selecting pages by packed routing codes stored per
 * sequence in logical page order.
 * Extension of ultrametric_decode (kernel_decode.py:22-124, :188-247): the
 *   serving-side page-routing format. seq_codes (B, H, max_pages) of
 *   code_bytes-byte unsigned codes (1, 2 or 4; TD * bits_per_level must fit),
 *   strides sc_strides[3] in codes: seq_codes[b, h, l] = the packed code
 *   (sa_pack_page_codes) of the physical page block_tables[b, l] for head h,
 *   written once when the page is appended. A workgroup then reads its heads'
 *   codes as contiguous rows, in the same round trip as the block table,
 *   instead of one scattered row per physical page. Entries past a
 *   sequence's pages are not read for selection.
 *   q_codes (B, H) uint32, strides qc_strides[2]. Other arguments as
 *   sa_sparse_paged_decode_codes; same results.
 */
int sa_sparse_paged_decode_seq_codes(const void* q, const void* k_cache, const void* v_cache,
                                     const int32_t* block_tables, const int32_t* context_lens,
                                     const void* seq_codes, int code_bytes, const uint32_t* q_codes,
                                     void* out, int B, int H, int H_kv, int D, int page_size, int TD,
                                     int bits_per_level, int max_pages, int num_phys_pages,
                                     int req_depth, int local_blocks, int sink_block,
                                     const int64_t* q_strides, const int64_t* k_strides,
                                     const int64_t* v_strides, const int64_t* bt_strides,
                                     const int64_t* sc_strides, const int64_t* qc_strides,
                                     const int64_t* o_strides, void* workspace, size_t workspace_bytes,
                                     int dtype, void* stream);

/*
 * Packs routing levels into one 32-bit code per (row, head).
 * Extension of ultrametric_decode (src/ultrametric/kernel_decode.py:22-124,
 *   whose kernel re-reads TD int32 levels per (page, head), :76-81): the
 *   packed per-page routing code that the hot-path scope lists as the next
 *   step for decode. No reference counterpart.
 *
 * router      (rows, H, TD) int32, strides[3]; every level must lie in
 *             [0, 2^bits_per_level).
 * codes       (rows, H) uint32 contiguous output: level l is stored in bits
 *             [bits_per_level (TD-1-l), bits_per_level (TD-l)), so level 0 is
 *             the most significant field and the first r levels of two rows
 *             agree iff their codes agree on the top bits_per_level * r bits.
 * Limits: 1 <= bits_per_level <= 16, TD * bits_per_level <= 32.
 */
int sa_pack_page_codes(const int32_t* router, const int64_t* strides, int rows, int H, int TD,
                       int bits_per_level, uint32_t* codes, void* stream);

/*
 * Sparse paged decode selecting pages by packed routing codes.
 * Same computation as sa_sparse_paged_decode (kernel_decode.py:22-124 and
 *   :188-247) with router / q_router replaced by their packed codes
 *   (sa_pack_page_codes of the same levels): page_codes (P, H) uint32,
 *   strides pc_strides[2]; q_codes (B, H) uint32, strides qc_strides[2].
 *   Reads 4 bytes per (page, head) instead of 4 * TD. Results equal
 *   sa_sparse_paged_decode's for levels that fit bits_per_level bits.
 * Limits: as sa_pack_page_codes for TD and bits_per_level.
 */
int sa_sparse_paged_decode_codes(const void* q, const void* k_cache, const void* v_cache,
                                 const int32_t* block_tables, const int32_t* context_lens,
                                 const uint32_t* page_codes, const uint32_t* q_codes, void* out,
                                 int B, int H, int H_kv, int D, int page_size, int TD,
                                 int bits_per_level, int max_pages, int num_phys_pages,
                                 int req_depth, int local_blocks, int sink_block,
                                 const int64_t* q_strides, const int64_t* k_strides,
                                 const int64_t* v_strides, const int64_t* bt_strides,
                                 const int64_t* pc_strides, const int64_t* qc_strides,
                                 const int64_t* o_strides, void* workspace, size_t workspace_bytes,
                                 int dtype, void* stream);

/*
 * Ternary (2-bit) quantize + pack of rows.
 * Replaces: TernaryQuantize + pack_ternary (src/llama_surgery/surgery.py:15-55).
 *
 * x           (rows, D) of dtype (F32/BF16/F16), strides[2] (row, element).
 * mode        0: gamma = mean |x| of the row; x > gamma/2 -> +1,
 *             x < -gamma/2 -> -1, else 0 (TernaryQuantize); scale = gamma.
 *             1: x already in {-1, 0, 1} (pack_ternary); scale = 1.
 * packed      (rows, D / 16) int32 contiguous: value i of word w in bits
 *             [2i, 2i + 2) of word w, code 0 -> 0, 1 -> +1, 2 -> -1.
 * scale       optional (rows,) fp32 contiguous.
 * Limits: D % 16 == 0.
 */
int sa_ternary_pack(const void* x, int dtype, const int64_t* strides, int rows, int D, int mode,
                    int32_t* packed, float* scale, void* stream);

/*
 * Causal block-sparse prefill over ternary packed K / V.
 * Replaces: _ternary_ultrametric_fwd_kernel and ternary_ultrametric_attention_triton
 *   (src/llama_surgery/kernel.py:147-249, :348-420), run over block lists
 *   (route block 128) that carry its block choice (routing match on the first
 *   req_depth levels, sink, local window, causal); GQA added.
 *
 * q, out      (Z, H, N, D) fp16, strides[4] (unit along D, 16-byte aligned rows).
 * k_packed, v_packed (Z, H_kv, N, D / 16) int32 (unit stride along the last dim),
 *             strides[4]; k_scale, v_scale (Z, H_kv, N) of scale_dtype, strides[3].
 *             Key j's vectors are unpack(k_packed[j]) * k_scale[j], and so for v.
 * lists / counts / max_count: block lists for route block 128 (is_causal,
 *             sink and local band applied).
 * shift_size  keys and queries interact only on the same side of
 *             N - shift_size (the reference's region mask).
 * Scale 1/sqrt(D); rows with no visible key get 0 (the reference yields NaN
 * for a row whose first visited block has no visible key).
 * Limits: D in {32, 64, 128}.
 */
int sa_ternary_prefill_fwd(const void* q, const int32_t* k_packed, const int32_t* v_packed,
                           const void* k_scale, const void* v_scale, int scale_dtype,
                           const int32_t* lists, const int32_t* counts, int max_count, void* out,
                           int Z, int H, int H_kv, int N, int D, int shift_size,
                           const int64_t* q_strides, const int64_t* kp_strides, const int64_t* vp_strides,
                           const int64_t* ks_strides, const int64_t* vs_strides, const int64_t* o_strides,
                           void* stream);

/*
 * Route-block majority vote of the surgery caller.
 * Replaces: the per-level majority vote of token argmax branches in
 *   SurgicalLlamaAttention._block_list_prefill
 *   (src/llama_surgery/surgery.py:543-547; with route_block = 1, the direct
 *   block routing of :536-541).
 *
 * assign      (B, H, S, L, p) branch scores, element type dtype (F32/BF16/F16),
 *             strides[5].
 * out         (B, H, ceil(S / route_block), r) int32 contiguous: for block i
 *             and level l < r, the branch chosen by the most tokens of the
 *             block (token vote = argmax over p, first maximum on ties; block
 *             winner = lowest branch id on ties). Tokens >= S do not vote.
 * Limits: p <= 64, r <= 32 (r <= L).
 */
int sa_route_block_vote(const void* assign, int dtype, const int64_t* strides, int B, int H, int S,
                        int L, int p, int r, int route_block, int32_t* out, void* stream);

/*
 * Writes new tokens into a paged KV cache and their pages' routing codes into
 * the per-sequence code array of sa_sparse_paged_decode_seq_codes.
 * Replaces the reference's decode-time cache update (the transformers cache
 * concatenating each layer's new K / V, which the eager decode masks of
 * src/llama_surgery/surgery.py:880-955 then scan token by token); the paged
 * layout is that of ultrametric_decode (src/ultrametric/kernel_decode.py:
 * 188-247), which has no writer in the reference.
 *
 * k_new, v_new (B, H_kv, T, D), dtype, strides kn_strides[4] / vn_strides[4]
 *             (the head dimension contiguous).
 * n_new       (B,) int32 tokens of each sequence (<= T), or NULL: T each.
 * context_lens (B,) int32: lengths that ALREADY include the new tokens
 *             (sa_paged_advance first): token t of sequence b lands at
 *             position context_lens[b] - n_new[b] + t, i.e. page slot
 *             pos / page_size (physical page block_tables[b, slot]), row
 *             pos % page_size.
 * k_cache, v_cache (P = num_pages, H_kv, page_size, D), strides kc / vc[4].
 * block_tables (B, max_pages) int32, strides bt_strides[2]; the pages must be
 *             allocated by the caller beforehand.
 * token_codes (B, H, T) uint32 packed routing codes of the new tokens
 *             (sa_pack_page_codes layout), strides tc_strides[3], and
 *             seq_codes (B, H, max_pages) of code_bytes (1, 2, 4) bytes,
 *             strides sc_strides[3]: a page's code is the code of its first
 *             token (position % page_size == 0), the first-token rule of
 *             routing_to_block_indices (src/ultrametric/kernel.py:152-191).
 *             Either NULL: no codes are written.
 * status      NULL or one int32: bit 0 is set (atomic OR) for a token whose
 *             page slot is >= max_pages or whose physical page is outside
 *             [0, num_pages); such tokens are not written.
 */
int sa_paged_kv_write(const void* k_new, const void* v_new, const int64_t* kn_strides,
                      const int64_t* vn_strides, const uint32_t* token_codes, const int64_t* tc_strides,
                      const int32_t* n_new, int B, int H_kv, int T, int D, int H, void* k_cache,
                      void* v_cache, const int64_t* kc_strides, const int64_t* vc_strides,
                      const int32_t* block_tables, const int64_t* bt_strides, const int32_t* context_lens,
                      int max_pages, int num_pages, int page_size, void* seq_codes, int code_bytes,
                      const int64_t* sc_strides, int dtype, int32_t* status, void* stream);

/*
 * context_lens[b] += n_new[b] (n_new NULL: += T) for b < B, on the device.
 * Companion of sa_paged_kv_write (same reference counterpart): one launch per
 * model step, before the layers write their K / V.
 */
int sa_paged_advance(int32_t* context_lens, const int32_t* n_new, int B, int T, void* stream);

/*
 * sa_sparse_paged_decode_seq_codes without the workspace argument: the
 * split-KV partials live in a file-scope device array of the library
 * (sa_noalloc_scratch_bytes() bytes = 8 MiB per GPU, held until the process
 * ends), so the call allocates nothing. 8 MiB holds the partials of every
 * head_dim <= 128 problem (at most (512 + B H_kv) x G x (D + 2) floats).
 * No counterpart in the reference. It is for callers that cannot allocate:
 * code under HIP graph capture, tight serving loops, harnesses that forbid
 * hipMalloc.
 * Same arguments (minus workspace / workspace_bytes) and same results as
 * sa_sparse_paged_decode_seq_codes. The current HIP device must be the one
 * the tensors and stream belong to; its array's address is looked up on the
 * first call there. Returns SA_EINVAL when the partials need more than
 * sa_noalloc_scratch_bytes() (sa_decode_workspace_bytes > 8 MiB). Every
 * call on one GPU shares that GPU's array: calls that overlap on one GPU
 * (concurrent streams) race; calls in one stream order are safe. Every
 * partial the merge reads is written by the same call, so nothing needs
 * clearing between calls.
 */
int sa_sparse_paged_decode_seq_codes_noalloc(const void* q, const void* k_cache, const void* v_cache,
                                             const int32_t* block_tables, const int32_t* context_lens,
                                             const void* seq_codes, int code_bytes, const uint32_t* q_codes,
                                             void* out, int B, int H, int H_kv, int D, int page_size, int TD,
                                             int bits_per_level, int max_pages, int num_phys_pages,
                                             int req_depth, int local_blocks, int sink_block,
                                             const int64_t* q_strides, const int64_t* k_strides,
                                             const int64_t* v_strides, const int64_t* bt_strides,
                                             const int64_t* sc_strides, const int64_t* qc_strides,
                                             const int64_t* o_strides, int dtype, void* stream);

/* Bytes of the no-allocation entry point's per-GPU scratch array. */
size_t sa_noalloc_scratch_bytes(void);

#ifdef __cplusplus
}
#endif

#endif /* SPARSE_ATTN_H */
