/*
 * fta.h -- C ABI of libfta_gfx950.so, the MI355X (gfx950) implementation of the
 * flash-topk-attention V2 hot path:
 *     block score -> top-k select -> q-block merge -> sparse attention fwd/bwd.
 *
 * Conventions
 *  - Every function returns an int status: FTA_OK (0), FTA_ERR_ARG (1, bad
 *    argument), FTA_ERR_UNSUPPORTED (2, outside the supported envelope) or
 *    FTA_ERR_HIP (3, launch error).  fta_last_error() returns the message of
 *    the last failure on the calling thread.  No C++ exception crosses the ABI.
 *  - All pointers are device pointers owned by the caller.  Functions that need
 *    scratch take (workspace, workspace_bytes); the matching *_workspace_size()
 *    returns the required size (0 for invalid geometry).
 *  - Work is enqueued on `stream` (a hipStream_t) and is asynchronous.
 *  - dtype: FTA_DTYPE_BF16 (0) or FTA_DTYPE_F16 (1); 16-bit tensors are passed
 *    as raw pointers.  Token tensors are addressed as [B][N][H][D] with element
 *    strides {stride_b, stride_h, stride_n} and unit stride along D; D-rows must
 *    be 16-byte aligned (strides and base pointer multiples of 8 elements).
 *    This covers both the reference's [B, N, H*D] and [B, H, N, D] layouts.
 *  - Index conventions follow the reference: -1 marks an empty slot; merged
 *    lists are [B][H][QM][W]; per-row outputs are [B][H][N].
 *
 * Reference interfaces replaced (paths relative to the reference repository):
 *  each entry point below names the pybind launcher (flash_topk_attn_v2/csrc/
 *  *.cpp) and Python wrapper it stands in for.
 */
#ifndef FTA_H_
#define FTA_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define FTA_OK 0
#define FTA_ERR_ARG 1
#define FTA_ERR_UNSUPPORTED 2
#define FTA_ERR_HIP 3

#define FTA_DTYPE_BF16 0
#define FTA_DTYPE_F16 1

/* Message of the last failing call on this thread ("" if none). */
const char* fta_last_error(void);
/* ABI version (1). */
int fta_version(void);

/* ---------------------------------------------------------------- scoring */

/*
 * Scoring stage 1 alone: blk_lse[b*H+h][m][n] = log2 sum_{keys of block m}
 * 2^(scale*log2(e) * q.k) and row_lse[b*H+h][n] = log2 of the row total (fp32).
 * score[n][m] = 2^(blk_lse - row_lse).  This is the MFMA-bound half of
 * block_score_launch (flash_topk_attn_v2/csrc/block_score_kernel.cu:19-227,
 * m_locals / l_locals) with the per-block state folded into one log value.
 */
int fta_block_score_lse(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                        const int64_t* q_strides, const int64_t* k_strides, int score_block_size,
                        int pad_head, int pad_tail, float scale, float* blk_lse, float* row_lse,
                        void* stream);

/* Workspace for fta_block_score: per-block log2-sum-exp [B*H][M][N] f32 plus
 * row totals [B*H][N] f32. */
size_t fta_block_score_workspace_size(int B, int H, int N, int M);

/*
 * Dense per-query block mass: scores[b][h][n][m] = sum over keys of block m of
 * softmax(q k^T * scale) (fp32, rows sum to 1), M = (pad_head+N+pad_tail)/b.
 * Replaces block_score_launch (flash_topk_attn_v2/csrc/block_score.cpp:3-15,
 * csrc/block_score_kernel.cu:414-438) behind flash_block_score_cuda
 * (flash_topk_attn_v2/block_score_cuda.py:45-161) and the Triton path of
 * flash_block_score (flash_topk_attn_v2/block_score.py:417-451).
 * q_strides/k_strides: {stride_b, stride_h, stride_n} in elements.
 */
int fta_block_score(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                    const int64_t* q_strides, const int64_t* k_strides, int score_block_size,
                    int pad_head, int pad_tail, float scale, float* scores, void* workspace,
                    size_t workspace_bytes, void* stream);

/*
 * Top-k block selection with threshold truncation over `rows` rows of M fp32
 * scores (element (r, m) at block_scores[r*stride_row + m*stride_m]).
 * Outputs [rows][M_OUT], M_OUT = min(max_topk, M) (M if max_topk == 0):
 * indices (-1 past the cut), raw = avg*valid_count (0 past the cut), avg.
 * Ties go to the lower block index; the cumulative sum is sequential fp32.
 * Replaces topk_select_launch (flash_topk_attn_v2/csrc/topk_select.cpp:3-15,
 * csrc/topk_select_kernel.cu:142-177) behind flash_topk_select
 * (flash_topk_attn_v2/topk_select.py:185-311, topk_select_cuda.py:27-114).
 */
int fta_topk_select(const float* block_scores, int64_t rows, int M, int64_t stride_row,
                    int64_t stride_m, int max_topk, int score_block_size, int pad_head, int pad_tail,
                    float threshold, int32_t* topk_indices, float* topk_raw, float* topk_avg,
                    void* stream);

/*
 * Workspace of fta_topk_score.  fta_topk_score_workspace_size covers every
 * path (any head dim, block size and max_topk); fta_topk_score_workspace_size_ex
 * returns the recommended size for one call's geometry (0 for an invalid one),
 * assuming a K token stride of at most 2^24 elements.
 *
 * b = 64 or 128, D <= 128 and at most 32 blocks per query run
 * on candidate streams: chunks of 1024 entries taken from a pool in the
 * workspace, one chunk per 64 queries plus a shared remainder, sized for the
 * expected number of entries (m_out (1 + 2 ln(M / m_out)) per query; 1.17e9
 * bytes at B1 H32 N32768 b64 top-16, against 2.15e9 for the per-block values
 * and 4.3e9 before the pool).  Any workspace of at least
 * fta_topk_score_workspace_min bytes (one chunk per 64 queries plus the fixed
 * parts) is accepted: the 256-query tiles whose streams do not fit are scored
 * and selected again by a fallback kernel (same results, more time).  Other
 * geometries store the [B][H][M][N] per-block values.
 */
size_t fta_topk_score_workspace_size(int B, int H, int N, int M);
size_t fta_topk_score_workspace_size_ex(int B, int H, int N, int D, int score_block_size, int pad_head,
                                        int pad_tail, int max_topk);
/* The least workspace fta_topk_score accepts for that geometry (the stream
 * path then holds one chunk per 64 queries and scores the rest again). */
size_t fta_topk_score_workspace_min(int B, int H, int N, int D, int score_block_size, int pad_head, int pad_tail,
                                    int max_topk);

/*
 * Fused scoring + selection: the result of fta_block_score followed by
 * fta_topk_select without materialising the [B][H][N][M] score tensor.
 * Replaces the composition in flash_topk_score (flash_topk_attn_v2/__init__.py:16-54).
 * Outputs are [B][H][N][M_OUT].
 */
int fta_topk_score(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                   const int64_t* q_strides, const int64_t* k_strides, int score_block_size,
                   int pad_head, int pad_tail, float scale, int max_topk, float threshold,
                   int32_t* topk_indices, float* topk_raw, float* topk_avg, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * Stage 1 of fta_topk_score alone, on its candidate-stream path (b = 64 or
 * 128, D <= 128, at most 32 blocks per query; FTA_ERR_UNSUPPORTED otherwise): the
 * scoring kernel writes, into the workspace, per-wave candidate streams of the
 * blocks that can still be in a query's top-k, the row totals and the bound
 * the selector starts from.  Exposed so that the scoring kernel can be timed
 * and profiled on its own; fta_topk_score runs it and then the selector.
 * Same arguments as fta_topk_score without threshold and outputs.  Stands for
 * the block-score half of the reference's composition (block_score_launch,
 * flash_topk_attn_v2/csrc/block_score_kernel.cu:19-258, as called from
 * flash_topk_attn_v2/__init__.py:16-54).
 */
int fta_topk_score_candidates(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                              const int64_t* q_strides, const int64_t* k_strides,
                              int score_block_size, int pad_head, int pad_tail, float scale,
                              int max_topk, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Stage 2 of fta_topk_score alone: the top-k selection (with the threshold
 * cut) over the candidate streams that fta_topk_score_candidates left in
 * `workspace` for the same inputs, geometry and max_topk, including the
 * fallback for tiles whose streams ran out of pool (which scores those tiles
 * again, so q and k are needed).  Same arguments as fta_topk_score;
 * FTA_ERR_UNSUPPORTED where fta_topk_score_candidates is.
 * fta_topk_score_candidates followed by this call gives the same outputs as
 * fta_topk_score.  On a workspace that no fta_topk_score_candidates call
 * filled for this geometry the outputs are undefined; the counts and chunk
 * ids read from it are clamped, so no access leaves the workspace and the
 * output arrays.  Stands for the reference's top-k stage (topk_select_launch,
 * flash_topk_attn_v2/csrc/topk_select.cpp, as called from
 * flash_topk_attn_v2/topk_select.py:185-311).
 */
int fta_topk_select_candidates(const void* q, const void* k, int dtype, int B, int H, int N, int D,
                               const int64_t* q_strides, const int64_t* k_strides, int score_block_size,
                               int pad_head, int pad_tail, float scale, int max_topk, float threshold,
                               int32_t* topk_indices, float* topk_raw, float* topk_avg, void* workspace,
                               size_t workspace_bytes, void* stream);

/* ---------------------------------------------------------------- indices */

/*
 * Per-(b, h, q-block) merge of g*K (index, score) pairs: sequential fp32
 * scatter-add in (row, slot) order, positive entries sorted by (score desc,
 * index asc), first qblock_topk kept, -1 / 0 padding; counts[slice] = #kept
 * (counts may be NULL, merged_scores may be NULL).
 * Replaces qblock_merge_launch (flash_topk_attn_v2/csrc/qblock_merge.cpp:3-14,
 * csrc/qblock_merge_kernel.cu:100-131) behind flash_qblock_merge
 * (flash_topk_attn_v2/qblock_merge.py:85-155).
 */
int fta_qblock_merge(const int32_t* topk_indices, const float* topk_scores, int64_t num_slices,
                     int q_block_size, int k_per_query, int num_score_blocks, int qblock_topk,
                     int32_t* merged_indices, float* merged_scores, int32_t* counts, void* stream);

/*
 * fta_qblock_merge with num_score_blocks = *max_index + 1 read on the device
 * (max_index: a device int32, the largest id in topk_indices, -1 if none),
 * so the caller need not synchronise before launching the merge.  Ids past
 * 4096 are outside the supported range; the caller checks the max on the host
 * (after this launch) and reports that case as an error.
 * Replaces the host-side max of build_qblock_topk_indices
 * (flash_topk_attn_v2/__init__.py:101-105) followed by qblock_merge_launch.
 */
int fta_qblock_merge_maxid(const int32_t* topk_indices, const float* topk_scores, int64_t num_slices,
                           int q_block_size, int k_per_query, const int32_t* max_index, int qblock_topk,
                           int32_t* merged_indices, float* merged_scores, int32_t* counts, void* stream);

/*
 * V1 q-block union: for each (b*h, q-block) the ascending unique non-negative
 * ids of the block's q_block_size * K top-k entries (query rows outside
 * [0, N) under the virtual q padding contribute nothing), written as a valid
 * prefix of merged_indices[bh][qm][0 .. s_max) followed by -1, and counts
 * [bh][qm] = the number of ids.  topk_indices is [BH, N, K] int32 contiguous;
 * s_max must be a power of two >= q_block_size * K and <= 8192.  Replaces
 * _build_qblock_indices_kernel behind V1 build_qblock_topk_indices
 * (flash_topk_attn/attention.py:23-138).
 */
int fta_qblock_union(const int32_t* topk_indices, int BH, int N, int K, int q_block_size, int q_pad_head,
                     int q_pad_tail, int s_max, int32_t* merged_indices, int32_t* counts, void* stream);

size_t fta_build_reverse_indices_workspace_size(int B, int H, int QM, int M);

/*
 * Reverse index: reverse_indices[b][h][m][:] = ascending q-block ids whose
 * merged list holds m (-1 padded to QM), reverse_counts[b][h][m], and
 * sorted_kv_indices[b][h][:] = stable descending argsort of the counts
 * (may be NULL).  Replaces build_reverse_indices_launch
 * (flash_topk_attn_v2/csrc/build_reverse_indices.cpp:3-14,
 * csrc/build_reverse_indices_kernel.cu:71-104) behind
 * flash_build_reverse_indices_cuda (flash_topk_attn_v2/build_reverse_indices_cuda.py:32-78).
 */
int fta_build_reverse_indices(const int32_t* merged_indices, const int32_t* counts, int B, int H,
                              int QM, int W, int M, int32_t* reverse_indices,
                              int32_t* reverse_counts, int32_t* sorted_kv_indices, void* workspace,
                              size_t workspace_bytes, void* stream);

/*
 * Stable descending sort of `total` int32 counts: sorted_counts and the
 * original positions sorted_ids.  Replaces sort_by_count_launch
 * (flash_topk_attn_v2/csrc/sort_by_count.cpp:3-13, csrc/sort_by_count_kernel.cu:6-51)
 * behind flash_sort_by_count_cuda (flash_topk_attn_v2/sort_by_count_cuda.py:33-67).
 */
int fta_sort_by_count(const int32_t* reverse_counts, int64_t total, int32_t* sorted_counts,
                      int32_t* sorted_ids, void* stream);

/* ---------------------------------------------------------------- attention */

size_t fta_sparse_attn_fwd_workspace_size(int B, int H, int N, int D, int q_block_size,
                                          int kv_block_size, int q_pad_head, int q_pad_tail,
                                          int kv_pad_head, int kv_pad_tail);

/*
 * Parts per workgroup walk of the forward with its workspace for this
 * geometry (0 for an invalid one): 1, or 2-4 when the grid has fewer than 128
 * workgroups and D <= 128.  Then each workgroup's walk over the union of its
 * q-blocks' lists (ascending, per 512-block segment) is split into that many
 * contiguous ranges, each with its own online-softmax anchor, and a combine
 * kernel merges the parts' (O, max, sum).  No counterpart in the reference
 * (its forward is never split); exposed so that callers and tests can tell
 * which schedule rounds P.
 */
int fta_sparse_attn_fwd_splits(int B, int H, int N, int D, int q_block_size, int kv_block_size,
                               int q_pad_head, int q_pad_tail, int kv_pad_head, int kv_pad_tail);

/*
 * Block-sparse attention forward over the merged KV-block lists
 * (merged_indices [B][H][QM][W], -1 entries ignored, order irrelevant):
 * o [B][N][H][D] (strided, same dtype) and lse [B][H][N] (natural log,
 * -inf and o = 0 for rows without candidate tokens).
 * Replaces sparse_attn_fwd_launch (flash_topk_attn_v2/csrc/sparse_attn.cpp:3-16,
 * csrc/sparse_attn_kernel.cu:368-457) behind flash_sparse_attn_cuda
 * (flash_topk_attn_v2/sparse_attn_cuda.py:42-110); lse = softmax_max + softmax_lse
 * of the reference (flash_topk_attn_v2/sparse_attn.py:391).
 * The workspace (fta_sparse_attn_fwd_workspace_size bytes: per-head work and
 * the XCD placement of the heads, and on small grids the split walks' partial
 * outputs, see fta_sparse_attn_fwd_splits) is optional: with workspace == NULL
 * or too few bytes the heads run in natural order and unsplit (the same o and
 * lse up to the rounding of P before P.V, which the split moves).
 */
int fta_sparse_attn_fwd(const void* q, const int64_t* q_strides, const void* k,
                        const int64_t* k_strides, const void* v, const int64_t* v_strides,
                        int dtype, int B, int H, int N, int D, const int32_t* merged_indices,
                        int QM, int W, int q_block_size, int kv_block_size, int q_pad_head,
                        int q_pad_tail, int kv_pad_head, int kv_pad_tail, float scale, void* o,
                        const int64_t* o_strides, float* lse, void* workspace,
                        size_t workspace_bytes, void* stream);

/*
 * delta[b][h][n] = sum_d o * dout (fp32).  Replaces preprocess_delta
 * (flash_topk_attn_v2/sparse_attn_bwd.py:12-33).
 */
int fta_preprocess_delta(const void* o, const int64_t* o_strides, const void* dout,
                         const int64_t* do_strides, int dtype, int B, int H, int N, int D,
                         float* delta, void* stream);

/*
 * Grouped-query forward: k and v hold Hk heads ([B][N][Hk][D] strided), query
 * head h reads K/V head h / (H / Hk); H must be a multiple of Hk.  The other
 * arguments and outputs are those of fta_sparse_attn_fwd (which equals this
 * call with Hk = H).  The reference rejects num_kv_heads != num_heads
 * (flash_topk_attn_v2/__init__.py:153-156); this extends flash_topk_attn there.
 */
int fta_sparse_attn_fwd_gqa(const void* q, const int64_t* q_strides, const void* k,
                            const int64_t* k_strides, const void* v, const int64_t* v_strides,
                            int dtype, int B, int H, int Hk, int N, int D,
                            const int32_t* merged_indices, int QM, int W, int q_block_size,
                            int kv_block_size, int q_pad_head, int q_pad_tail, int kv_pad_head,
                            int kv_pad_tail, float scale, void* o, const int64_t* o_strides,
                            float* lse, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Backward workspace: the membership bitmap, the lse in log2 units and the
 * dK/dV launch order, plus, on small grids, room for split walks (one region,
 * used by dK/dV and then by dQ): dK/dV with fewer workgroups than the GPU holds
 * at once (64-key blocks at D 64 / 128 / 256) and dQ with fewer than 128
 * workgroups (at most 128 at D 160 / 256) walk their lists in 2-4 parts whose
 * fp32 sums are added by a combine kernel.  A smaller workspace (at least the bitmap, lse and order)
 * runs the walks unsplit: the results then differ only in fp32 summation
 * order.  Sized for Hk = H; with Hk < H the dK/dV parts may not fit, and
 * dK/dV then runs unsplit.
 */
size_t fta_sparse_attn_bwd_workspace_size(int B, int H, int N, int D, int q_block_size,
                                          int kv_block_size, int q_pad_head, int q_pad_tail,
                                          int kv_pad_head, int kv_pad_tail);

/*
 * Backward: dq, dk, dv ([B][N][H][D] strided, same dtype as q) from the
 * forward's lse and delta.  dQ walks the merged lists; dK/dV walk the
 * transposed membership (built internally in the workspace) without atomics.
 * Replaces sparse_attn_bwd_dq_launch and sparse_attn_bwd_dkv_launch
 * (flash_topk_attn_v2/csrc/sparse_attn_bwd_dq.cpp:3-19, sparse_attn_bwd_dkv.cpp:3-20)
 * behind flash_sparse_attn_bwd_dq_cuda / flash_sparse_attn_bwd_dkv_cuda
 * (flash_topk_attn_v2/sparse_attn_bwd_dq_cuda.py:44-108,
 * sparse_attn_bwd_dkv_cuda.py:44-118) as called from
 * FlashSparseAttnFunc.backward (flash_topk_attn_v2/sparse_attn.py:163-224).
 * Runs dK/dV first, then dQ in the XCD head placement the dK/dV pass left in
 * the workspace (when every query head has its own K/V head).
 */
int fta_sparse_attn_bwd(const void* q, const int64_t* q_strides, const void* k,
                        const int64_t* k_strides, const void* v, const int64_t* v_strides,
                        const void* dout, const int64_t* do_strides, int dtype, int B, int H, int N,
                        int D, const int32_t* merged_indices, int QM, int W, int q_block_size,
                        int kv_block_size, int q_pad_head, int q_pad_tail, int kv_pad_head,
                        int kv_pad_tail, float scale, const float* lse, const float* delta, void* dq,
                        const int64_t* dq_strides, void* dk, const int64_t* dk_strides, void* dv,
                        const int64_t* dv_strides, void* workspace, size_t workspace_bytes,
                        void* stream);

/*
 * dQ alone ([B][N][H][D] strided; k, v with Hk heads): replaces
 * sparse_attn_bwd_dq_launch (flash_topk_attn_v2/csrc/sparse_attn_bwd_dq.cpp:3-19)
 * behind flash_sparse_attn_bwd_dq_cuda (sparse_attn_bwd_dq_cuda.py:44-108).
 * Needs no workspace (heads in natural order).
 */
int fta_sparse_attn_bwd_dq(const void* q, const int64_t* q_strides, const void* k,
                           const int64_t* k_strides, const void* v, const int64_t* v_strides,
                           const void* dout, const int64_t* do_strides, int dtype, int B, int H,
                           int Hk, int N, int D, const int32_t* merged_indices, int QM, int W,
                           int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail,
                           int kv_pad_head, int kv_pad_tail, float scale, const float* lse,
                           const float* delta, void* dq, const int64_t* dq_strides, void* stream);

/*
 * dK / dV alone (Hk heads, each summed over its H / Hk query heads without
 * atomics).  Builds the KV block -> q-block membership bitmap and the lse in
 * log2 units in the workspace (fta_sparse_attn_bwd_workspace_size bytes) and
 * walks it; for 64-key blocks at D 64 / 128 / 256 the workspace also holds the launch
 * order (KV blocks by selection count) and the XCD placement of the heads.  Replaces build_reverse_indices_launch + sparse_attn_bwd_dkv_launch
 * (flash_topk_attn_v2/csrc/build_reverse_indices.cpp:3-14,
 * sparse_attn_bwd_dkv.cpp:3-20) behind flash_sparse_attn_bwd_dkv_cuda
 * (sparse_attn_bwd_dkv_cuda.py:44-118).
 */
int fta_sparse_attn_bwd_dkv(const void* q, const int64_t* q_strides, const void* k,
                            const int64_t* k_strides, const void* v, const int64_t* v_strides,
                            const void* dout, const int64_t* do_strides, int dtype, int B, int H,
                            int Hk, int N, int D, const int32_t* merged_indices, int QM, int W,
                            int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail,
                            int kv_pad_head, int kv_pad_tail, float scale, const float* lse,
                            const float* delta, void* dk, const int64_t* dk_strides, void* dv,
                            const int64_t* dv_strides, void* workspace, size_t workspace_bytes,
                            void* stream);

/*
 * Grouped-query backward: dk and dv have Hk heads; each is the sum over the
 * H / Hk query heads that share the K/V head (accumulated in fp32 inside one
 * workgroup, no atomics).  Otherwise as fta_sparse_attn_bwd (= Hk = H).
 * Runs fta_sparse_attn_bwd_dq, then fta_sparse_attn_bwd_dkv.
 * Extends the reference the same way as fta_sparse_attn_fwd_gqa.
 */
int fta_sparse_attn_bwd_gqa(const void* q, const int64_t* q_strides, const void* k,
                            const int64_t* k_strides, const void* v, const int64_t* v_strides,
                            const void* dout, const int64_t* do_strides, int dtype, int B, int H,
                            int Hk, int N, int D, const int32_t* merged_indices, int QM, int W,
                            int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail,
                            int kv_pad_head, int kv_pad_tail, float scale, const float* lse,
                            const float* delta, void* dq, const int64_t* dq_strides, void* dk,
                            const int64_t* dk_strides, void* dv, const int64_t* dv_strides,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free backward.  No counterpart in the reference: it is for callers
 * that cannot allocate device memory (code under HIP graph capture, tight
 * serving or training loops, harnesses that forbid hipMalloc).  Same arguments
 * and results as fta_sparse_attn_bwd_gqa without (workspace, workspace_bytes):
 * the scratch (membership bitmap + lse in log2 units + launch order, and the
 * split parts of small grids when they fit too) lives in a device array of
 * FTA_NOALLOC_SCRATCH_BYTES inside the library, one per GPU, held until the
 * process ends.  The array belongs to the library's code object: every process
 * that loads the library reserves it on each GPU where the library's kernels
 * are loaded, whether or not it ever calls this entry point (64 MiB per GPU;
 * change FTA_NOALLOC_SCRATCH_BYTES here and rebuild to resize it).  A problem needing more returns FTA_ERR_UNSUPPORTED.  The call
 * allocates nothing (no hipMalloc, no library allocator); it uses the current
 * device's array, so `stream` must belong to the current device.  Calls that
 * overlap on one GPU (different streams, or host threads) race on the array.
 */
#define FTA_NOALLOC_SCRATCH_BYTES (64u << 20)
int fta_sparse_attn_bwd_noalloc(const void* q, const int64_t* q_strides, const void* k,
                                const int64_t* k_strides, const void* v, const int64_t* v_strides,
                                const void* dout, const int64_t* do_strides, int dtype, int B, int H,
                                int Hk, int N, int D, const int32_t* merged_indices, int QM, int W,
                                int q_block_size, int kv_block_size, int q_pad_head, int q_pad_tail,
                                int kv_pad_head, int kv_pad_tail, float scale, const float* lse,
                                const float* delta, void* dq, const int64_t* dq_strides, void* dk,
                                const int64_t* dk_strides, void* dv, const int64_t* dv_strides,
                                void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FTA_H_ */
