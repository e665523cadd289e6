/*
 * leanselect_hip.h -- C ABI of the MI355X (gfx950) LeanSelect prefill hot path.
 *
 * Plain pointers and sizes only.  Every tensor argument is a device pointer to
 * caller-owned memory; `cu_seqlens*` arrays are int32 device arrays of
 * `batch + 1` prefix offsets.  `stream` is a hipStream_t passed as void*.
 * Each entry point enqueues its work on `stream` and returns without
 * synchronising.  The return value is LS_OK or an LS_ERR_* code;
 * ls_last_error() then describes the failure (thread-local).
 *
 * Element types (argument `dtype`): LS_F32, LS_BF16, LS_F16.
 *
 * Paths in comments are relative to the LeanSelect repository root;
 * "paper1.patch:N" is line N of third_party/infllmv2/paper1.patch.
 */
#ifndef LEANSELECT_HIP_H
#define LEANSELECT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { LS_F32 = 0, LS_BF16 = 1, LS_F16 = 2 };

enum { LS_ATTN_RING_TIMEOUT = 1 };

/*
 * Column range of the varlen page max-pool (argument `clip`): a row of
 * sequence b pools the columns [0, cu_seqlens_k[b + 1] - cu_seqlens_k[b]) of
 * its score row (LS_POOL_CLIP_SEQUENCE) or the whole padded row [0,
 * max_seqlen_k) (LS_POOL_CLIP_ROW).  The two differ only where a shorter
 * sequence's padding columns hold values above -inf (the CIS window means
 * are 0 there).  The upstream kernel body that fixes this choice is not part
 * of the reference tree (third_party/infllmv2/paper1.patch:1831-1860 shows
 * only its offsets).
 */
enum { LS_POOL_CLIP_SEQUENCE = 0, LS_POOL_CLIP_ROW = 1 };

enum {
  LS_OK = 0,
  LS_ERR_INVALID = 1,     /* bad shape, geometry or pointer */
  LS_ERR_UNSUPPORTED = 2, /* valid request outside what the kernels support */
  LS_ERR_WORKSPACE = 3,   /* workspace missing or too small */
  LS_ERR_HIP = 4          /* a HIP runtime call failed */
};

/* Library version (major*10000 + minor*100 + patch). */
int ls_version(void);

/* Message for the last failing call on this host thread. */
const char* ls_last_error(void);

/*
 * Compressed keys: mean of `kernel_size`-token windows at `kernel_stride`,
 * per sequence (windows never cross a sequence boundary; a sequence shorter
 * than `kernel_size` yields no window).
 *   k        [total_k, num_kv_heads, head_dim], rows `k_row_stride` elements apart
 *   out      [total_atoms, num_kv_heads, head_dim] contiguous, same dtype
 *   cu_out   int32 [batch + 1] compressed prefix offsets (written)
 * `total_atoms` must equal sum_b max(0, (len_b - kernel_size) / kernel_stride + 1).
 * Replaces CompressK.forward + calc_chunks_with_stride
 * (leanselect/models/minicpm.py:1158-1185, 711-750).
 */
int ls_compress_k_varlen(const void* k, int64_t k_row_stride, const int32_t* cu_seqlens_k,
                         int32_t batch, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                         int32_t kernel_size, int32_t kernel_stride, void* out,
                         int64_t total_atoms, int32_t* cu_out, void* stream);

/*
 * Folded router weights in the reference layout:
 *   q_fused[h, d, r*F + j]  = head_mix[h, r]    * q_proj[r, d, j]   ([H, D, R*F])
 *   kv_fused[g, d, r*F + j] = kv_head_mix[g, r] * k_proj[r, d, j]   ([G, D, R*F])
 * Masters are float32; outputs are `dtype`.
 * Replaces LeanSelectSelector.fused_weights (leanselect/selector.py:144-158).
 */
int ls_fused_weights(const float* head_mix, const float* kv_head_mix, const float* q_proj,
                     const float* k_proj, int32_t num_heads, int32_t num_kv_heads,
                     int32_t head_dim, int32_t router_heads, int32_t router_dim, int32_t dtype,
                     void* q_fused, void* kv_fused, void* stream);

/*
 * Workspace bytes needed by ls_project_queries / ls_project_atom_keys /
 * ls_score_pages / ls_select_prefill.  Pass the sizes the call will see and 0
 * for those it does not take (total_atoms and max_pages for
 * ls_project_queries; total_q, batch and max_pages for ls_project_atom_keys;
 * batch and max_pages for ls_score_pages).  max_pages = ceil(max_seqlen_q /
 * block_size).
 */
size_t ls_select_workspace_size(int64_t total_q, int64_t total_atoms, int32_t batch,
                                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t router_heads, int32_t router_dim, int32_t max_pages,
                                int32_t dtype);

/*
 * GQA-group-summed query projection: out[g, n, f] =
 *   sum_{s < H/G, d} query[n, g*H/G + s, d] * q_fused[g*H/G + s, d, f], rounded to dtype.
 *   query [total_q, H, D] with rows `q_row_stride` elements apart; out [G, total_q, R*F].
 * The fused weights are formed from the float32 masters inside the call.
 * Replaces LeanSelectSelector.project_queries (leanselect/selector.py:160-177).
 */
int ls_project_queries(const void* query, int64_t q_row_stride, int64_t total_q,
                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                       const float* head_mix, const float* q_proj, int32_t router_heads,
                       int32_t router_dim, int32_t dtype, void* out, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * Rotary embedding of the query heads fused with ls_project_queries: the H
 * query heads of query [total_q, H, D] (rows q_row_stride elements apart) are
 * rotated in place exactly as ls_rope_inplace rotates them (positions int32,
 * cos_table / sin_table float32 [table_rows, 128]), and out [G, total_q, R*F]
 * is the projection of the rotated rows, bit-identical to calling
 * ls_rope_inplace and then ls_project_queries.  bf16 or fp16, head_dim 128,
 * router width R*F 64 or 128.  Workspace as for ls_project_queries.
 * Replaces apply_rotary_pos_emb on the queries (leanselect/models/minicpm.py:
 * 1027-1070, called at 2219-2222) followed by LeanSelectSelector.project_queries
 * on the rotated queries (selector.py:160-177, reached from minicpm.py:
 * 2504-2508 and 3061-3142): the projection no longer reads the queries again.
 */
int ls_rope_project_queries(void* query, int64_t q_row_stride, const int32_t* positions,
                            int64_t total_q, int32_t num_heads, int32_t num_kv_heads,
                            int32_t head_dim, const float* cos_table, const float* sin_table,
                            int64_t table_rows, const float* head_mix, const float* q_proj,
                            int32_t router_heads, int32_t router_dim, int32_t dtype, void* out,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Atom-key projection: out[g, a, f] = sum_d kc[a, g, d] * kv_fused[g, d, f].
 *   kc [n_atoms, G, D] with rows `kc_row_stride` elements apart; out [G, n_atoms, R*F].
 * Replaces LeanSelectSelector.project_atom_keys (leanselect/selector.py:179-190).
 */
int ls_project_atom_keys(const void* kc, int64_t kc_row_stride, int64_t n_atoms,
                         int32_t num_kv_heads, int32_t head_dim, const float* kv_head_mix,
                         const float* k_proj, int32_t router_heads, int32_t router_dim,
                         int32_t dtype, void* out, void* workspace, size_t workspace_bytes,
                         void* stream);

/*
 * Page scores of one sequence: atom scores q~ . k~ (rounded to dtype) max-pooled
 * over the overlapping window [p*s - 1, p*s + s) of atoms, s = block_size /
 * kernel_stride, -inf where the window holds no atom.
 *   query [n, H, D], kc [n_atoms, G, D], out [G, n, ceil(seq_len / block_size)].
 * Replaces LeanSelectSelector.score_pages + pool_atoms_to_pages(reduce="max")
 * (leanselect/selector.py:192-214; leanselect/pages.py:146-187).
 */
int ls_score_pages(const void* query, int64_t q_row_stride, int64_t n_queries,
                   const void* kc, int64_t kc_row_stride, int64_t n_atoms, int32_t num_heads,
                   int32_t num_kv_heads, int32_t head_dim, const float* head_mix,
                   const float* kv_head_mix, const float* q_proj, const float* k_proj,
                   int32_t router_heads, int32_t router_dim, int32_t dtype, int64_t seq_len,
                   int32_t block_size, int32_t kernel_stride, void* out, void* workspace,
                   size_t workspace_bytes, void* stream);

/*
 * Page max-pool of atom scores: out[r, p] = max over atoms
 * [p*pool_stride - 1, p*pool_stride + pool_stride) clipped to [0, n_atoms) of
 * atom_scores[r, a] (-inf when empty); rows `row_stride` elements apart,
 * out [rows, n_pages] contiguous.
 * Replaces pool_atoms_to_pages(reduce="max") (leanselect/pages.py:146-187).
 */
int ls_pool_atoms_to_pages(const void* atom_scores, int64_t rows, int64_t n_atoms,
                           int64_t row_stride, int32_t dtype, int64_t n_pages,
                           int32_t pool_stride, void* out, void* stream);

/*
 * Forced-page mask: out[i, p] = p < init_blocks || (qp_i >= p && qp_i <= p + local_blocks)
 * with qp_i = floor(positions[i] / block_size); positions int64 [n], out uint8 [n, num_pages].
 * Replaces forced_page_mask (leanselect/pages.py:222-240).
 */
int ls_forced_page_mask(const int64_t* positions, int64_t n, int64_t num_pages,
                        int32_t block_size, int32_t init_blocks, int32_t local_blocks,
                        uint8_t* out, void* stream);

/*
 * Prefill page plans.  For each sequence b, query row t (relative page
 * qp = t / block_size) and KV group g: pages p > qp are invisible, pages
 * p < init_blocks and qp - local_blocks <= p <= qp are forced, and the
 * remaining slots of take_b = min(take, ceil(len_q_b / block_size)) go to the
 * highest page scores (ties to the lower page index).  Each row of
 * topk_idx [G, total_q, take] (int32) lists its ids in ascending order and is
 * padded with -1.  Rows of a sequence without query or compressed key are all -1.
 *   q [total_q, H, D] (rows q_row_stride apart), kc [total_atoms, G, D] (rows
 *   kc_row_stride apart), cu_seqlens_q / cu_seqlens_kc int32 [batch + 1],
 *   take = min(topk, ceil(max_seqlen_q / block_size)).
 * Replaces MiniCPMInfLLMv2Attention._lightweight_compressed_attention
 * (leanselect/models/minicpm.py:3061-3142).
 */
int ls_select_prefill(const void* q, int64_t q_row_stride, int64_t total_q, const void* kc,
                      int64_t kc_row_stride, int64_t total_atoms, const int32_t* cu_seqlens_q,
                      const int32_t* cu_seqlens_kc, int32_t batch, int32_t max_seqlen_q,
                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                      const float* head_mix, const float* kv_head_mix, const float* q_proj,
                      const float* k_proj, int32_t router_heads, int32_t router_dim,
                      int32_t dtype, int32_t topk, int32_t block_size, int32_t kernel_stride,
                      int32_t init_blocks, int32_t local_blocks, int32_t* topk_idx,
                      int32_t take, void* workspace, size_t workspace_bytes, void* stream);

/*
 * ls_select_prefill with the query projection q_tilde [G, total_q, R*F]
 * (dtype, dense) given instead of the queries, e.g. from
 * ls_rope_project_queries; only the key-side masters (kv_head_mix, k_proj)
 * are read.  Same plans as ls_select_prefill on the queries q_tilde was
 * projected from.
 * Replaces the same selection (leanselect/models/minicpm.py:3061-3142) with
 * its q~ produced where the queries are rotated (minicpm.py:2219-2222).
 */
int ls_select_prefill_qt(const void* q_tilde, int64_t total_q, const void* kc,
                         int64_t kc_row_stride, int64_t total_atoms, const int32_t* cu_seqlens_q,
                         const int32_t* cu_seqlens_kc, int32_t batch, int32_t max_seqlen_q,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                         const float* kv_head_mix, const float* k_proj, int32_t router_heads,
                         int32_t router_dim, int32_t dtype, int32_t topk, int32_t block_size,
                         int32_t kernel_stride, int32_t init_blocks, int32_t local_blocks,
                         int32_t* topk_idx, int32_t take, void* workspace,
                         size_t workspace_bytes, void* stream);

/*
 * Workspace bytes needed by ls_sparse_attn_varlen.
 *
 * Status word: the first 4 bytes of an attention workspace (this entry point's
 * and ls_nosa_attn_varlen's) hold an int32 status once the call's kernels have
 * completed on `stream`: 0, or LS_ATTN_RING_TIMEOUT when a wave's bounded wait
 * for a staged page expired, in which case the outputs are invalid.  The
 * kernels never synchronise; a caller reads the word after the stream work
 * ends (the Python mirror does so after every call and raises RuntimeError).
 */
size_t ls_sparse_attn_workspace_size(int64_t total_k, int32_t batch, int32_t num_kv_heads,
                                     int32_t head_dim, int32_t max_seqlen_k, int32_t dtype);

/*
 * Block-sparse attention over per-token page plans:
 *   out[t, h] = softmax_j(scale * q[t, h] . k[j, h / (H/G)]) v[j, h / (H/G)]
 * over keys j of the valid ids in topk_idx[h / (H/G), t, :] (each id once;
 * -1 and out-of-range ids ignored) with, when causal, j <= t + len_k - len_q
 * (relative to the sequence starts).  A row without any key gets out = 0 and
 * lse = +inf.  lse [H, total_q] float32 (natural log) is written when non-null.
 *   q [total_q, H, D], k / v [total_k, G, D] (rows *_row_stride apart),
 *   topk_idx int32 [G, total_q, take], out [total_q, H, D] contiguous.
 * Supports dtype LS_BF16 and LS_F16, head_dim 128, page (block) size 64.
 * softmax_scale <= 0 selects head_dim^-0.5.
 * Replaces infllmv2_attn_varlen_func(..., topk_idx=) (paper1.patch:1993-2100,
 * called at leanselect/models/minicpm.py:3216-3244 and nosa.py:2213-2254).
 */
int ls_sparse_attn_varlen(const void* q, int64_t q_row_stride, const void* k,
                          int64_t k_row_stride, const void* v, int64_t v_row_stride,
                          const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                          int32_t batch, int64_t total_q, int64_t total_k, int32_t max_seqlen_q,
                          int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads,
                          int32_t head_dim, int32_t dtype, const int32_t* topk_idx,
                          int32_t take, int32_t block_size, float softmax_scale,
                          int32_t causal, void* out, float* lse, void* workspace,
                          size_t workspace_bytes, void* stream);

/*
 * Allocation-free ls_sparse_attn_varlen.  No counterpart in the reference: it
 * is for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments and results as ls_sparse_attn_varlen without the workspace: the
 * kernels use a static device array of the library, LS_NOALLOC_SCRATCH_BYTES
 * (64 MiB) per GPU, held from the library's first use of that GPU until the
 * process ends.  The call allocates nothing (no hipMalloc / hipFree and no
 * allocating library routine); a request whose workspace would exceed the
 * array (ls_sparse_attn_workspace_size > 64 MiB, about 65000 keys at 2 KV
 * heads) fails with LS_ERR_UNSUPPORTED before any device work.  `status`
 * (optional, device int32) receives the status word described above (0 for a
 * call with no query row or no sequence, written by a one-thread kernel);
 * without it the word stays in the array.  Every call on one GPU shares that GPU's
 * array, so calls that overlap on one GPU (concurrent streams or host threads)
 * race and must be serialised by the caller.
 */
#define LS_NOALLOC_SCRATCH_BYTES (64u << 20)
int ls_sparse_attn_varlen_noalloc(const void* q, int64_t q_row_stride, const void* k,
                                  int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                  const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                  int32_t batch, int64_t total_q, int64_t total_k,
                                  int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                                  int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                  const int32_t* topk_idx, int32_t take, int32_t block_size,
                                  float softmax_scale, int32_t causal, void* out, float* lse,
                                  int32_t* status, void* stream);

/*
 * Bound of one wait of the attention kernels for a staged page, in polls
 * (default 1 << 22, far above any wait of a working launch).  Sets the bound
 * for later launches from this process and returns the previous one; a
 * negative value restores the default.  A testing hook: a bound of 0 makes
 * every wait expire at once (the kernels still finish, with the status word
 * set), so the error path can be exercised without a fault.  No counterpart in
 * the reference.
 */
int32_t ls_attn_set_spin_limit(int32_t spins);

/* ------------------------------------------------------------------------ */
/* NOSA variant (leanselect/models/nosa.py, --method leanselect)             */
/* ------------------------------------------------------------------------ */

/*
 * CIS mean pooling: out[h, t, m] = mean of cis[cu_seqlens[b] + 16 m + i, h]
 * over i < 32 for every row t of sequence b when 16 m + 32 <= len(b), else 0.
 *   cis [total_n, num_heads] (rows cis_row_stride elements apart);
 *   out [num_heads, total_n, out_cols] contiguous, out_cols = max_seqlen / 16 - 1.
 * Sums in float32, rounded once to dtype.  kernel_size 32, stride 16 only.
 * Replaces nosa_mean_pooling (leanselect/ops/cis_pooling.py:8-72).
 */
int ls_cis_mean_pool(const void* cis, int64_t cis_row_stride, int64_t total_n,
                     int32_t num_heads, const int32_t* cu_seqlens, int32_t batch,
                     int32_t max_seqlen, int32_t kernel_size, int32_t stride, int32_t dtype,
                     void* out, int32_t out_cols, void* stream);

/*
 * Varlen page max-pool with the forced overlay:
 *   input [num_heads, total_q, max_seqlen_k] -> out [num_heads, total_q, out_len].
 * Row t of sequence b has page off = (t - cu_seqlens_q[b] + cache_lens[b]) /
 * block_size.  Page p is +inf when p < init_blocks or off - local_blocks <= p
 * <= off, else the max of input[h, t, j] over j in [p s - 1, p s + s) clipped
 * to [0, min(cu_seqlens_k[b + 1] - cu_seqlens_k[b], max_seqlen_k))
 * (clip = LS_POOL_CLIP_SEQUENCE) or to [0, max_seqlen_k) (LS_POOL_CLIP_ROW),
 * -inf when empty, s = block_size / stride.
 * Replaces infllm_v2.max_pooling_1d_varlen (third_party/infllmv2/paper1.patch:2664-2760,
 * called at leanselect/models/nosa.py:1263-1286).
 */
int ls_page_maxpool_varlen(const void* input, const int32_t* cu_seqlens_q,
                           const int32_t* cu_seqlens_k, const int32_t* cache_lens, int32_t batch,
                           int32_t num_heads, int64_t total_q, int64_t max_seqlen_k,
                           int64_t out_len, int32_t local_blocks, int32_t init_blocks,
                           int32_t block_size, int32_t stride, int32_t clip, int32_t dtype,
                           void* out, void* stream);

/*
 * Workspace bytes needed by ls_nosa_select_prefill (max_pages =
 * ceil(max_seqlen_q / block_size)).
 */
size_t ls_nosa_select_workspace_size(int64_t total_q, int64_t total_atoms, int32_t batch,
                                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t router_heads, int32_t router_dim,
                                     int32_t max_pages, int32_t dtype);

/*
 * NOSA prefill page plans, the LeanSelect branch of compressed_attention:
 *   1. qk page scores: the folded-router atom scores (as ls_select_prefill),
 *      max-pooled to pages with sink and local pages +inf, no causal mask
 *      (-inf past the sequence's atoms, so the clip does not change them);
 *   2. the min(init + local + select, out_len) best qk pages (ties to the
 *      lower page) form a shortlist;
 *   3. CIS page scores: CIS window means (cis [total_k, num_kv_heads], rows
 *      cis_row_stride apart, of cis_dtype; windows of sequence b per
 *      cu_seqlens_k; 0 past the sequence's windows up to the longest
 *      sequence's count) max-pooled to pages under `pool_clip` (an
 *      LS_POOL_CLIP_* value: the sequence's own windows, or every column up
 *      to the longest sequence's window count), sink/local pages +inf, pages
 *      after q_idx -inf, shortlisted pages +inf;
 *   4. topk_idx [num_kv_heads, total_q, take] int32: the take = min(topk,
 *      out_len) best pages, ascending, ids after q_idx replaced by -1.
 * out_len = ceil(max_seqlen_q / block_size); q_idx = (t - cu_seqlens_q[b] +
 * max_seqlen_q - len_q(b)) / block_size.  block_size 64, kernel_stride 16.
 * Replaces compressed_attention(..., precomputed_qk_score=...) with
 * _leanselect_atom_scores (leanselect/models/nosa.py:1144-1307, 1822-1853).
 */
int ls_nosa_select_prefill(const void* q, int64_t q_row_stride, int64_t total_q, const void* kc,
                           int64_t kc_row_stride, int64_t total_atoms, const void* cis,
                           int64_t cis_row_stride, int32_t cis_dtype,
                           const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kc,
                           const int32_t* cu_seqlens_k, int32_t batch, int32_t max_seqlen_q,
                           int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                           const float* head_mix, const float* kv_head_mix, const float* q_proj,
                           const float* k_proj, int32_t router_heads, int32_t router_dim,
                           int32_t dtype, int32_t topk, int32_t block_size,
                           int32_t kernel_stride, int32_t init_blocks, int32_t local_blocks,
                           int32_t select_blocks, int32_t pool_clip, int32_t* topk_idx,
                           int32_t take, void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace bytes needed by ls_nosa_attn_varlen.
 */
size_t ls_nosa_attn_workspace_size(int64_t total_k, int32_t batch, int32_t num_kv_heads,
                                   int32_t head_dim, int32_t max_seqlen_k, int32_t dtype);

/*
 * NOSA attention: ls_sparse_attn_varlen (causal) with a per-key bias,
 *   out[t, h] = sum_j w_j v[j] / sum_j w_j,  w_j = exp(scale * q[t, h] . k[j] + cis[j, g]),
 * the closed form of attn(q, k, v * e^cis) / attn(q, k, e^cis) (both through
 * infllmv2_attn_varlen_func at leanselect/models/nosa.py:2211-2255) in one
 * pass.  cis [total_k, num_kv_heads] of cis_dtype (finite), rows
 * cis_row_stride apart.  lse (optional) is the log of sum_j w_j.
 */
int ls_nosa_attn_varlen(const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride,
                        const void* v, int64_t v_row_stride, const void* cis,
                        int64_t cis_row_stride, int32_t cis_dtype, const int32_t* cu_seqlens_q,
                        const int32_t* cu_seqlens_k, int32_t batch, int64_t total_q,
                        int64_t total_k, int32_t max_seqlen_q, int32_t max_seqlen_k,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                        const int32_t* topk_idx, int32_t take, int32_t block_size,
                        float softmax_scale, void* out, float* lse, void* workspace,
                        size_t workspace_bytes, void* stream);

/* ------------------------------------------------------------------------
 * Decoder-layer producers and consumers of the LeanSelect attention layer
 * (MiniCPM4.1 prefill, leanselect/models/minicpm.py:3562-3630).  16-bit
 * dtypes only; rows are `*_row_stride` elements apart; every tensor is
 * 16-byte aligned.  Each output element is rounded where the reference's
 * torch expression rounds.
 * ------------------------------------------------------------------------ */

/*
 * RMSNorm: out = round(round(x * (1 / sqrt(mean(x^2) + eps))) * weight), the
 * statistics in float32.  x, out [n_rows, hidden]; weight [hidden].
 * hidden is a multiple of 8 up to 8192.
 * Replaces rms_layernorm (leanselect/models/minicpm.py:772-788).
 */
int ls_rmsnorm(const void* x, int64_t x_row_stride, const void* weight, int64_t n_rows,
               int32_t hidden, float eps, int32_t dtype, void* out, int64_t out_row_stride,
               void* stream);

/*
 * Scaled residual add fused with the next RMSNorm:
 *   residual = round(residual + round(h * h_scale))   (in place)
 *   out      = RMSNorm(residual) as ls_rmsnorm.
 * Replaces `residual + hidden_states * (scale_depth / sqrt(num_layers))`
 * followed by the next MiniCPMRMSNorm (leanselect/models/minicpm.py:3616-3625,
 * 3578; the last layer's add feeds the model's final norm, 3698).
 */
int ls_add_rmsnorm(void* residual, int64_t res_row_stride, const void* h, int64_t h_row_stride,
                   float h_scale, const void* weight, int64_t n_rows, int32_t hidden, float eps,
                   int32_t dtype, void* out, int64_t out_row_stride, void* stream);

/*
 * Rotary embedding in place on the query heads (columns [0, n_q_heads *
 * head_dim)) and key heads (columns k_col_offset + [0, n_k_heads * head_dim))
 * of each row: x = round(x * cos[p] + rotate_half(x) * sin[p]) in float32
 * (no fused multiply-add), p = positions[row] (int32, 0 <= p < table_rows;
 * the kernel clamps out-of-range values).  cos_table / sin_table are float32
 * [table_rows, head_dim].  head_dim must be 128.
 * Replaces apply_rotary_pos_emb on the q/k projections
 * (leanselect/models/minicpm.py:1027-1070, called at 2218-2222).
 */
int ls_rope_inplace(void* x, int64_t row_stride, const int32_t* positions, int64_t n_rows,
                    int32_t n_q_heads, int32_t n_k_heads, int64_t k_col_offset, int32_t head_dim,
                    const float* cos_table, const float* sin_table, int64_t table_rows,
                    int32_t dtype, void* stream);

/*
 * Rotary embedding of the key heads fused with the compressed keys: rotates
 * the n_k_heads key heads (columns k_col_offset + [0, n_k_heads * 128)) of every
 * row in place exactly as ls_rope_inplace, and writes the compressed keys of
 * the rotated rows as ls_compress_k_varlen would (windows of 32 rows at
 * stride 16 inside each sequence of cu_seqlens, float32 sums, one rounding):
 *   kc_out [total_atoms, n_k_heads, 128] contiguous, cu_out int32 [batch + 1].
 * Each rotated row is summed while it is written, so the keys are not read
 * again.  head_dim 128, kernel 32 / stride 16; workspace from
 * ls_rope_k_compress_workspace_size.
 * Replaces apply_rotary_pos_emb on the keys (leanselect/models/minicpm.py:1027-1070,
 * 2218-2222) followed by CompressK.forward (minicpm.py:1158-1185) on them.
 */
size_t ls_rope_k_compress_workspace_size(int64_t n_rows, int32_t batch, int32_t n_k_heads,
                                         int32_t head_dim);
int ls_rope_k_compress(void* x, int64_t row_stride, const int32_t* positions,
                       const int32_t* cu_seqlens, int32_t batch, int64_t n_rows,
                       int32_t n_k_heads, int64_t k_col_offset, int32_t head_dim,
                       const float* cos_table, const float* sin_table, int64_t table_rows,
                       int32_t dtype, void* kc_out, int64_t total_atoms, int32_t* cu_out,
                       void* workspace, size_t workspace_bytes, void* stream);

/*
 * SiLU-gated activation: out = round(round(silu(g)) * u), g = columns
 * [0, inter) and u = columns [inter, 2 inter) of gate_up.
 * Replaces act_fn(gate_proj(x)) * up_proj(x) in MiniCPMMLP.forward
 * (leanselect/models/minicpm.py:1098-1135).
 */
int ls_silu_mul(const void* gate_up, int64_t gu_row_stride, int64_t n_rows, int32_t inter,
                int32_t dtype, void* out, int64_t out_row_stride, void* stream);

/*
 * Scaled token embedding: out[n] = round(table[ids[n]] * scale), out
 * [n, hidden] contiguous; ids int32 in [0, vocab) (clamped otherwise).
 * Replaces `embed_tokens(input_ids) * scale_emb`
 * (leanselect/models/minicpm.py:3773-3774).
 */
int ls_embed_scale(const int32_t* ids, int64_t n, const void* table, int64_t vocab,
                   int32_t hidden, float scale, int32_t dtype, void* out, void* stream);

/* ------------------------------------------------------------------------
 * Decode over a KV cache.  k_cache / v_cache hold [batch][capacity][G][D]
 * rows and kc_cache [batch][kc_capacity][G][D] (strides in elements, head
 * stride D); cache_seqlens (int32 [batch], device) counts each sequence's
 * tokens.  bf16 or fp16.
 * ------------------------------------------------------------------------ */

/*
 * Append packed new tokens (k_new / v_new [total_new, G, D], row stride
 * new_row_stride; sequence b's rows are [cu_seqlens_new[b], cu_seqlens_new[b+1]))
 * at positions cache_seqlens[b] + i, and, when kc_cache is given, write every
 * compressed key window the new tokens complete: window w of sequence b is
 * the mean of key rows [w * kernel_stride, w * kernel_stride + kernel_size)
 * (float32 sums, one rounding; for 2 x stride windows the two half sums are
 * added, as ls_compress_k_varlen sums them, so both give the same bits).
 * cache_seqlens is not advanced: the caller adds the new lengths afterwards.
 * max_new_windows bounds the new windows of the whole batch (the grid size;
 * sum over b of ceil(n_new(b) / kernel_stride) + batch always suffices);
 * cu_windows is int32 [batch + 1] device scratch.  The caller guarantees
 * cache_seqlens[b] + n_new(b) <= capacity and the windows fit kc_capacity.
 * Replaces DynamicLayer.update plus InfLLMv2CacheLayer.update_no_compress_k /
 * update_compress_k (leanselect/models/minicpm.py:1237-1325, called at
 * 2776-2823 and 2888-2958).
 */
int ls_kvcache_append(void* k_cache, void* v_cache, int64_t cache_batch_stride,
                      int64_t cache_row_stride, const int32_t* cache_seqlens, const void* k_new,
                      const void* v_new, int64_t new_row_stride, const int32_t* cu_seqlens_new,
                      int64_t total_new, int32_t batch, int32_t num_kv_heads, int32_t head_dim,
                      int32_t dtype, void* kc_cache, int64_t kc_batch_stride,
                      int64_t kc_row_stride, int64_t max_new_windows, int32_t kernel_size,
                      int32_t kernel_stride, int32_t* cu_windows, void* stream);

/*
 * Stage-1 page plans for decode rows: q [total_q, H, D] packed by
 * cu_seqlens_q (row i of sequence b sits at position
 * cache_seqlens[b] - len_q(b) + i, cache_seqlens counting the rows' own
 * tokens).  Per row and KV group g:
 *   score[j] = sum_{h in g} softmax_j(softmax_scale * q_h . kc_j)
 * over the sequence's n_c = (len - kernel_size) / kernel_stride + 1 compressed
 * keys (no causal limit), rounded to the query dtype and then to bf16; the
 * page max-pool with forced sink / local pages of ls_page_maxpool_varlen
 * (cache_lens = len - len_q); then the `take` = min(topk, out_len) best pages
 * (ties to the lower page), ascending, ids past the row's own page replaced
 * by -1.  topk_idx: int32 [G, total_q, take].  max_kc = n_c of the longest
 * sequence; out_len = ceil((max len_q + max(len - len_q)) / block_size)
 * (at most 30720).  head_dim 128, at most 16 query heads per KV head; kc_cache rows
 * dense (kc_row_stride = G * D).  Workspace from
 * ls_decode_select_workspace_size.
 * Replaces compressed_attention with cache_lens (leanselect/models/minicpm.py:594-705,
 * called at 2718-2736 with cache_lens = seq_lens_k - 1 from 2509-2512) on
 * infllmv2_attn_stage1 with causal=False (third_party/infllmv2/paper1.patch:
 * 1103-1302, 2340-2362) and max_pooling_1d_varlen (paper1.patch:2664-2760).
 */
size_t ls_decode_select_workspace_size(int64_t total_q, int32_t batch, int32_t num_kv_heads,
                                       int64_t max_kc, int64_t out_len);
int ls_decode_select(const void* q, int64_t q_row_stride, const int32_t* cu_seqlens_q,
                     int64_t total_q, const void* kc_cache, int64_t kc_batch_stride,
                     int64_t kc_row_stride, const int32_t* cache_seqlens, int32_t batch,
                     int64_t max_kc, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                     int32_t dtype, float softmax_scale, int32_t topk, int32_t block_size,
                     int32_t kernel_size, int32_t kernel_stride, int32_t init_blocks,
                     int32_t local_blocks, int64_t out_len, int32_t take, int32_t* topk_idx,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Stage-1 scores of packed query rows over packed compressed keys, without a
 * causal limit (the decode form):
 *   out[g, t, j] = sum over the heads h of group g of softmax_j(scale * q[t, h]
 *                  . kc[cu_seqlens_kc[b] + j, g])   for j < n_c(b),
 * n_c(b) = min(cu_seqlens_kc[b + 1] - cu_seqlens_kc[b], max_kc) for the row's
 * sequence b; 0 for j >= n_c(b) and where the score is NaN.  Rounded to the
 * query dtype.  q [total_q, H, D] (rows q_row_stride apart), kc [total_kc, G,
 * D] (rows kc_row_stride apart), out [G, total_q, out_cols] contiguous.
 * head_dim 128, at most 16 query heads per KV head, bf16 or fp16.  Workspace
 * from ls_stage1_scores_workspace_size.
 * Replaces infllmv2_attn_stage1(q, k, v, cu_seqlens_q=, cu_seqlens_k=,
 * cu_seqlens_v=, max_seqlen_q=, max_seqlen_k=, causal=False)
 * (third_party/infllmv2/paper1.patch:2312-2361, NaN -> 0 at 2359), which
 * compressed_attention calls when decoding (leanselect/models/minicpm.py:
 * 673-683).
 */
size_t ls_stage1_scores_workspace_size(int64_t total_q, int32_t num_kv_heads, int64_t max_kc);
int ls_stage1_scores(const void* q, int64_t q_row_stride, const int32_t* cu_seqlens_q,
                     int64_t total_q, const void* kc, int64_t kc_row_stride,
                     const int32_t* cu_seqlens_kc, int32_t batch, int64_t max_kc,
                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                     float softmax_scale, void* out, int64_t out_cols, void* workspace,
                     size_t workspace_bytes, void* stream);

/*
 * Block-sparse attention of packed query rows over the cache: row i of
 * sequence b attends the keys of its valid plan ids (topk_idx [G, total_q,
 * topk], each page once) with j < cache_seqlens[b] (causal = 0) or
 * j <= cache_seqlens[b] - len_q(b) + i (causal = 1).  out [total_q, H, D] in
 * the cache dtype, softmax_lse float32 [H, total_q] (natural log; +inf and a
 * zero row when no key is visible) or NULL.  Split-K: each (row, group) plan
 * is cut into n_splits slices (1 <= n_splits <= 64), each run by a workgroup of
 * four waves, and the slices are merged by a second kernel.  head_dim 128,
 * at most 16 query heads per KV head, topk <= 256.  Workspace from
 * ls_sparse_attn_kvcache_workspace_size.
 * Replaces infllmv2_attn_with_kvcache(q, k_cache, v_cache, cache_seqlens=,
 * causal=, topk_idx=) (third_party/infllmv2/paper1.patch:2511-2615) and the
 * decode call infllmv2_attn_varlen_func(..., causal=False, topk_idx=) over the
 * cached keys (leanselect/models/minicpm.py:3216-3244).
 */
size_t ls_sparse_attn_kvcache_workspace_size(int64_t total_q, int32_t num_kv_heads,
                                             int32_t n_splits);
int ls_sparse_attn_kvcache(const void* q, int64_t q_row_stride, const int32_t* cu_seqlens_q,
                           int64_t total_q, const void* k_cache, const void* v_cache,
                           int64_t cache_batch_stride, int64_t cache_row_stride,
                           const int32_t* cache_seqlens, int32_t batch, int32_t num_heads,
                           int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                           const int32_t* topk_idx, int32_t topk, float softmax_scale,
                           int32_t causal, int32_t n_splits, void* out, float* softmax_lse,
                           void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* LEANSELECT_HIP_H */
