// NOSA variant of the LeanSelect prefill selection.
//
//   ls_cis_mean_pool        nosa_mean_pooling             leanselect/ops/cis_pooling.py:8-72
//   ls_page_maxpool_varlen  max_pooling_1d_varlen         third_party/infllmv2/paper1.patch:2664-2760
//                           (contract as restated in leanselect/baselines/page_topk.py:4-26, 94-117)
//   NOSA top-k (internal)   compressed_attention tail     leanselect/models/nosa.py:1262-1305
//
// The fused selection entry point (ls_nosa_select_prefill) lives with the
// projections and page scoring in ls_select.hip and calls the launchers here.
#include "ls_common.h"
#include "ls_nosa_internal.h"

// ---------------------------------------------------------------------------
// CIS mean pooling, the drop-in form: out[h][t][m] = mean of the 32 CIS values
// cis[start_b + 16 m .. +32][h] for every row t of sequence b when that window
// lies inside the sequence, else 0.  One workgroup per (64 windows, sequence,
// head): the 64 means are computed once (float32 sum of 32 values, one
// rounding) and broadcast to the sequence's rows.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void ls_cis_mean_pool_kernel(
    const typename LsElem<DT>::T* __restrict__ cis, int64_t cis_rs, const int32_t* __restrict__ cu,
    int64_t total_n, int M, typename LsElem<DT>::T* __restrict__ out) {
  __shared__ typename LsElem<DT>::T s_mean[64];
  const int b = blockIdx.y, h = blockIdx.z;
  const int m0 = blockIdx.x * 64;
  const int64_t start = cu[b], end = cu[b + 1];
  const int64_t n = end - start;
  const int tid = threadIdx.x;
  if (tid < 64) {
    const int m = m0 + tid;
    typename LsElem<DT>::T v = LsElem<DT>::from_f(0.f);
    if (m < M && (int64_t)m * 16 + 32 <= n) {
      float acc = 0.f;
      for (int i = 0; i < 32; ++i) acc += LsElem<DT>::to_f(cis[(start + (int64_t)m * 16 + i) * cis_rs + h]);
      v = LsElem<DT>::from_f(acc * (1.f / 32.f));
    }
    s_mean[tid] = v;
  }
  __syncthreads();
  const int mw = min(64, M - m0);
  for (int64_t i = tid; i < n * mw; i += 256) {
    const int64_t t = start + i / mw;
    const int mm = (int)(i % mw);
    out[((int64_t)h * total_n + t) * M + m0 + mm] = s_mean[mm];
  }
}

extern "C" int ls_cis_mean_pool(const void* cis, int64_t cis_row_stride, int64_t total_n,
                                int32_t num_heads, const int32_t* cu_seqlens, int32_t batch,
                                int32_t max_seqlen, int32_t kernel_size, int32_t stride,
                                int32_t dtype, void* out, int32_t out_cols, void* stream) {
  LS_REQUIRE(kernel_size == 32 && stride == 16, LS_ERR_UNSUPPORTED,
             "ls_cis_mean_pool: kernel_size 32 and stride 16 only (got %d/%d)", kernel_size, stride);
  LS_REQUIRE(total_n >= 0 && num_heads >= 0 && batch >= 0 && max_seqlen >= 0, LS_ERR_INVALID,
             "ls_cis_mean_pool: bad sizes");
  const int M = max_seqlen / stride - 1;
  LS_REQUIRE(out_cols == (M > 0 ? M : 0), LS_ERR_INVALID,
             "ls_cis_mean_pool: out must have max_seqlen // 16 - 1 = %d columns", M > 0 ? M : 0);
  LS_REQUIRE(dtype == LS_F32 || dtype == LS_BF16 || dtype == LS_F16, LS_ERR_INVALID,
             "ls_cis_mean_pool: unknown dtype %d", dtype);
  if (M <= 0 || total_n == 0 || num_heads == 0 || batch == 0) return LS_OK;
  LS_REQUIRE(cis && cu_seqlens && out, LS_ERR_INVALID, "ls_cis_mean_pool: null pointer");
  const dim3 grid((unsigned)((M + 63) / 64), batch, num_heads);
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_cis_mean_pool_kernel<LS_BF16>, grid, dim3(256), 0, s, (const uint16_t*)cis,
                       cis_row_stride, cu_seqlens, total_n, M, (uint16_t*)out);
  else if (dtype == LS_F16)
    hipLaunchKernelGGL(ls_cis_mean_pool_kernel<LS_F16>, grid, dim3(256), 0, s, (const uint16_t*)cis,
                       cis_row_stride, cu_seqlens, total_n, M, (uint16_t*)out);
  else
    hipLaunchKernelGGL(ls_cis_mean_pool_kernel<LS_F32>, grid, dim3(256), 0, s, (const float*)cis,
                       cis_row_stride, cu_seqlens, total_n, M, (float*)out);
  return ls_check_launch("ls_cis_mean_pool_kernel");
}

// ---------------------------------------------------------------------------
// Varlen page max-pool with the forced overlay, the drop-in form:
// in [Hk][total_q][max_k] -> out [Hk][total_q][out_len].  Row t of sequence b
// has page off_bq = (t - cu_q[b] + cache_len[b]) / block_size; page p is +inf
// when p < init_blocks or off_bq - local_blocks <= p <= off_bq, else the max of
// in[h][t][j] over j in [p*s - 1, p*s + s) clipped to [0, lk) (-inf when
// empty), s = block_size / stride.  lk is the sequence's cu_k[b + 1] - cu_k[b]
// columns (LS_POOL_CLIP_SEQUENCE, at most max_k) or the row width max_k
// (LS_POOL_CLIP_ROW).  One workgroup per (row, head), threads over pages (the
// reference's grid).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void ls_page_maxpool_kernel(
    const typename LsElem<DT>::T* __restrict__ in, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_k, const int32_t* __restrict__ cache_lens, int batch,
    int64_t total_q, int64_t max_k, int64_t out_len, int s, int block_size, int init_blocks,
    int local_blocks, int clip_row, typename LsElem<DT>::T* __restrict__ out) {
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y;
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t lk = clip_row ? max_k : min((int64_t)(cu_k[b + 1] - cu_k[b]), max_k);
  const int64_t off_bq = (t - cu_q[b] + cache_lens[b]) / block_size;
  const typename LsElem<DT>::T* row = in + ((int64_t)h * total_q + t) * max_k;
  typename LsElem<DT>::T* orow = out + ((int64_t)h * total_q + t) * out_len;
  for (int64_t p = threadIdx.x; p < out_len; p += 256) {
    float v;
    if (p < init_blocks || (off_bq - local_blocks <= p && p <= off_bq)) {
      v = INFINITY;
    } else {
      v = -INFINITY;
      const int64_t lo = p * s - 1 < 0 ? 0 : p * s - 1;
      const int64_t hi = p * s + s < lk ? p * s + s : lk;
      for (int64_t j = lo; j < hi; ++j) v = fmaxf(v, LsElem<DT>::to_f(row[j]));
    }
    orow[p] = LsElem<DT>::from_f(v);
  }
}

extern "C" int ls_page_maxpool_varlen(const void* input, const int32_t* cu_seqlens_q,
                                      const int32_t* cu_seqlens_k, const int32_t* cache_lens,
                                      int32_t batch, int32_t num_heads, int64_t total_q,
                                      int64_t max_seqlen_k, int64_t out_len, int32_t local_blocks,
                                      int32_t init_blocks, int32_t block_size, int32_t stride,
                                      int32_t clip, int32_t dtype, void* out, void* stream) {
  LS_REQUIRE(batch >= 0 && num_heads >= 0 && total_q >= 0 && max_seqlen_k >= 0 && out_len >= 0,
             LS_ERR_INVALID, "ls_page_maxpool_varlen: bad sizes");
  LS_REQUIRE(block_size > 0 && stride > 0 && block_size % stride == 0, LS_ERR_INVALID,
             "ls_page_maxpool_varlen: block_size must be a positive multiple of stride");
  LS_REQUIRE(dtype == LS_F32 || dtype == LS_BF16 || dtype == LS_F16, LS_ERR_INVALID,
             "ls_page_maxpool_varlen: unknown dtype %d", dtype);
  LS_REQUIRE(clip == LS_POOL_CLIP_SEQUENCE || clip == LS_POOL_CLIP_ROW, LS_ERR_INVALID,
             "ls_page_maxpool_varlen: unknown clip %d", clip);
  LS_REQUIRE(total_q <= 0x7fffffffLL && num_heads <= 65535, LS_ERR_UNSUPPORTED,
             "ls_page_maxpool_varlen: too many rows or heads");
  if (total_q == 0 || num_heads == 0 || out_len == 0 || batch == 0) return LS_OK;
  LS_REQUIRE(input && cu_seqlens_q && cu_seqlens_k && cache_lens && out, LS_ERR_INVALID,
             "ls_page_maxpool_varlen: null pointer");
  const dim3 grid((unsigned)total_q, num_heads);
  hipStream_t s = (hipStream_t)stream;
  const int sp = block_size / stride;
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_page_maxpool_kernel<LS_BF16>, grid, dim3(256), 0, s, (const uint16_t*)input,
                       cu_seqlens_q, cu_seqlens_k, cache_lens, batch, total_q, max_seqlen_k,
                       out_len, sp, block_size, init_blocks, local_blocks, clip, (uint16_t*)out);
  else if (dtype == LS_F16)
    hipLaunchKernelGGL(ls_page_maxpool_kernel<LS_F16>, grid, dim3(256), 0, s, (const uint16_t*)input,
                       cu_seqlens_q, cu_seqlens_k, cache_lens, batch, total_q, max_seqlen_k,
                       out_len, sp, block_size, init_blocks, local_blocks, clip, (uint16_t*)out);
  else
    hipLaunchKernelGGL(ls_page_maxpool_kernel<LS_F32>, grid, dim3(256), 0, s, (const float*)input,
                       cu_seqlens_q, cu_seqlens_k, cache_lens, batch, total_q, max_seqlen_k,
                       out_len, sp, block_size, init_blocks, local_blocks, clip, (float*)out);
  return ls_check_launch("ls_page_maxpool_kernel");
}

// ---------------------------------------------------------------------------
// Fused-path CIS page scores: cpg[g][pg_off[b] + p] = max over the CIS window
// means m in [4p - 1, 4p + 4) ∩ [0, W) of sequence b, for p <= A_b / 4 (each
// mean rounded to the CIS dtype, as the drop-in pooling stores it; 0 for a
// window that does not fit in the sequence's keys and for m >= A_b).  W = A_b
// under LS_POOL_CLIP_SEQUENCE, W = A_max = max_b A_b (the width of the
// window-mean rows) under LS_POOL_CLIP_ROW.
// pg_off[b] = sum over earlier sequences of (A_b > 0 ? A_b / 4 + 1 : 0);
// pg_off[batch + 1] = A_max.
// ---------------------------------------------------------------------------
__global__ void ls_nosa_plan_kernel(const int32_t* __restrict__ cu_a, int batch,
                                    int32_t* __restrict__ pg_off) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t acc = 0, a_max = 0;
  pg_off[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int a = cu_a[b + 1] - cu_a[b];
    acc += a > 0 ? a / 4 + 1 : 0;
    a_max = a > a_max ? a : a_max;
    pg_off[b + 1] = acc;
  }
  pg_off[batch + 1] = a_max;
}

template <int CT>
__global__ __launch_bounds__(256) void ls_nosa_cis_pages_kernel(
    const typename LsElem<CT>::T* __restrict__ cis, int64_t cis_rs, const int32_t* __restrict__ cu_k,
    const int32_t* __restrict__ cu_a, const int32_t* __restrict__ pg_off, int batch,
    int clip_row, int64_t n_pages_launch, float* __restrict__ cpg, int64_t cpg_g_stride) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int g = blockIdx.y;
  if (i >= pg_off[batch] || i >= n_pages_launch) return;
  const int b = ls_find_segment(pg_off, batch, i);
  const int p = (int)(i - pg_off[b]);
  const int A = cu_a[b + 1] - cu_a[b];
  const int W = clip_row ? pg_off[batch + 1] : A;
  const int64_t start = cu_k[b], n_k = (int64_t)cu_k[b + 1] - start;
  float best = -INFINITY;
  const int lo = 4 * p - 1 < 0 ? 0 : 4 * p - 1;
  const int hi = 4 * p + 4 < W ? 4 * p + 4 : W;
  for (int m = lo; m < hi; ++m) {
    float acc = 0.f;
    if (m < A && (int64_t)m * 16 + 32 <= n_k)  // a window past the sequence end pools to 0
      for (int j = 0; j < 32; ++j)
        acc += LsElem<CT>::to_f(cis[(start + (int64_t)m * 16 + j) * cis_rs + g]);
    best = fmaxf(best, LsElem<CT>::to_f(LsElem<CT>::from_f(acc * (1.f / 32.f))));
  }
  cpg[(int64_t)g * cpg_g_stride + i] = best;
}

int ls_nosa_cis_pages_launch(const void* cis, int64_t cis_rs, int cis_dtype, const int32_t* cu_k,
                             const int32_t* cu_a, int batch, int64_t total_atoms, int G,
                             int clip_row, int32_t* pg_off, float* cpg, int64_t cpg_g_stride,
                             hipStream_t s) {
  hipLaunchKernelGGL(ls_nosa_plan_kernel, dim3(1), dim3(64), 0, s, cu_a, batch, pg_off);
  int rc = ls_check_launch("ls_nosa_plan_kernel");
  if (rc) return rc;
  const int64_t n = total_atoms / 4 + batch;  // bound on the number of CIS pages
  if (n == 0) return LS_OK;
  const dim3 grid((unsigned)((n + 255) / 256), G);
  if (cis_dtype == LS_BF16)
    hipLaunchKernelGGL(ls_nosa_cis_pages_kernel<LS_BF16>, grid, dim3(256), 0, s,
                       (const uint16_t*)cis, cis_rs, cu_k, cu_a, pg_off, batch, clip_row, n, cpg,
                       cpg_g_stride);
  else if (cis_dtype == LS_F16)
    hipLaunchKernelGGL(ls_nosa_cis_pages_kernel<LS_F16>, grid, dim3(256), 0, s,
                       (const uint16_t*)cis, cis_rs, cu_k, cu_a, pg_off, batch, clip_row, n, cpg,
                       cpg_g_stride);
  else
    hipLaunchKernelGGL(ls_nosa_cis_pages_kernel<LS_F32>, grid, dim3(256), 0, s,
                       (const float*)cis, cis_rs, cu_k, cu_a, pg_off, batch, clip_row, n, cpg,
                       cpg_g_stride);
  return ls_check_launch("ls_nosa_cis_pages_kernel");
}

// ---------------------------------------------------------------------------
// NOSA two-stage top-k.  One wave per (group, row); the row's out_len pages
// are held as keys in NS register slots of 64 lanes (page p = 64 s + lane).
//   stage 1: qk keys (forced pages +inf, pages p <= A_b / 4 from the page-score
//            scratch, others -inf); the qk_select best pages (ties to the lower
//            page) form the shortlist S;
//   stage 2: CIS keys (shortlisted pages +inf; other pages after the row's
//            q_idx -inf; forced pages +inf; others the sequence's CIS page
//            score, -inf past A_b / 4); the `take` best pages, emitted
//            ascending, ids past q_idx as -1 at the tail.
// off_bq = t_rel / block_size places the forced pages; q_idx =
// (t_rel + max_seqlen_q - len_q(b)) / block_size is aligned to the longest
// sequence (nosa.py:1175-1189).
//
// Stage 2 does not rank each row's pages again.  Outside S a row's stage-2
// key depends only on (off_bq, q_idx) and the sequence's CIS page scores, so
// the rows of one 64-row query block share it: with K0 the row-independent
// key, the stage-2 choice is S (all +inf; the forced pages are in S, since
// stage 1 puts them first and qk_select covers them) plus the first
// take - |S| pages of the block's order of K0 (key descending, page
// ascending) that are not in S.  ls_nosa_cis_rank_kernel writes the first
// take + qk_select pages of that order once per block and q_idx value, which
// covers every row (at most |S| of them are skipped).
// ---------------------------------------------------------------------------
// Threshold T such that #{key > T} < kk <= #{key >= T} (bisection over the
// key bits with ballot counts; keys of inactive lanes are 0).
// Marks the kk largest keys (ties to the lower page) in sel (bit s of the lane).
template <int NS>
__device__ __forceinline__ void ls_mark_topk(const uint32_t (&key)[NS], uint32_t T, int kk,
                                             uint32_t (&sel)[(NS + 31) / 32]) {
  int gt = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) gt += __popcll(__ballot(key[s] > T));
  const int m = kk - gt;
  int eq_before = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool eq = key[s] == T && key[s] != 0u;
    const uint64_t eq_mask = __ballot(eq);
    const bool take = key[s] > T || (eq && eq_before + ls_lanes_below(eq_mask) < m);
    if (take) sel[s >> 5] |= 1u << (s & 31);
    eq_before += __popcll(eq_mask);
  }
}

// Stage 1 from n gathered entries key << 16 | page (page order) held in NP
// slots of the wave's scratch: the kk-th key T bisected from the common bit
// prefix of lo and the row maximum (per-lane maxima m1, reduced here), then the
// kk chosen pages (key > T, then the lowest pages with key == T) set in the
// scratch, cleared first to an n_words page bitmap.  Returns |S|.
template <int NP>
__device__ __forceinline__ int ls_nosa_mark_packed(uint32_t* __restrict__ scr, int n, uint32_t lo,
                                                   uint32_t m1, int kk, int n_words, int lane) {
  uint32_t pk[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) pk[i] = i * 64 + lane < n ? scr[i * 64 + lane] : 0u;
  const uint32_t hi = ls_wave_max_u32(m1);
  uint32_t T = lo;
  const uint32_t d = lo ^ hi;
  if (d != 0u) {
    const int tb = 31 - __builtin_clz(d);
    T = lo & ~((2u << tb) - 1u);
#pragma unroll 1
    for (int bit = tb; bit >= 0; --bit) {
      const uint32_t cand = (T | (1u << bit)) << 16;
      int cnt = 0;
#pragma unroll
      for (int i = 0; i < NP; ++i) cnt += __popcll(__ballot(pk[i] >= cand));
      if (cnt >= kk) T |= 1u << bit;
    }
  }
  const uint32_t above = (T << 16) | 0xffffu;  // packed entries above T
  int gt = 0;
#pragma unroll
  for (int i = 0; i < NP; ++i) gt += __popcll(__ballot(pk[i] > above));
  const int m = kk - gt;
  // Every lane has read its entries: the scratch becomes the bitmap.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int i = lane; i < n_words; i += 64) scr[i] = 0u;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int n_sel = 0, eq_before = 0;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const bool valid = i * 64 + lane < n;
    const bool eq = valid && (pk[i] >> 16) == T;
    const uint64_t eq_mask = __ballot(eq);
    const int eq_rank = eq_before + ls_lanes_below(eq_mask);
    const bool sel = valid && (pk[i] > above || (eq && eq_rank < m));
    if (sel) {
      const uint32_t page = pk[i] & 0xffffu;
      atomicOr(&scr[page >> 5], 1u << (page & 31));
    }
    n_sel += __popcll(__ballot(sel));
    eq_before += __popcll(eq_mask);
  }
  return n_sel;
}

// Stage 1 of a row of bf16 page scores through a fast path: the shortlist S =
// every forced page plus the kq - F best other pages (F forced pages), valid
// when no loaded score is NaN or +inf (then nothing ties with the forced
// pages' +inf) and the kq-th largest of the lanes' two largest scores, lo, is
// positive.  The row is read through a buffer resource bounded at the scored
// columns (reads past them return +0, which a positive lo leaves out), scores
// are compared as float32, and the scores >= lo are gathered as raw bits << 16
// | page in page order (at most 256).  lo is a lower bound of the (kq - F)-th
// best non-forced score: of the kq largest among the lanes' top two (values of
// distinct pages), at most F are forced pages.  The gathered non-forced
// entries then hold every non-forced score >= lo; their (kq - F)-th largest
// order key T is bisected, and the pages above T plus the lowest pages at T
// are marked with the forced ones in the page bitmap that replaces the
// scratch.  Returns |S| (= kq), or -1 (nothing marked) when the row needs the
// general path.
template <int NP>
__device__ __forceinline__ int ls_nosa_stage1_finish(uint32_t* __restrict__ scr, int n,
                                                     uint32_t lo, int kq, int k2, int lo_end,
                                                     int la, int lb, int n_words, int lane) {
  uint32_t pk[NP];
  uint32_t hk = 0u;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const bool valid = i * 64 + lane < n;
    const uint32_t e = valid ? scr[i * 64 + lane] : 0u;
    const int page = (int)(e & 0xffffu);
    const bool forced = page < lo_end || (page >= la && page <= lb);
    // Positive bf16 scores: bf16 | 0x8000 is the order key.
    pk[i] = valid && !forced ? (e | 0x80000000u) : 0u;
    hk = max(hk, pk[i] >> 16);
  }
  const uint32_t hi = ls_wave_max_u32(hk);
  uint32_t T = lo;
  const uint32_t d = lo ^ hi;
  if (d != 0u) {
    const int tb = 31 - __builtin_clz(d);
    T = lo & ~((2u << tb) - 1u);
#pragma unroll 1
    for (int bit = tb; bit >= 0; --bit) {
      const uint32_t cand = (T | (1u << bit)) << 16;
      int cnt = 0;
#pragma unroll
      for (int i = 0; i < NP; ++i) cnt += __popcll(__ballot(pk[i] >= cand));
      if (cnt >= k2) T |= 1u << bit;
    }
  }
  const uint32_t above = (T << 16) | 0xffffu;
  int gt = 0;
#pragma unroll
  for (int i = 0; i < NP; ++i) gt += __popcll(__ballot(pk[i] > above));
  const int m = k2 - gt;
  // Every lane has read its entries: the scratch becomes the bitmap.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int i = lane; i < n_words; i += 64) scr[i] = 0u;
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  int eq_before = 0;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const bool eq = pk[i] != 0u && (pk[i] >> 16) == T;
    const uint64_t eq_mask = __ballot(eq);
    const int eq_rank = eq_before + ls_lanes_below(eq_mask);
    if (pk[i] > above || (eq && eq_rank < m)) {
      const uint32_t page = pk[i] & 0xffffu;
      atomicOr(&scr[page >> 5], 1u << (page & 31));
    }
    eq_before += __popcll(eq_mask);
  }
  const int nf = kq - k2;
  for (int i = lane; i < nf; i += 64) {
    const int page = i < lo_end ? i : la + (i - lo_end);
    atomicOr(&scr[page >> 5], 1u << (page & 31));
  }
  return kq;
}

template <int NS>
__device__ __forceinline__ int ls_nosa_stage1_bf16(const uint16_t* __restrict__ row, int n_scored,
                                                   int out_len, int off_bq, int init_blocks,
                                                   int local_blocks, int kq, int n_words,
                                                   int lane, uint32_t* __restrict__ scr) {
  if (kq < 1 || kq > 128) return -1;
  const int lo_end = min(init_blocks, out_len);
  const int la = max(off_bq - local_blocks, lo_end), lb = min(off_bq, out_len - 1);
  const int nf = lo_end + max(0, lb - la + 1);  // forced pages
  if (nf >= kq) return -1;
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)row, (short)0, n_scored * 2, 0x00020000);
  uint32_t f[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    // The whole byte offset in a lane register (none of it in the scalar
    // offset, which the hardware range check leaves out).
    uint32_t off = (uint32_t)(lane * 2 + 128 * s);
    asm("" : "+v"(off));
    f[s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0) << 16;
  }
  float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float x = __uint_as_float(f[s]);
    m2 = __builtin_amdgcn_fmed3f(m1, m2, x);
    m1 = __builtin_elementwise_maximum(m1, x);
  }
  if (__ballot(__builtin_isnan(m1) || m1 == INFINITY) != 0ull) return -1;
  const uint32_t k1 = ls_order_key16((uint16_t)(__float_as_uint(m1) >> 16));
  const uint32_t kb = ls_order_key16((uint16_t)(__float_as_uint(m2) >> 16));
  const uint32_t kmin = ls_wave_min_u32(kb), kmax = ls_wave_max_u32(k1);
  const uint32_t dk = kmin ^ kmax;
  const int top = dk ? 31 - __builtin_clz(dk) : -1;
  uint32_t lo = top >= 0 ? kmin & ~((2u << top) - 1u) : kmin;
#pragma unroll
  for (int bit = 15; bit >= 0; --bit) {
    if (bit <= top) {
      const uint32_t cand = lo | (1u << bit);
      const int cnt = __popcll(__ballot(k1 >= cand)) + __popcll(__ballot(kb >= cand));
      lo = cnt >= kq ? cand : lo;
    }
  }
  if (lo <= 0x8000u) return -1;  // the bound must be a positive score
  const float lo_f = __uint_as_float((lo & 0x7fffu) << 16);
  int n = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool sv = __uint_as_float(f[s]) >= lo_f;
    const uint64_t mk = __ballot(sv);
    int pos = (int)__builtin_amdgcn_mbcnt_hi(
        (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, (uint32_t)n));
    asm("" : "+v"(pos));  // formed in every lane: the store below needs no branch
    scr[sv ? min(pos, 255) : 256 + lane] = f[s] | (uint32_t)(s * 64 + lane);
    n += __popcll(mk);
  }
  if (n > 256) return -1;
  const int k2 = kq - nf;
  if (n <= 64) return ls_nosa_stage1_finish<1>(scr, n, lo, kq, k2, lo_end, la, lb, n_words, lane);
  if (n <= 128) return ls_nosa_stage1_finish<2>(scr, n, lo, kq, k2, lo_end, la, lb, n_words, lane);
  return ls_nosa_stage1_finish<4>(scr, n, lo, kq, k2, lo_end, la, lb, n_words, lane);
}

// Key widths: stage 1 uses 16-bit keys for 16-bit page scores (KEY32 off);
// stage 2 uses the top 16 bits of the float32 keys when the CIS page scores
// are bf16 values (CIS32 off: their low 16 bits are zero), so each bisection
// runs over 16 bits instead of 32.
template <int NS, bool KEY32>
__device__ __forceinline__ void ls_nosa_topk_row(
    const void* __restrict__ P, int64_t prow, int n_scored, int out_len, int off_bq, int q_idx,
    int init_blocks, int local_blocks, int qk_select, int take, uint32_t pinf1, uint32_t ninf1,
    int lane, int32_t* __restrict__ orow, uint32_t* __restrict__ scr,
    const int32_t* __restrict__ order, int n_order, int bf16) {
  constexpr int NW = (NS + 31) / 32;
  // Stage 1 ends with the shortlist S as a page bitmap in the wave's scratch
  // (n_s = |S|); stage 2 then adds the block order's first take - |S| pages
  // outside S to it.
  const int n_words = (out_len + 31) >> 5;
  int n_s = -1;
  if constexpr (!KEY32 && NS > 4)
    if (bf16)
      n_s = ls_nosa_stage1_bf16<NS>((const uint16_t*)P + prow, n_scored, out_len, off_bq,
                                    init_blocks, local_blocks, qk_select, n_words, lane, scr);
  if (n_s < 0) {
  // Every +inf (forced or shortlisted) and every -inf is one key, so ties among
  // them go to the lower page as in a stable sort.  Stage 1 keys come from the
  // page-score dtype (pinf1 / ninf1).
  uint32_t key[NS];
  // Stage 1 keys.
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int p = s * 64 + lane;
    uint32_t raw = 0u;
    if (p < n_scored) {
      if constexpr (KEY32) raw = ((const uint32_t*)P)[prow + p];
      else raw = ((const uint16_t*)P)[prow + p];
    }
    key[s] = raw;
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int p = s * 64 + lane;
    uint32_t k;
    if (p >= out_len) k = 0u;
    else if (p < init_blocks || (off_bq - local_blocks <= p && p <= off_bq)) k = pinf1;
    else if (p < n_scored) k = KEY32 ? ls_order_key32(key[s]) : ls_order_key16((uint16_t)key[s]);
    else k = ninf1;
    key[s] = k;
  }
  if constexpr (!KEY32 && NS > 4) {
    // Long rows: the keys >= lo (lo = the qk_select-th largest of the lanes'
    // two largest keys) are gathered as key << 16 | page in page order, and S
    // is marked from them (ls_nosa_mark_packed); otherwise the generic path.
    if (qk_select >= 1 && qk_select <= 128) {
      uint32_t m1 = 0u, m2 = 0u;
#pragma unroll
      for (int s = 0; s < NS; ++s) {
        m2 = max(m2, min(m1, key[s]));
        m1 = max(m1, key[s]);
      }
      const uint32_t mm[2] = {m1, m2};
      const uint32_t lo = ls_kth_bisect<2>(mm, qk_select, 0u, 15);
      int n = 0;
      if (lo != 0u) {
#pragma unroll
        for (int s = 0; s < NS; ++s) {
          if (n <= 256) {
            const bool sv = key[s] >= lo;
            const uint64_t mk = __ballot(sv);
            const int pos = (int)__builtin_amdgcn_mbcnt_hi(
                (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, (uint32_t)n));
            if (sv) scr[pos] = (key[s] << 16) | (uint32_t)(s * 64 + lane);
            n += __popcll(mk);
          }
        }
        if (n <= 64) n_s = ls_nosa_mark_packed<1>(scr, n, lo, m1, qk_select, n_words, lane);
        else if (n <= 128) n_s = ls_nosa_mark_packed<2>(scr, n, lo, m1, qk_select, n_words, lane);
        else if (n <= 256) n_s = ls_nosa_mark_packed<4>(scr, n, lo, m1, qk_select, n_words, lane);
      }
    }
  }
  if (n_s < 0) {
    uint32_t shortlist[NW];
#pragma unroll
    for (int i = 0; i < NW; ++i) shortlist[i] = 0u;
    ls_mark_topk<NS>(key, ls_kth_key_row<NS, KEY32 ? 32 : 16>(key, qk_select, scr, lane),
                     qk_select, shortlist);
    for (int i = lane; i < n_words; i += 64) scr[i] = 0u;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    n_s = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const uint64_t m = __ballot((shortlist[s >> 5] >> (s & 31)) & 1u);
      if (lane < 2) scr[2 * s + lane] = lane ? (uint32_t)(m >> 32) : (uint32_t)m;
      n_s += __popcll(m);
    }
  }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  if (n_s > take) {
    // More shortlisted pages than the budget (topk below init + local +
    // select): all are +inf, so the lowest `take` of them are chosen.
    int before = 0;
    for (int w0 = 0; w0 < n_words; w0 += 64) {
      const int wi = w0 + lane;
      uint32_t word = wi < n_words ? scr[wi] : 0u;
      const int cnt = __popc(word);
      int x = cnt;
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const int y = __shfl_up(x, d, LS_WAVE);
        if (lane >= d) x += y;
      }
      const int pre = before + x - cnt;
      if (pre >= take) {
        word = 0u;
      } else if (pre + cnt > take) {  // keep the word's lowest take - pre pages
        uint32_t kept = 0u, wcopy = word;
        for (int c = 0; c < take - pre; ++c) {
          const uint32_t low = wcopy & (0u - wcopy);
          kept |= low;
          wcopy ^= low;
        }
        word = kept;
      }
      if (wi < n_words) scr[wi] = word;
      before += __shfl(x, 63, LS_WAVE);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
  const int need = take - n_s;
  int picked = 0;
  for (int i0 = 0; i0 < n_order && picked < need; i0 += 64) {
    const int i = i0 + lane;
    const int page = i < n_order ? order[i] : -1;
    const bool avail = page >= 0 && !((scr[page >> 5] >> (page & 31)) & 1u);
    const uint64_t m = __ballot(avail);
    if (avail && picked + ls_lanes_below(m) < need) atomicOr(&scr[page >> 5], 1u << (page & 31));
    picked += __popcll(m);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  // Emission: chosen pages <= q_idx in ascending order, then -1.
  int out_pos = 0;
  for (int w0 = 0; w0 < n_words; w0 += 64) {
    const int wi = w0 + lane;
    uint32_t word = wi < n_words ? scr[wi] : 0u;
    if (32 * wi > q_idx) word = 0u;
    else if (32 * wi + 31 > q_idx) word &= (2u << (q_idx & 31)) - 1u;
    const int cnt = __popc(word);
    int x = cnt;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(x, d, LS_WAVE);
      if (lane >= d) x += y;
    }
    int pos = out_pos + x - cnt;
    while (word) {
      const int bit = __builtin_ctz(word);
      word &= word - 1u;
      if (pos < take) orow[pos] = 32 * wi + bit;  // at most take by construction
      ++pos;
    }
    out_pos += __shfl(x, 63, LS_WAVE);
  }
  for (int i = out_pos + lane; i < take; i += 64) orow[i] = -1;
}

// The block's stage-2 order.  One wave per (64-row query block, group, q_idx
// variant): the rows of block j of sequence b have off_bq = j and q_idx = qa
// or qa + 1, qa = (64 j + max_seqlen_q - len_q(b)) / 64.  Keys K0 of pages
// p < out_len: -inf after q_idx, +inf forced, -inf without a CIS page score
// (p > A_b / 4), else the float32 CIS page score; the n_order best (ties to
// the lower page) are written best first to order[((g * n_blk + blk) * 2 + v)
// * n_order + i] (entries past out_len pages stay -1).  Under
// LS_POOL_CLIP_ROW the pages A_b / 4 < p <= A_max / 4 pool only padding
// windows and score 0 (pages [n_scored, n_zero)).
template <int NS>
__device__ __forceinline__ void ls_nosa_rank_block(const float* __restrict__ cpg_seq, int n_scored,
                                                   int n_zero, int out_len, int off_bq, int q_idx,
                                                   int init_blocks, int local_blocks, int n_order,
                                                   int lane, int32_t* __restrict__ out,
                                                   uint32_t* __restrict__ scr,
                                                   uint32_t* __restrict__ s_key,
                                                   int32_t* __restrict__ s_page) {
  constexpr int NW = (NS + 31) / 32;
  const uint32_t pinf = ls_order_key32(0x7f800000u), ninf = ls_order_key32(0xff800000u);
  const uint32_t zero = ls_order_key32(0u);
  uint32_t key[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int p = s * 64 + lane;
    uint32_t k;
    if (p >= out_len) k = 0u;
    else if (p > q_idx) k = ninf;
    else if (p < init_blocks || (off_bq - local_blocks <= p && p <= off_bq)) k = pinf;
    else if (p >= n_zero) k = ninf;
    else if (p >= n_scored) k = zero;
    else k = ls_order_key32(__builtin_bit_cast(uint32_t, cpg_seq[p]));
    key[s] = k;
  }
  const int kk = n_order < out_len ? n_order : out_len;
  uint32_t sel[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) sel[i] = 0u;
  ls_mark_topk<NS>(key, ls_kth_key_row<NS, 32>(key, kk, scr, lane), kk, sel);
  // The chosen (key, page) pairs in page order, then each one's rank.
  int n = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool on = (sel[s >> 5] >> (s & 31)) & 1u;
    const uint64_t m = __ballot(on);
    if (on) {
      const int pos = n + ls_lanes_below(m);
      s_key[pos] = key[s];
      s_page[pos] = s * 64 + lane;
    }
    n += __popcll(m);
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  for (int i = lane; i < n; i += 64) {
    const uint32_t ki = s_key[i];
    const int pi = s_page[i];
    int rank = 0;
    for (int j = 0; j < n; ++j) {
      const uint32_t kj = s_key[j];
      rank += (kj > ki || (kj == ki && s_page[j] < pi)) ? 1 : 0;
    }
    out[rank] = pi;
  }
  for (int i = n + lane; i < n_order; i += 64) out[i] = -1;
}

#define LS_NOSA_MAX_ORDER LS_NOSA_ORDER_STRIDE  // bound on take + qk_select

template <int KPL>
__global__ __launch_bounds__(64) void ls_nosa_cis_rank_kernel(
    const float* __restrict__ cpg, int64_t cpg_g_stride, const int32_t* __restrict__ pg_off,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_a,
    const int32_t* __restrict__ blk_off, int batch, int64_t n_blk, int max_seqlen_q, int out_len,
    int init_blocks, int local_blocks, int block_size, int clip_row, int n_order,
    int32_t* __restrict__ order) {
  __shared__ uint32_t s_scr[256];
  __shared__ uint32_t s_key[LS_NOSA_MAX_ORDER];
  __shared__ int32_t s_page[LS_NOSA_MAX_ORDER];
  const int64_t blk = blockIdx.x;
  const int g = blockIdx.y, v = blockIdx.z;
  const int lane = threadIdx.x;
  if (blk >= blk_off[batch]) return;
  const int b = ls_find_segment(blk_off, batch, blk);
  const int j = (int)(blk - blk_off[b]);
  const int lq = cu_q[b + 1] - cu_q[b];
  const int qa = (block_size * j + max_seqlen_q - lq) / block_size;
  const int t_last = min(block_size * j + block_size - 1, lq - 1);
  int32_t* out = order + (((int64_t)g * n_blk + blk) * 2 + v) * n_order;
  if (v == 1 && (t_last + max_seqlen_q - lq) / block_size == qa) return;  // one q_idx only
  const int A = cu_a[b + 1] - cu_a[b];
  const int n_scored = min(A > 0 ? A / 4 + 1 : 0, out_len);
  const int a_max = pg_off[batch + 1];
  const int n_zero = clip_row ? min(a_max > 0 ? a_max / 4 + 1 : 0, out_len) : n_scored;
  const float* cpg_seq = cpg + (int64_t)g * cpg_g_stride + pg_off[b];
  const int n_slots = (out_len + 63) >> 6;
#define LS_RANK(NSV) ls_nosa_rank_block<NSV>(cpg_seq, n_scored, n_zero, out_len, j, qa + v,     \
                                             init_blocks, local_blocks, n_order, lane, out,     \
                                             s_scr, s_key, s_page)
  if (n_slots <= 1) return LS_RANK(1);
  if (n_slots <= 4 || KPL <= 4) return LS_RANK(KPL < 4 ? KPL : 4);
  if (n_slots <= 16 || KPL <= 16) return LS_RANK(KPL < 16 ? KPL : 16);
  if (n_slots <= 32 || KPL <= 32) return LS_RANK(KPL < 32 ? KPL : 32);
  if (n_slots <= 64 || KPL <= 64) return LS_RANK(KPL < 64 ? KPL : 64);
  return LS_RANK(KPL);
#undef LS_RANK
}

template <int KPL, bool KEY32>
__global__ __launch_bounds__(256) void ls_nosa_topk_kernel(
    const void* __restrict__ P, int64_t p_stride, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_a, const int32_t* __restrict__ blk_off, int batch,
    int64_t total_q, int G, int max_seqlen_q, int out_len, int init_blocks, int local_blocks,
    int qk_select, int take, int block_size, uint32_t pinf1, uint32_t ninf1,
    const int32_t* __restrict__ order, int64_t n_blk, int n_order, int bf16,
    int32_t* __restrict__ topk_idx) {
  __shared__ uint32_t s_scr[4][320];  // per-wave k-th key scratch, then the chosen-page bitmap
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n_rows = (int64_t)G * total_q;
  const int64_t row = (int64_t)blockIdx.x * 4 + wv;
  if (row >= n_rows) return;
  uint32_t* const scr = s_scr[wv];
  const int g = (int)(row / total_q);
  const int64_t t = row - (int64_t)g * total_q;
  const int b = ls_find_segment(cu_q, batch, t);
  const int t_rel = (int)(t - cu_q[b]);
  const int lq = cu_q[b + 1] - cu_q[b];
  const int A = cu_a[b + 1] - cu_a[b];
  int n_scored = A > 0 ? A / 4 + 1 : 0;
  if (n_scored > out_len) n_scored = out_len;
  const int off_bq = t_rel / block_size;
  const int q_idx = (t_rel + max_seqlen_q - lq) / block_size;
  const int qa = (block_size * off_bq + max_seqlen_q - lq) / block_size;
  const int32_t* ord = order + (((int64_t)g * n_blk + blk_off[b] + off_bq) * 2 + (q_idx - qa)) * n_order;
  int32_t* orow = topk_idx + row * take;
  const int64_t prow = row * p_stride;
  const int n_slots = (out_len + 63) >> 6;
  const int n_ord = n_order < out_len ? n_order : out_len;
#define LS_ROW(NSV) ls_nosa_topk_row<NSV, KEY32>(P, prow, n_scored, out_len, off_bq, q_idx, \
    init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, ord, n_ord, bf16)
  if (n_slots <= 1) return LS_ROW(1);
  if (n_slots <= 2) return LS_ROW(2);
  if (n_slots <= 4 || KPL <= 4) return LS_ROW(KPL < 4 ? KPL : 4);
  if (n_slots <= 8 || KPL <= 8) return LS_ROW(KPL < 8 ? KPL : 8);
  if (n_slots <= 16 || KPL <= 16) return LS_ROW(KPL < 16 ? KPL : 16);
  if (n_slots <= 32 || KPL <= 32) return LS_ROW(KPL < 32 ? KPL : 32);
  if (n_slots <= 64 || KPL <= 64) return LS_ROW(KPL < 64 ? KPL : 64);
  return LS_ROW(KPL);
#undef LS_ROW
}

size_t ls_nosa_order_bytes(int64_t n_blk, int G, int n_order) {
  return (size_t)G * n_blk * 2 * n_order * 4;
}

template <bool KEY32>
static int launch_nosa_topk_k(int out_len, hipStream_t s, const void* P, int64_t ps,
                              const float* cpg, int64_t cs, const int32_t* pg_off,
                              const int32_t* cu_q, const int32_t* cu_a, const int32_t* blk_off,
                              int64_t n_blk, int batch, int64_t total_q, int G, int max_q,
                              int init, int local, int qk_select, int take, int bs,
                              int clip_row, uint32_t pinf1, uint32_t ninf1, int bf16,
                              int32_t* order, int32_t* out) {
  const int n_order = take + qk_select;
  const dim3 rgrid((unsigned)n_blk, G, 2);
  const dim3 grid((unsigned)(((int64_t)G * total_q + 3) / 4));
#define LS_NOSA_TOPK(K)                                                                          \
  do {                                                                                         \
    hipLaunchKernelGGL((ls_nosa_cis_rank_kernel<K>), rgrid, dim3(64), 0, s, cpg, cs, pg_off,   \
                       cu_q, cu_a, blk_off, batch, n_blk, max_q, out_len, init, local, bs,    \
                       clip_row, n_order, order);                                              \
    if (int rc = ls_check_launch("ls_nosa_cis_rank_kernel")) return rc;                       \
    hipLaunchKernelGGL((ls_nosa_topk_kernel<K, KEY32>), grid, dim3(256), 0, s, P, ps, cu_q,   \
                       cu_a, blk_off, batch, total_q, G, max_q, out_len, init, local,         \
                       qk_select, take, bs, pinf1, ninf1, order, n_blk, n_order, bf16, out);  \
  } while (0)
  if (out_len <= 256) LS_NOSA_TOPK(4);
  else if (out_len <= 1024) LS_NOSA_TOPK(16);
  else if (out_len <= 2048) LS_NOSA_TOPK(32);
  else if (out_len <= 4096) LS_NOSA_TOPK(64);
  else if (out_len <= 8192) LS_NOSA_TOPK(128);
  else return ls_fail(LS_ERR_UNSUPPORTED, "NOSA selection: at most 8192 pages per row (got %d)", out_len);
#undef LS_NOSA_TOPK
  return ls_check_launch("ls_nosa_topk_kernel");
}

int ls_nosa_topk_launch(int p_dtype, int out_len, const void* P, int64_t p_stride, const float* cpg,
                        int64_t cpg_g_stride, const int32_t* pg_off, const int32_t* cu_q,
                        const int32_t* cu_a, const int32_t* blk_off, int64_t n_blk, int batch,
                        int64_t total_q, int G, int max_seqlen_q, int init_blocks,
                        int local_blocks, int qk_select, int take, int block_size,
                        int clip_row, int32_t* order, int32_t* topk_idx, hipStream_t s) {
  if (total_q == 0 || G == 0 || take == 0) return LS_OK;
  if (take + qk_select > LS_NOSA_MAX_ORDER)
    return ls_fail(LS_ERR_UNSUPPORTED, "NOSA selection: topk + init + local + select blocks "
                   "above %d", LS_NOSA_MAX_ORDER);
#define LS_NOSA_TOPK_ARGS                                                                      \
  out_len, s, P, p_stride, cpg, cpg_g_stride, pg_off, cu_q, cu_a, blk_off, n_blk, batch,     \
      total_q, G, max_seqlen_q, init_blocks, local_blocks, qk_select, take, block_size,       \
      clip_row, pinf, ninf, p_dtype == LS_BF16 ? 1 : 0, order, topk_idx
  if (p_dtype == LS_F32) {
    const uint32_t pinf = ls_order_key32(0x7f800000u), ninf = ls_order_key32(0xff800000u);
    return launch_nosa_topk_k<true>(LS_NOSA_TOPK_ARGS);
  }
  const uint32_t pinf = ls_order_key16(p_dtype == LS_BF16 ? 0x7f80u : 0x7c00u);
  const uint32_t ninf = ls_order_key16(p_dtype == LS_BF16 ? 0xff80u : 0xfc00u);
  return launch_nosa_topk_k<false>(LS_NOSA_TOPK_ARGS);
#undef LS_NOSA_TOPK_ARGS
}
