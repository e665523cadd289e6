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
// in[h][t][j] over j in [p*s - 1, p*s + s) clipped to the sequence's
// cu_k[b + 1] - cu_k[b] columns (-inf when empty), s = block_size / stride.
// One workgroup per (row, head), threads over pages (the reference's grid).
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void ls_page_maxpool_kernel(
    const typename LsElem<DT>::T* __restrict__ in, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_k, const int32_t* __restrict__ cache_lens, int batch,
    int64_t total_q, int64_t max_k, int64_t out_len, int s, int block_size, int init_blocks,
    int local_blocks, typename LsElem<DT>::T* __restrict__ out) {
  const int64_t t = blockIdx.x;
  const int h = blockIdx.y;
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t lk = min((int64_t)(cu_k[b + 1] - cu_k[b]), max_k);
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
                                      int32_t dtype, void* out, void* stream) {
  LS_REQUIRE(batch >= 0 && num_heads >= 0 && total_q >= 0 && max_seqlen_k >= 0 && out_len >= 0,
             LS_ERR_INVALID, "ls_page_maxpool_varlen: bad sizes");
  LS_REQUIRE(block_size > 0 && stride > 0 && block_size % stride == 0, LS_ERR_INVALID,
             "ls_page_maxpool_varlen: block_size must be a positive multiple of stride");
  LS_REQUIRE(dtype == LS_F32 || dtype == LS_BF16 || dtype == LS_F16, LS_ERR_INVALID,
             "ls_page_maxpool_varlen: unknown dtype %d", dtype);
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
                       out_len, sp, block_size, init_blocks, local_blocks, (uint16_t*)out);
  else if (dtype == LS_F16)
    hipLaunchKernelGGL(ls_page_maxpool_kernel<LS_F16>, grid, dim3(256), 0, s, (const uint16_t*)input,
                       cu_seqlens_q, cu_seqlens_k, cache_lens, batch, total_q, max_seqlen_k,
                       out_len, sp, block_size, init_blocks, local_blocks, (uint16_t*)out);
  else
    hipLaunchKernelGGL(ls_page_maxpool_kernel<LS_F32>, grid, dim3(256), 0, s, (const float*)input,
                       cu_seqlens_q, cu_seqlens_k, cache_lens, batch, total_q, max_seqlen_k,
                       out_len, sp, block_size, init_blocks, local_blocks, (float*)out);
  return ls_check_launch("ls_page_maxpool_kernel");
}

// ---------------------------------------------------------------------------
// Fused-path CIS page scores: cpg[g][pg_off[b] + p] = max over the CIS window
// means m in [4p - 1, 4p + 4) ∩ [0, A_b) of sequence b (each mean rounded to
// the CIS dtype, as the drop-in pooling stores it; 0 for a window that does
// not fit in the sequence's keys), for p <= A_b / 4.
// pg_off[b] = sum over earlier sequences of (A_b > 0 ? A_b / 4 + 1 : 0).
// ---------------------------------------------------------------------------
__global__ void ls_nosa_plan_kernel(const int32_t* __restrict__ cu_a, int batch,
                                    int32_t* __restrict__ pg_off) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t acc = 0;
  pg_off[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int a = cu_a[b + 1] - cu_a[b];
    acc += a > 0 ? a / 4 + 1 : 0;
    pg_off[b + 1] = acc;
  }
}

template <int CT>
__global__ __launch_bounds__(256) void ls_nosa_cis_pages_kernel(
    const typename LsElem<CT>::T* __restrict__ cis, int64_t cis_rs, const int32_t* __restrict__ cu_k,
    const int32_t* __restrict__ cu_a, const int32_t* __restrict__ pg_off, int batch,
    int64_t n_pages_launch, float* __restrict__ cpg, int64_t cpg_g_stride) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int g = blockIdx.y;
  if (i >= pg_off[batch] || i >= n_pages_launch) return;
  const int b = ls_find_segment(pg_off, batch, i);
  const int p = (int)(i - pg_off[b]);
  const int A = cu_a[b + 1] - cu_a[b];
  const int64_t start = cu_k[b], n_k = (int64_t)cu_k[b + 1] - start;
  float best = -INFINITY;
  const int lo = 4 * p - 1 < 0 ? 0 : 4 * p - 1;
  const int hi = 4 * p + 4 < A ? 4 * p + 4 : A;
  for (int m = lo; m < hi; ++m) {
    float acc = 0.f;
    if ((int64_t)m * 16 + 32 <= n_k)  // a window past the sequence end pools to 0
      for (int j = 0; j < 32; ++j)
        acc += LsElem<CT>::to_f(cis[(start + (int64_t)m * 16 + j) * cis_rs + g]);
    best = fmaxf(best, LsElem<CT>::to_f(LsElem<CT>::from_f(acc * (1.f / 32.f))));
  }
  cpg[(int64_t)g * cpg_g_stride + i] = best;
}

int ls_nosa_cis_pages_launch(const void* cis, int64_t cis_rs, int cis_dtype, const int32_t* cu_k,
                             const int32_t* cu_a, int batch, int64_t total_atoms, int G,
                             int32_t* pg_off, float* cpg, int64_t cpg_g_stride, hipStream_t s) {
  hipLaunchKernelGGL(ls_nosa_plan_kernel, dim3(1), dim3(64), 0, s, cu_a, batch, pg_off);
  int rc = ls_check_launch("ls_nosa_plan_kernel");
  if (rc) return rc;
  const int64_t n = total_atoms / 4 + batch;  // bound on the number of CIS pages
  if (n == 0) return LS_OK;
  const dim3 grid((unsigned)((n + 255) / 256), G);
  if (cis_dtype == LS_BF16)
    hipLaunchKernelGGL(ls_nosa_cis_pages_kernel<LS_BF16>, grid, dim3(256), 0, s,
                       (const uint16_t*)cis, cis_rs, cu_k, cu_a, pg_off, batch, n, cpg, cpg_g_stride);
  else if (cis_dtype == LS_F16)
    hipLaunchKernelGGL(ls_nosa_cis_pages_kernel<LS_F16>, grid, dim3(256), 0, s,
                       (const uint16_t*)cis, cis_rs, cu_k, cu_a, pg_off, batch, n, cpg, cpg_g_stride);
  else
    hipLaunchKernelGGL(ls_nosa_cis_pages_kernel<LS_F32>, grid, dim3(256), 0, s,
                       (const float*)cis, cis_rs, cu_k, cu_a, pg_off, batch, n, cpg, cpg_g_stride);
  return ls_check_launch("ls_nosa_cis_pages_kernel");
}

// ---------------------------------------------------------------------------
// NOSA two-stage top-k.  One wave per (group, row); the row's out_len pages
// are held as keys in NS register slots of 64 lanes (page p = 64 s + lane).
//   stage 1: qk keys (forced pages +inf, pages p <= A_b / 4 from the page-score
//            scratch, others -inf); the qk_select best pages (ties to the lower
//            page) form the shortlist;
//   stage 2: CIS keys (shortlisted pages +inf; other pages after the row's
//            q_idx -inf; forced pages +inf; others the sequence's CIS page
//            score, -inf past A_b / 4); the `take` best pages, emitted
//            ascending, ids past q_idx as -1 at the tail.
// off_bq = t_rel / block_size places the forced pages; q_idx =
// (t_rel + max_seqlen_q - len_q(b)) / block_size is aligned to the longest
// sequence (nosa.py:1175-1189).
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

// Key widths: stage 1 uses 16-bit keys for 16-bit page scores (KEY32 off);
// stage 2 uses the top 16 bits of the float32 keys when the CIS page scores
// are bf16 values (CIS32 off: their low 16 bits are zero), so each bisection
// runs over 16 bits instead of 32.
template <int NS, bool KEY32, bool CIS32>
__device__ __forceinline__ void ls_nosa_topk_row(
    const void* __restrict__ P, int64_t prow, const float* __restrict__ cpg_seq, int n_scored,
    int out_len, int off_bq, int q_idx, int init_blocks, int local_blocks, int qk_select,
    int take, uint32_t pinf1, uint32_t ninf1, int lane, int32_t* __restrict__ orow,
    uint32_t* __restrict__ scr, const float* __restrict__ cpg_lds) {
  constexpr int NW = (NS + 31) / 32;
  // Every +inf (forced or shortlisted) and every -inf is one key, so ties among
  // them go to the lower page as in a stable sort.  Stage 1 keys come from the
  // page-score dtype (pinf1 / ninf1), stage 2 keys from float32.
  constexpr int SH2 = CIS32 ? 0 : 16;
  const uint32_t pinf2 = ls_order_key32(0x7f800000u) >> SH2;
  const uint32_t ninf2 = ls_order_key32(0xff800000u) >> SH2;
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
  uint32_t shortlist[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) shortlist[i] = 0u;
  ls_mark_topk<NS>(key, ls_kth_key_row<NS, KEY32 ? 32 : 16>(key, qk_select, scr, lane), qk_select,
                   shortlist);
  // Stage 2 keys (the CIS page scores from the workgroup's LDS copy when its
  // rows share a sequence and group).
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int p = s * 64 + lane;
    const float cis_lds = cpg_lds ? cpg_lds[p] : 0.f;
    uint32_t k;
    // The reference's order: pooled CIS scores with the forced overlay, then
    // pages after q_idx -inf, then the shortlist +inf.
    if (p >= out_len) k = 0u;
    else if ((shortlist[s >> 5] >> (s & 31)) & 1u) k = pinf2;
    else if (p > q_idx) k = ninf2;
    else if (p < init_blocks || (off_bq - local_blocks <= p && p <= off_bq)) k = pinf2;
    else if (p >= n_scored) k = ninf2;
    else k = ls_order_key32(__builtin_bit_cast(uint32_t, cpg_lds ? cis_lds : cpg_seq[p])) >> SH2;
    key[s] = k;
  }
  uint32_t chosen[NW];
#pragma unroll
  for (int i = 0; i < NW; ++i) chosen[i] = 0u;
  ls_mark_topk<NS>(key, ls_kth_key_row<NS, CIS32 ? 32 : 16>(key, take, scr, lane), take, chosen);
  // Emission: chosen pages <= q_idx in ascending order, then -1.
  int out_pos = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int p = s * 64 + lane;
    const bool emit = ((chosen[s >> 5] >> (s & 31)) & 1u) && p <= q_idx;
    const uint64_t m = __ballot(emit);
    const int pos = out_pos + ls_lanes_below(m);
    if (emit && pos < take) orow[pos] = p;  // at most take by construction
    out_pos += __popcll(m);
  }
  for (int i = out_pos + lane; i < take; i += 64) orow[i] = -1;
}

template <int KPL, bool KEY32, bool CIS32>
__global__ __launch_bounds__(256) void ls_nosa_topk_kernel(
    const void* __restrict__ P, int64_t p_stride, const float* __restrict__ cpg, int64_t cpg_g_stride,
    const int32_t* __restrict__ pg_off, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_a, int batch, int64_t total_q, int G, int max_seqlen_q,
    int out_len, int init_blocks, int local_blocks, int qk_select, int take, int block_size,
    uint32_t pinf1, uint32_t ninf1, int32_t* __restrict__ topk_idx) {
  __shared__ uint32_t s_scr[4][256];  // per-wave gather space of the k-th key search
  // The CIS page scores of the workgroup's sequence and group, when its four
  // rows share them (all but the workgroups that straddle a boundary).
  __shared__ __align__(16) float s_cpg[KPL * 64];
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t n_rows = (int64_t)G * total_q;
  const int64_t row0 = (int64_t)blockIdx.x * 4;
  const int64_t row_l = min(row0 + 3, n_rows - 1);
  const int g0 = (int)(row0 / total_q), gl = (int)(row_l / total_q);
  const int b0 = ls_find_segment(cu_q, batch, row0 - (int64_t)g0 * total_q);
  const int bl = ls_find_segment(cu_q, batch, row_l - (int64_t)gl * total_q);
  const bool shared_cis = g0 == gl && b0 == bl;
  if (shared_cis) {
    const int A0 = cu_a[b0 + 1] - cu_a[b0];
    const int n_sc = min(A0 > 0 ? A0 / 4 + 1 : 0, out_len);
    const int last = n_sc > 0 ? n_sc - 1 : 0;
    const float* cs = cpg + (int64_t)g0 * cpg_g_stride + pg_off[b0];
    const uint32_t base = (uint32_t)(uintptr_t)(ls_lds_void*)s_cpg;
    for (int sl = wv; sl < (n_sc + 63) / 64; sl += 4)
      ls_dma4(cs, 4u * (uint32_t)min(sl * 64 + lane, last), base + 256u * (uint32_t)sl);
    LS_WAIT_VMCNT(0);
  }
  __syncthreads();
  const int64_t row = row0 + wv;
  if (row >= n_rows) return;
  uint32_t* const scr = s_scr[wv];
  const float* const cpg_lds = shared_cis ? s_cpg : nullptr;
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
  const float* cpg_seq = cpg + (int64_t)g * cpg_g_stride + pg_off[b];
  int32_t* orow = topk_idx + row * take;
  const int64_t prow = row * p_stride;
  const int n_slots = (out_len + 63) >> 6;
  if (n_slots <= 1) return ls_nosa_topk_row<1, KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
  if (n_slots <= 2) return ls_nosa_topk_row<2, KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
  if (n_slots <= 4 || KPL <= 4) return ls_nosa_topk_row<(KPL < 4 ? KPL : 4), KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
  if (n_slots <= 8 || KPL <= 8) return ls_nosa_topk_row<(KPL < 8 ? KPL : 8), KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
  if (n_slots <= 16 || KPL <= 16) return ls_nosa_topk_row<(KPL < 16 ? KPL : 16), KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
  if (n_slots <= 32 || KPL <= 32) return ls_nosa_topk_row<(KPL < 32 ? KPL : 32), KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
  if (n_slots <= 64 || KPL <= 64) return ls_nosa_topk_row<(KPL < 64 ? KPL : 64), KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
  return ls_nosa_topk_row<KPL, KEY32, CIS32>(P, prow, cpg_seq, n_scored, out_len, off_bq, q_idx, init_blocks, local_blocks, qk_select, take, pinf1, ninf1, lane, orow, scr, cpg_lds);
}

template <bool KEY32, bool CIS32>
static int launch_nosa_topk_k(int out_len, dim3 grid, hipStream_t s, const void* P, int64_t ps,
                              const float* cpg, int64_t cs, const int32_t* pg_off,
                              const int32_t* cu_q, const int32_t* cu_a, int batch, int64_t total_q,
                              int G, int max_q, int init, int local, int qk_select, int take,
                              int bs, uint32_t pinf1, uint32_t ninf1, int32_t* out) {
#define LS_NOSA_TOPK(K)                                                                          \
  hipLaunchKernelGGL((ls_nosa_topk_kernel<K, KEY32, CIS32>), grid, dim3(256), 0, s, P, ps, cpg, cs,    \
                     pg_off, cu_q, cu_a, batch, total_q, G, max_q, out_len, init, local,       \
                     qk_select, take, bs, pinf1, ninf1, out)
  if (out_len <= 256) LS_NOSA_TOPK(4);
  else if (out_len <= 1024) LS_NOSA_TOPK(16);
  else if (out_len <= 2048) LS_NOSA_TOPK(32);
  else if (out_len <= 4096) LS_NOSA_TOPK(64);
  else if (out_len <= 8192) LS_NOSA_TOPK(128);
  else return ls_fail(LS_ERR_UNSUPPORTED, "NOSA selection: at most 8192 pages per row (got %d)", out_len);
#undef LS_NOSA_TOPK
  return ls_check_launch("ls_nosa_topk_kernel");
}

int ls_nosa_topk_launch(int p_dtype, int cis_dtype, int out_len, const void* P, int64_t p_stride, const float* cpg,
                        int64_t cpg_g_stride, const int32_t* pg_off, const int32_t* cu_q,
                        const int32_t* cu_a, int batch, int64_t total_q, int G, int max_seqlen_q,
                        int init_blocks, int local_blocks, int qk_select, int take,
                        int block_size, int32_t* topk_idx, hipStream_t s) {
  if (total_q == 0 || G == 0 || take == 0) return LS_OK;
  const dim3 grid((unsigned)(((int64_t)G * total_q + 3) / 4));
  const bool cis16 = cis_dtype == LS_BF16;
#define LS_NOSA_TOPK_ARGS                                                                      \
  out_len, grid, s, P, p_stride, cpg, cpg_g_stride, pg_off, cu_q, cu_a, batch, total_q, G,   \
      max_seqlen_q, init_blocks, local_blocks, qk_select, take, block_size, pinf, ninf, topk_idx
  if (p_dtype == LS_F32) {
    const uint32_t pinf = ls_order_key32(0x7f800000u), ninf = ls_order_key32(0xff800000u);
    return cis16 ? launch_nosa_topk_k<true, false>(LS_NOSA_TOPK_ARGS)
                 : launch_nosa_topk_k<true, true>(LS_NOSA_TOPK_ARGS);
  }
  const uint32_t pinf = ls_order_key16(p_dtype == LS_BF16 ? 0x7f80u : 0x7c00u);
  const uint32_t ninf = ls_order_key16(p_dtype == LS_BF16 ? 0xff80u : 0xfc00u);
  return cis16 ? launch_nosa_topk_k<false, false>(LS_NOSA_TOPK_ARGS)
               : launch_nosa_topk_k<false, true>(LS_NOSA_TOPK_ARGS);
#undef LS_NOSA_TOPK_ARGS
}
