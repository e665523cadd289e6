// Decode over a KV cache: appending tokens (with the compressed keys they
// complete), stage-1 page selection for decode queries, and block-sparse
// split-K attention over the cache.
//
// Cache layout (the caller's tensors): k_cache and v_cache hold
// [batch][capacity][G][D] rows, kc_cache [batch][kc_capacity][G][D], with the
// given batch and row strides (elements; the head stride is D).  Sequence b
// holds cache_seqlens[b] tokens.  Rows past a sequence's length are never
// read as values: keys there are masked before the softmax and values are
// replaced by zeros when they are staged.
//
// Follows the decode branch of the reference: InfLLMv2CacheLayer's compressed
// key update (leanselect/models/minicpm.py:1237-1325, 2888-2958),
// compressed_attention with cache_lens (minicpm.py:594-705) on the stage-1
// scores (infllmv2_attn_stage1, third_party/infllmv2/paper1.patch:1103-1302,
// 2340-2362), and infllmv2_attn_with_kvcache with topk_idx
// (paper1.patch:2511-2615).
#include <type_traits>

#include "ls_common.h"
#include "ls_topk_row.h"

#define LS_TID ((int)__builtin_amdgcn_workitem_id_x())
#define LS_BID_X ((int)__builtin_amdgcn_workgroup_id_x())
#define LS_BID_Y ((int)__builtin_amdgcn_workgroup_id_y())
#define LS_BID_Z ((int)__builtin_amdgcn_workgroup_id_z())

// Compressed windows of a sequence of `len` tokens: (len - ks) / stride + 1,
// or 0 when len < ks.
__host__ __device__ __forceinline__ int64_t ls_n_windows(int64_t len, int ks, int stride) {
  return len >= ks ? (len - ks) / stride + 1 : 0;
}

// ---------------------------------------------------------------------------
// Append.  Thread (row, g, chunk of 8 channels) copies 16 bytes of K and of V
// from the packed new rows to position cache_seqlens[b] + (row - cu_new[b]).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ls_cache_append_kernel(
    uint16_t* __restrict__ kc_, uint16_t* __restrict__ vc_, int64_t cbs, int64_t crs,
    const int32_t* __restrict__ cache_seqlens, const uint16_t* __restrict__ kn,
    const uint16_t* __restrict__ vn, int64_t nrs, const int32_t* __restrict__ cu_new,
    int64_t total_new, int batch, int G, int D) {
  const int c8 = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_row = (int64_t)G * c8;
  const int64_t row = idx / per_row;
  if (row >= total_new) return;
  const int rem = (int)(idx - row * per_row);
  const int g = rem / c8, c = rem - g * c8;
  const int b = ls_find_segment(cu_new, batch, row);
  const int64_t pos = (int64_t)cache_seqlens[b] + (row - cu_new[b]);
  const int64_t src = row * nrs + (int64_t)g * D + 8 * c;
  const int64_t dst = (int64_t)b * cbs + pos * crs + (int64_t)g * D + 8 * c;
  *reinterpret_cast<ls_u32x4*>(kc_ + dst) = ls_load16(kn + src);
  *reinterpret_cast<ls_u32x4*>(vc_ + dst) = ls_load16(vn + src);
}

// cu_win[b] = sum_{b' < b} (windows after the append - windows before it).
__global__ void ls_cache_window_plan_kernel(const int32_t* __restrict__ cache_seqlens,
                                            const int32_t* __restrict__ cu_new, int batch, int ks,
                                            int stride, int32_t* __restrict__ cu_win) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t acc = 0;
  cu_win[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int64_t l0 = cache_seqlens[b], l1 = l0 + (cu_new[b + 1] - cu_new[b]);
    acc += (int32_t)(ls_n_windows(l1, ks, stride) - ls_n_windows(l0, ks, stride));
    cu_win[b + 1] = acc;
  }
}

// One thread per (new window, g, 8 channels): the window's mean over the
// cache rows [w*stride, w*stride + ks), summed in float32 in token order.  For
// windows of two strides the two halves are summed separately and added, the
// order of the prefill's half-window kernel, so a window formed here is
// bit-identical to the one the prefill forms from the same keys.
template <int DT>
__global__ __launch_bounds__(256) void ls_cache_compress_kernel(
    const uint16_t* __restrict__ kcache, int64_t cbs, int64_t crs,
    const int32_t* __restrict__ cache_seqlens, const int32_t* __restrict__ cu_win, int batch,
    int G, int D, int ks, int stride, uint16_t* __restrict__ kcc, int64_t kbs, int64_t krs,
    int64_t max_windows) {
  const int c8 = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_win = (int64_t)G * c8;
  const int64_t wi = idx / per_win;
  if (wi >= max_windows || wi >= (int64_t)cu_win[batch]) return;
  const int rem = (int)(idx - wi * per_win);
  const int g = rem / c8, c = rem - g * c8;
  const int b = ls_find_segment(cu_win, batch, wi);
  const int64_t w = ls_n_windows(cache_seqlens[b], ks, stride) + (wi - cu_win[b]);
  const uint16_t* src = kcache + (int64_t)b * cbs + (w * stride) * crs + (int64_t)g * D + 8 * c;
  // Unrolled so that a block of row loads is in flight at once; the sums
  // still run in token order.
  auto add_rows = [&](int r0, int r1, float (&s)[8]) {
#pragma unroll 16
    for (int t = r0; t < r1; ++t) {
      const ls_u32x4 a = ls_load16(src + (int64_t)t * crs);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        s[2 * e] += LsElem<DT>::to_f((uint16_t)(a[e] & 0xffffu));
        s[2 * e + 1] += LsElem<DT>::to_f((uint16_t)(a[e] >> 16));
      }
    }
  };
  float acc[8], second[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) acc[e] = second[e] = 0.f;
  if (ks == 2 * stride) {
    add_rows(0, stride, acc);
    add_rows(stride, ks, second);
  } else {
    add_rows(0, ks, acc);
  }
  const float n_win = (float)ks;
  ls_u32x4 o;
#pragma unroll
  for (int e = 0; e < 4; ++e)
    o[e] = ls_pack2(LsElem<DT>::from_f((acc[2 * e] + second[2 * e]) / n_win),
                    LsElem<DT>::from_f((acc[2 * e + 1] + second[2 * e + 1]) / n_win));
  *reinterpret_cast<ls_u32x4*>(kcc + (int64_t)b * kbs + w * krs + (int64_t)g * D + 8 * c) = o;
}

// ---------------------------------------------------------------------------
// Stage-1 decode scores.  Row t (sequence b) and KV group g:
//   score[j] = sum_{h in g} softmax_j(scale * q[t][h] . kc[b][j][g])
// over the n_c(b) compressed keys of the sequence (no causal limit: the
// reference calls stage 1 with causal=False when decoding), rounded to the
// query dtype and then to bf16 (compressed_attention's .to(bfloat16)), then
// max-pooled into pages.  n_c(b) is the window count of the sequence's
// current length, clipped to max_kc.
//
// Pass 1 (one wave per 64-key chunk, row and group): S^T = Kc . Q^T on the
// 16x16x32 MFMA (keys are rows, the group's heads columns); the raw scores in
// base-2 units go to the workspace with each head's chunk maximum and
// sum of 2^(x - max).  Pass 2 (one workgroup per block of pages, row and
// group): each head's log2-sum-exp from the chunk partials, the scores of the
// keys in the block's page windows, and their page maxima.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int ls_dec_n_c(int64_t len, int ks, int stride, int64_t max_kc) {
  return (int)min(ls_n_windows(len, ks, stride), max_kc);
}

// x[g][t][h][j] (float, base-2 units, -inf past n_c), part[g][t][c][h] = (max, sum).
// Cache form (VARLEN false): sequence b's compressed keys are rows
// kcc[b kbs + j krs] and n_c(b) follows from its token count lens[b].  Packed
// form (VARLEN true): they are rows kcc[(lens[b] + j) krs] with n_c(b) =
// lens[b + 1] - lens[b] (lens = cu_seqlens of the compressed keys).
template <int DT, bool VARLEN = false>
__global__ __launch_bounds__(64) void ls_stage1_chunk_kernel(
    const uint16_t* __restrict__ q, int64_t qrs, const int32_t* __restrict__ cu_q, int batch,
    int64_t total_q, const uint16_t* __restrict__ kcc, int64_t kbs, int64_t krs,
    const int32_t* __restrict__ cache_seqlens, int ks, int stride, int64_t max_kc, int gs, int D,
    float scale_log2, int64_t ncpad, int n_chunks, float* __restrict__ x,
    float* __restrict__ part) {
  const int c = LS_BID_X;
  const int64_t t = LS_BID_Y;
  const int g = LS_BID_Z;
  const int lane = LS_TID, r = lane & 15, qg = lane >> 4;
  const int b = ls_find_segment(cu_q, batch, t);
  const int nc = VARLEN ? (int)min((int64_t)(cache_seqlens[b + 1] - cache_seqlens[b]), max_kc)
                        : ls_dec_n_c(cache_seqlens[b], ks, stride, max_kc);
  const int64_t kbase = VARLEN ? (int64_t)cache_seqlens[b] * krs : (int64_t)b * kbs;
  float* xrow = x + ((int64_t)g * total_q + t) * 16 * ncpad;
  float* prow = part + (((int64_t)g * total_q + t) * n_chunks + c) * 32;
  // Q^T fragments (B operand): lane (r, qg) holds head r, dims 32 ks + 8 qg + 0..7.
  ls_u32x4 qf[4];
  const bool head_ok = r < gs;
  const uint16_t* qrow = q + t * qrs + ((int64_t)g * gs + r) * D + 8 * qg;
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4)
    qf[k4] = head_ok ? ls_load16(qrow + 32 * k4) : ls_u32x4{0u, 0u, 0u, 0u};
  float m = -INFINITY;
  float sv[16];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int j = 64 * c + 16 * kb + r;  // key row of this lane's A fragment
    ls_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const bool key_ok = j < nc;
    const uint16_t* krow = kcc + kbase + (int64_t)j * krs + (int64_t)g * D + 8 * qg;
#pragma unroll
    for (int k4 = 0; k4 < 4; ++k4) {
      const ls_u32x4 kf = key_ok ? ls_load16(krow + 32 * k4) : ls_u32x4{0u, 0u, 0u, 0u};
      acc = LsElem<DT>::mfma(kf, qf[k4], acc);
    }
    // acc[i]: head r (column), key 64 c + 16 kb + 4 qg + i (row).
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int jj = 64 * c + 16 * kb + 4 * qg + i;
      const float v = jj < nc ? acc[i] * scale_log2 : -INFINITY;
      sv[4 * kb + i] = v;
      m = fmaxf(m, v);
    }
  }
  m = fmaxf(m, ls_shfl_xor(m, 16));
  m = fmaxf(m, ls_shfl_xor(m, 32));
  float l = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) l += m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sv[i] - m);
  l += ls_shfl_xor(l, 16);
  l += ls_shfl_xor(l, 32);
  if (head_ok) {
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int jj = 64 * c + 16 * kb + 4 * qg;
      *reinterpret_cast<ls_f32x4*>(xrow + (int64_t)r * ncpad + jj) =
          ls_f32x4{sv[4 * kb], sv[4 * kb + 1], sv[4 * kb + 2], sv[4 * kb + 3]};
    }
    if (qg == 0) {
      prow[2 * r] = m;
      prow[2 * r + 1] = l;
    }
  }
}

// Each head's log2-sum-exp of one (row, group) from its nch chunk partials
// prow[c * 32 + 2 h] = (max, sum), into s_lse[h] for h < gs, by the 256
// threads of a workgroup (every thread calls it): sixteen consecutive threads
// per head (four heads per wave) reduce the head's partials, each a strided
// share, then butterfly shuffles.
__device__ __forceinline__ void ls_stage1_lse(const float* __restrict__ prow, int nch, int gs,
                                              int tid, float* __restrict__ s_lse) {
  const int h = tid >> 4, share = tid & 15;
  // A thread's first eight (max, sum) pairs (chunks share + 16 i: all of
  // them up to 128 chunks) are loaded once, together, and kept for the sum;
  // chunks beyond are read in the loops.
  constexpr int NP = 8;
  float pm[NP], pl[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const int c = share + 16 * i;
    const bool ok = h < gs && c < nch;
    const float2 v = ok ? *reinterpret_cast<const float2*>(prow + c * 32 + 2 * h)
                        : make_float2(-INFINITY, 0.f);
    pm[i] = v.x;
    pl[i] = v.y;
  }
  float M = -INFINITY;
#pragma unroll
  for (int i = 0; i < NP; ++i) M = fmaxf(M, pm[i]);
  if (h < gs)
    for (int c = share + 16 * NP; c < nch; c += 16) M = fmaxf(M, prow[c * 32 + 2 * h]);
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) M = fmaxf(M, ls_shfl_xor(M, o));
  float L = 0.f;
  if (h < gs && M != -INFINITY) {
#pragma unroll
    for (int i = 0; i < NP; ++i)
      if (pm[i] != -INFINITY) L += pl[i] * __builtin_amdgcn_exp2f(pm[i] - M);
    for (int c = share + 16 * NP; c < nch; c += 16) {
      const float mc = prow[c * 32 + 2 * h];
      if (mc != -INFINITY) L += prow[c * 32 + 2 * h + 1] * __builtin_amdgcn_exp2f(mc - M);
    }
  }
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) L += ls_shfl_xor(L, o);
  if (h < gs && share == 0) s_lse[h] = M + __log2f(L);
}

// Pass 2 and the page max-pool of max_pooling_1d_varlen, fused.  Workgroup
// (page block pb, row t, group g) covers pages [ppb pb, ppb pb + ppb) of
// sp = block_size / kernel_stride keys each (ppb sp <= 256).  It forms each
// head's log2-sum-exp from the chunk partials, scores the keys
// [ppb sp pb - 1, ppb sp (pb + 1)) into LDS (-inf outside [0, n_c)), and writes
//   pooled[g][t][p] = +inf            if p < init_blocks or
//                                        q_page - local_blocks <= p <= q_page,
//                     max of the scores of keys [p sp - 1, p sp + sp)  otherwise
// (-inf when none exists), q_page = (len_b - len_q(b) + i) / block_size for
// row i of sequence b.
template <int DT>
__global__ __launch_bounds__(256) void ls_stage1_pool_kernel(
    const float* __restrict__ x, const float* __restrict__ part, const int32_t* __restrict__ cu_q,
    int batch, int64_t total_q, const int32_t* __restrict__ cache_seqlens, int ks, int stride,
    int64_t max_kc, int gs, int64_t ncpad, int n_chunks, int sp, int ppb, int64_t out_len,
    int block_size, int init_blocks, int local_blocks, uint16_t* __restrict__ pooled) {
  const int64_t p0 = (int64_t)ppb * LS_BID_X;
  const int64_t t = LS_BID_Y;
  const int g = LS_BID_Z;
  const int tid = LS_TID;
  __shared__ float s_lse[16];
  __shared__ float s_sc[257];
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t len_b = cache_seqlens[b];
  const int nc = ls_dec_n_c(len_b, ks, stride, max_kc);
  const int64_t j0 = p0 * sp - 1;  // key of LDS slot 0
  const int n_keys = ppb * sp + 1;
  const bool has_keys = max((int64_t)0, j0) < (int64_t)nc;  // uniform
  if (has_keys)
    ls_stage1_lse(part + ((int64_t)g * total_q + t) * n_chunks * 32, (nc + 63) / 64, gs, tid,
                  s_lse);
  __syncthreads();
  const float* xrow = x + ((int64_t)g * total_q + t) * 16 * ncpad;
  for (int i = tid; i < n_keys; i += 256) {
    const int64_t j = j0 + i;
    float v = -INFINITY;
    if (j >= 0 && j < nc) {
      float s = 0.f;
#pragma unroll 16
      for (int h = 0; h < gs; ++h) s += __builtin_amdgcn_exp2f(xrow[(int64_t)h * ncpad + j] - s_lse[h]);
      uint16_t o;
      if constexpr (DT == LS_F16)
        o = ls_f32_to_bf16(ls_f16_to_f32(ls_f32_to_f16(s)));
      else
        o = ls_f32_to_bf16(s);
      v = ls_bf16_to_f32(o);
    }
    s_sc[i] = v;
  }
  __syncthreads();
  const int64_t q_page = (len_b - (cu_q[b + 1] - cu_q[b]) + (t - cu_q[b])) / block_size;
  uint16_t* orow = pooled + ((int64_t)g * total_q + t) * out_len;
  for (int i = tid; i < ppb; i += 256) {
    const int64_t p = p0 + i;
    if (p >= out_len) break;
    float v;
    if (p < init_blocks || (q_page - local_blocks <= p && p <= q_page)) {
      v = INFINITY;
    } else {
      v = -INFINITY;
      for (int e = 0; e <= sp; ++e) v = fmaxf(v, s_sc[i * sp + e]);
    }
    orow[p] = ls_f32_to_bf16(v);
  }
}

// Stage-1 scores as infllmv2_attn_stage1 returns them when decoding
// (paper1.patch:2312-2361 with causal=False): out[g][t][j] = sum over the
// group's heads of softmax_j(scale q[t][h] . kc[j][g]) for the n_c(b)
// compressed keys of the row's sequence, rounded to the query dtype, 0 for
// j >= n_c(b) and where the score is NaN.  One workgroup per (row, group).
template <int DT>
__global__ __launch_bounds__(256) void ls_stage1_scores_kernel(
    const float* __restrict__ x, const float* __restrict__ part, const int32_t* __restrict__ cu_q,
    int batch, int64_t total_q, const int32_t* __restrict__ cu_kc, int64_t max_kc, int gs,
    int64_t ncpad, int n_chunks, int64_t out_cols, uint16_t* __restrict__ out) {
  const int64_t t = LS_BID_X;
  const int g = LS_BID_Y;
  const int tid = LS_TID;
  __shared__ float s_lse[16];
  const int b = ls_find_segment(cu_q, batch, t);
  const int nc = (int)min((int64_t)(cu_kc[b + 1] - cu_kc[b]), max_kc);
  if (nc > 0)
    ls_stage1_lse(part + ((int64_t)g * total_q + t) * n_chunks * 32, (nc + 63) / 64, gs, tid,
                  s_lse);
  __syncthreads();
  const float* xrow = x + ((int64_t)g * total_q + t) * 16 * ncpad;
  uint16_t* orow = out + ((int64_t)g * total_q + t) * out_cols;
  for (int64_t j = tid; j < out_cols; j += 256) {
    float v = 0.f;
    if (j < nc) {
      float sum = 0.f;
      for (int h = 0; h < gs; ++h) sum += __builtin_amdgcn_exp2f(xrow[(int64_t)h * ncpad + j] - s_lse[h]);
      v = sum;
    }
    const uint16_t o = LsElem<DT>::from_f(v);
    orow[j] = (__builtin_isnan(v) ? (uint16_t)0 : o);
  }
}

// ---------------------------------------------------------------------------
// Decode top-k over pooled page scores pooled[g][t][out_len] (bf16, forced
// pages +inf, pages without keys -inf): the `take` best pages (ties to the
// lower page), ascending, ids past the row's page q_idx replaced by -1 (they
// sort last, so the list is the kept ids then -1 padding).  One workgroup per
// (row, group).  The row's 16-bit order keys are held in LDS; the take-th
// largest key T is found by a two-pass 8-bit radix select (histogram of the
// high byte, then of the low byte among keys with T's high byte, each bucket
// found with a parallel suffix sum), and the pages with key > T plus the
// lowest-page m = take - #{key > T} pages with key == T are compacted in page
// order (thread i owns a contiguous run of pages).
// ---------------------------------------------------------------------------
#define LS_DEC_TOPK_MAX_PAGES 30720  // LDS keys (60 KB, with the static arrays under 64 KB)

__global__ __launch_bounds__(256) void ls_decode_topk_kernel(
    const uint16_t* __restrict__ pooled, const int32_t* __restrict__ cu_q, int batch,
    int64_t total_q, const int32_t* __restrict__ cache_seqlens, int out_len, int block_size,
    int take, int32_t* __restrict__ ids) {
  const int64_t t = LS_BID_X;
  const int g = LS_BID_Y;
  const int tid = LS_TID, lane = tid & 63, w = tid >> 6;
  extern __shared__ uint16_t s_key[];  // out_len order keys
  __shared__ uint32_t s_hist[256];
  __shared__ int32_t s_wtot[4];
  __shared__ uint32_t s_sel[3];  // bucket, keys still needed inside it, keys above it
  const uint16_t* row = pooled + ((int64_t)g * total_q + t) * out_len;
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t q_idx =
      ((int64_t)cache_seqlens[b] - (cu_q[b + 1] - cu_q[b]) + (t - cu_q[b])) / block_size;
  for (int p = tid; p < out_len; p += 256) s_key[p] = (uint16_t)ls_order_key16(row[p]);
  s_hist[tid] = 0u;
  __syncthreads();
  // The bucket d holding the need-th largest key: #{bucket > d} < need <= #{bucket >= d}.
  auto find_bucket = [&](uint32_t need) {
    const uint32_t h = s_hist[tid];
    uint32_t sfx = h;  // keys in buckets tid .. (wave's last)
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const uint32_t y = (uint32_t)__shfl_down((int)sfx, off, 64);
      if (lane + off < 64) sfx += y;
    }
    if (lane == 0) s_wtot[w] = (int32_t)sfx;
    __syncthreads();
    for (int v = w + 1; v < 4; ++v) sfx += (uint32_t)s_wtot[v];
    const uint32_t above = sfx - h;
    if (h > 0u && sfx >= need && above < need) {
      s_sel[0] = (uint32_t)tid;
      s_sel[1] = need - above;
      s_sel[2] = above;
    }
    __syncthreads();
  };
  for (int p = tid; p < out_len; p += 256) atomicAdd(&s_hist[s_key[p] >> 8], 1u);
  __syncthreads();
  find_bucket((uint32_t)take);
  const uint32_t hi = s_sel[0], need_lo = s_sel[1];
  s_hist[tid] = 0u;
  __syncthreads();
  for (int p = tid; p < out_len; p += 256) {
    const uint32_t k = s_key[p];
    if ((k >> 8) == hi) atomicAdd(&s_hist[k & 255u], 1u);
  }
  __syncthreads();
  find_bucket(need_lo);
  const uint32_t T = (hi << 8) | s_sel[0];
  const int m = (int)s_sel[1];  // keys equal to T that are taken (the lowest pages)
  // Block-wide exclusive scan of one count per thread (also returns the total).
  auto block_scan = [&](int v, int* total) {
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int y = __shfl_up(x, off, 64);
      if (lane >= off) x += y;
    }
    __syncthreads();  // earlier readers of s_wtot are done
    if (lane == 63) s_wtot[w] = x;
    __syncthreads();
    int before = x - v, tot = 0;
    for (int v2 = 0; v2 < 4; ++v2) {
      if (v2 < w) before += s_wtot[v2];
      tot += s_wtot[v2];
    }
    *total = tot;
    return before;
  };
  const int per = (out_len + 255) / 256;
  const int p0 = min(out_len, tid * per), p1 = min(out_len, p0 + per);
  int n_eq = 0;
  for (int p = p0; p < p1; ++p) n_eq += s_key[p] == T ? 1 : 0;
  int unused;
  int eq_rank = block_scan(n_eq, &unused);
  int n_keep = 0;
  for (int p = p0; p < p1; ++p) {
    const uint32_t k = s_key[p];
    const bool sel = k > T || (k == T && eq_rank < m);
    eq_rank += k == T ? 1 : 0;
    n_keep += (sel && p <= q_idx) ? 1 : 0;
  }
  int kept;
  int pos = block_scan(n_keep, &kept);
  int32_t* orow = ids + ((int64_t)g * total_q + t) * take;
  eq_rank = eq_rank - n_eq;  // back to this thread's first page
  for (int p = p0; p < p1; ++p) {
    const uint32_t k = s_key[p];
    const bool sel = k > T || (k == T && eq_rank < m);
    eq_rank += k == T ? 1 : 0;
    if (sel && p <= q_idx) orow[pos++] = p;
  }
  for (int i = kept + tid; i < take; i += 256) orow[i] = -1;
}
// The same selection for rows of at most 64 * KPL pages, one wave per (row,
// group): the prefill path's wave-level top-k (the lanes' two largest keys
// bound the take-th key from below, the keys above the bound are gathered
// with their pages and bisected) over the whole pooled row, written in page
// order with the ids above q_idx as -1 (the ascending list's tail).
template <int KPL>
__global__ __launch_bounds__(256) void ls_decode_topk_wave_kernel(
    const uint16_t* __restrict__ pooled, const int32_t* __restrict__ cu_q, int batch,
    int64_t total_q, int G, const int32_t* __restrict__ cache_seqlens, int out_len,
    int block_size, int take, int32_t* __restrict__ ids) {
  __shared__ uint32_t s_scr[4][320];  // per-wave gather space
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int64_t row = (int64_t)blockIdx.x * 4 + wv;  // g * total_q + t
  if (row >= (int64_t)G * total_q) return;
  const int g = (int)(row / total_q);
  const int64_t t = row - (int64_t)g * total_q;
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t q_idx =
      ((int64_t)cache_seqlens[b] - (cu_q[b + 1] - cu_q[b]) + (t - cu_q[b])) / block_size;
  ls_topk_select16<KPL>(pooled, row * out_len, out_len, take, 0, lane, ids + row * take,
                        s_scr[wv], (int)min(q_idx, (int64_t)INT32_MAX));
}

// The same selection with the four waves of a workgroup sharing one (row,
// group), for rows of 5 to 4 * 64 * NSW pages and take <= 128: wave w holds
// slots [w NSW, (w + 1) NSW) of the row (16-bit order keys << 16), the lanes'
// two largest keys of all four waves bound the take-th key from below (lo),
// each wave gathers its keys >= lo packed with their page, in page order after
// the waves before it, and wave 0 bisects and emits from the gathered keys.
// More than 256 keys above the bound (or none) hands the row to the one-wave
// selection.
template <int NSW>
__global__ __launch_bounds__(256) void ls_decode_topk_wg_kernel(
    const uint16_t* __restrict__ pooled, const int32_t* __restrict__ cu_q, int batch,
    int64_t total_q, int G, const int32_t* __restrict__ cache_seqlens, int out_len,
    int block_size, int take, int32_t* __restrict__ ids) {
  __shared__ uint32_t s_m[2][256];   // each lane's two largest keys (<< 16)
  __shared__ uint32_t s_scr[320];    // gathered key | page, page order
  __shared__ int s_cnt[4];
  __shared__ uint32_t s_lo;
  const int tid = threadIdx.x, lane = tid & 63;
  const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int64_t row = blockIdx.x;  // g * total_q + t
  const int g = (int)(row / total_q);
  const int64_t t = row - (int64_t)g * total_q;
  const int cn = out_len;
  const uint16_t* rowp = pooled + row * out_len;
  int32_t* orow = ids + row * take;
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t q_idx =
      ((int64_t)cache_seqlens[b] - (cu_q[b + 1] - cu_q[b]) + (t - cu_q[b])) / block_size;
  const int id_max = (int)min(q_idx, (int64_t)INT32_MAX);
  uint32_t key[NSW];
#pragma unroll
  for (int s = 0; s < NSW; ++s) key[s] = rowp[min((w * NSW + s) * 64 + lane, cn - 1)];
  uint32_t m1 = 0u, m2 = 0u;
#pragma unroll
  for (int s = 0; s < NSW; ++s) {
    const uint32_t b16 = key[s];
    uint32_t k = (b16 ^ ((b16 >> 15) * 0x7fffu) ^ 0x8000u) << 16;  // ls_order_key16 << 16
    if ((w * NSW + s) * 64 + lane >= cn) k = 0u;
    key[s] = k;
    m2 = max(m2, min(m1, k));
    m1 = max(m1, k);
  }
  s_m[0][tid] = m1;
  s_m[1][tid] = m2;
  __syncthreads();
  if (w == 0) {
    uint32_t mm[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mm[2 * i] = s_m[0][64 * i + lane] >> 16;
      mm[2 * i + 1] = s_m[1][64 * i + lane] >> 16;
    }
    const uint32_t lo = ls_kth_bisect<8>(mm, take, 0u, 15);
    if (lane == 0) s_lo = lo;
  }
  __syncthreads();
  const uint32_t lo = s_lo;
  const uint32_t lo_sh = lo << 16;
  int n = 0;  // this wave's keys >= lo
#pragma unroll
  for (int s = 0; s < NSW; ++s) n += __popcll(__ballot(lo != 0u && key[s] >= lo_sh));
  if (lane == 0) s_cnt[w] = n;
  __syncthreads();
  int off = 0, total = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    off += i < w ? s_cnt[i] : 0;
    total += s_cnt[i];
  }
  if (lo == 0u || total > 256) {  // no usable bound: the one-wave selection takes the row
    if (w == 0) {
      uint32_t* scr = s_scr;
      ls_topk_select16<4 * NSW>(pooled, row * out_len, cn, take, 0, lane, orow, scr, id_max);
    }
    return;
  }
  int pos0 = off;
#pragma unroll
  for (int s = 0; s < NSW; ++s) {
    const bool sv = key[s] >= lo_sh;
    const uint64_t mk = __ballot(sv);
    const int pos = (int)__builtin_amdgcn_mbcnt_hi(
        (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, (uint32_t)pos0));
    if (sv) s_scr[pos] = key[s] | (uint32_t)((w * NSW + s) * 64 + lane);
    pos0 += __popcll(mk);
  }
  __syncthreads();
  if (w != 0) return;
  uint32_t hi = 0u;  // this lane's maximum over the four waves (reduced inside)
#pragma unroll
  for (int i = 0; i < 4; ++i) hi = max(hi, s_m[0][64 * i + lane] >> 16);
  if (total <= 64) ls_topk_emit_packed<1>(s_scr, total, lo, hi, take, 0, lane, orow, id_max);
  else if (total <= 128) ls_topk_emit_packed<2>(s_scr, total, lo, hi, take, 0, lane, orow, id_max);
  else ls_topk_emit_packed<4>(s_scr, total, lo, hi, take, 0, lane, orow, id_max);
}

// ---------------------------------------------------------------------------
// Split-K attention over the cache.  Workgroup (split s, row t, group g) has
// four waves; wave w runs the pages of plan slots
// [(4 s + w) ppw, (4 s + w + 1) ppw) of row t (valid ids, each page once: a
// slot repeating an earlier slot's id is skipped) with an online softmax.  The
// four waves merge their per-head maximum, sum and unnormalised O through LDS
// and write one partial per workgroup; the combine kernel merges the splits.
// Keys visible to row t of sequence b (i = t - cu_q[b]): j < len_b
// (causal=false) or j <= len_b - len_q(b) + i (causal, the bottom-right
// alignment of flash-attention's kvcache call).
// S^T = K . Q^T (keys rows, heads columns) on the bf16/fp16 MFMA, with the
// keys of each 32-key chunk permuted so lane group q holds keys 8q..8q+7 of
// the chunk: P^T then feeds O^T = V^T . P^T from registers.  P is split into
// a 16-bit head and a 16-bit remainder (two MFMAs) so it carries about 16
// significant bits; V^T fragments come from the wave's LDS copy of the page.
// ---------------------------------------------------------------------------
#define LS_DEC_VPITCH 260  // bytes per staged V row (65 dwords: conflict-free transposed reads)
#define LS_DEC_VBYTES (64 * LS_DEC_VPITCH)
#define LS_DEC_PART (16 * 128 + 32)  // floats per partial: O [16][128], m [16], l [16]
#define LS_DEC_MAX_SPLITS 64
#define LS_DEC_ID_REGS 4     // plan ids held in registers: topk <= 256

__device__ __forceinline__ void ls_dec_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int DT>
__global__ __launch_bounds__(256) void ls_decode_attn_kernel(
    const uint16_t* __restrict__ q, int64_t qrs, const int32_t* __restrict__ cu_q, int batch,
    int64_t total_q, const uint16_t* __restrict__ kc_, const uint16_t* __restrict__ vc_,
    int64_t cbs, int64_t crs, const int32_t* __restrict__ cache_seqlens, int gs, int D,
    const int32_t* __restrict__ topk_idx, int topk, int ppw, int n_splits, float scale_log2,
    int causal, float* __restrict__ part) {
  const int s = LS_BID_X;
  const int64_t t = LS_BID_Y;
  const int g = LS_BID_Z;
  const int tid = LS_TID, lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, qg = lane >> 4;
  __shared__ __attribute__((aligned(16))) uint8_t s_v[4][LS_DEC_VBYTES];
  uint8_t* sv_w = s_v[w];
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t len_b = cache_seqlens[b];
  const int64_t i_row = t - cu_q[b];
  const int64_t len_q = cu_q[b + 1] - cu_q[b];
  const int64_t limit = causal ? len_b - len_q + i_row + 1 : len_b;  // keys j < limit
  const int64_t n_pages = (len_b + 63) / 64;
  const bool head_ok = r < gs;
  ls_u32x4 qf[4];
  const uint16_t* qrow = q + t * qrs + ((int64_t)g * gs + r) * D + 8 * qg;
#pragma unroll
  for (int k4 = 0; k4 < 4; ++k4)
    qf[k4] = head_ok ? ls_load16(qrow + 32 * k4) : ls_u32x4{0u, 0u, 0u, 0u};
  float m_run = -INFINITY, l_run = 0.f;
  ls_f32x4 o[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) o[db] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
  // The row's plan ids, 64 per register (topk <= 64 * LS_DEC_ID_REGS).
  const int32_t* idrow = topk_idx + ((int64_t)g * total_q + t) * topk;
  int idr[LS_DEC_ID_REGS];
#pragma unroll
  for (int k = 0; k < LS_DEC_ID_REGS; ++k) idr[k] = 64 * k + lane < topk ? idrow[64 * k + lane] : -1;
  const uint16_t* kseq = kc_ + (int64_t)b * cbs + (int64_t)g * D;
  const uint16_t* vseq = vc_ + (int64_t)b * cbs + (int64_t)g * D;
  const int slot0 = (4 * s + w) * ppw, slot1 = min(topk, slot0 + ppw);
  for (int slot = slot0; slot < slot1; ++slot) {
    int held = idr[0];
#pragma unroll
    for (int k = 1; k < LS_DEC_ID_REGS; ++k)
      if ((slot >> 6) == k) held = idr[k];
    const int id = __builtin_amdgcn_readlane(held, slot & 63);
    if (id < 0 || (int64_t)id >= n_pages || 64LL * id >= limit) continue;
    // Skip a repeated id (the reference forms a page bitmask, so each page counts once).
    bool dup = false;
#pragma unroll
    for (int k = 0; k < LS_DEC_ID_REGS; ++k) dup |= __ballot(64 * k + lane < slot && idr[k] == id) != 0ull;
    if (dup) continue;
    const int64_t key0 = 64LL * id;
    const int64_t nvis = min((int64_t)64, limit - key0);  // visible keys of this page (> 0)
    // The page's K fragments and V rows are loaded together (keys past nvis as
    // zeros).  K block kb = 2 c + nb, MFMA row R holds key 32 c + 8 (R / 4) + 4 nb + R % 4.
    ls_u32x4 kf[4][4], vv[16];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int krow = 32 * (kb >> 1) + 8 * (r >> 2) + 4 * (kb & 1) + (r & 3);
      const uint16_t* kp = kseq + (key0 + krow) * crs + 8 * qg;
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4)
        kf[kb][k4] = krow < nvis ? ls_load16(kp + 32 * k4) : ls_u32x4{0u, 0u, 0u, 0u};
    }
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int ci = it * 64 + lane, kr = ci >> 4, c16 = ci & 15;
      vv[it] = kr < nvis ? ls_load16(vseq + (key0 + kr) * crs + 8 * c16) : ls_u32x4{0u, 0u, 0u, 0u};
    }
    float sv[16];
    float pm = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int cch = kb >> 1, nb = kb & 1;
      ls_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) acc = LsElem<DT>::mfma(kf[kb][k4], qf[k4], acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 32 * cch + 8 * qg + 4 * nb + i;  // row 4 qg + i of block kb
        const float v = key < nvis ? acc[i] * scale_log2 : -INFINITY;
        sv[4 * kb + i] = v;
        pm = fmaxf(pm, v);
      }
    }
    // V into the wave's LDS, rows of 128 values.
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int ci = it * 64 + lane, kr = ci >> 4, c16 = ci & 15;
      uint32_t* dst = reinterpret_cast<uint32_t*>(sv_w + kr * LS_DEC_VPITCH + 16 * c16);
      dst[0] = vv[it][0];
      dst[1] = vv[it][1];
      dst[2] = vv[it][2];
      dst[3] = vv[it][3];
    }
    pm = fmaxf(pm, ls_shfl_xor(pm, 16));
    pm = fmaxf(pm, ls_shfl_xor(pm, 32));
    const float m_new = fmaxf(m_run, pm);  // finite: every page here has a visible key
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    m_run = m_new;
    l_run *= alpha;
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db] *= alpha;
    ls_dec_wave_sync();  // the page's V rows are in the wave's LDS
#pragma unroll
    for (int cch = 0; cch < 2; ++cch) {
      // P^T fragment: lane (r, qg) holds head r, keys 32 cch + 8 qg + 0..7
      // (block 2 cch rows 4 qg..4 qg+3, then block 2 cch + 1).
      float p[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        p[i] = __builtin_amdgcn_exp2f(sv[4 * (2 * cch) + i] - m_new);
        p[4 + i] = __builtin_amdgcn_exp2f(sv[4 * (2 * cch + 1) + i] - m_new);
      }
      ls_u32x4 phi, plo;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint16_t h0 = LsElem<DT>::from_f(p[2 * i]), h1 = LsElem<DT>::from_f(p[2 * i + 1]);
        phi[i] = ls_pack2(h0, h1);
        plo[i] = ls_pack2(LsElem<DT>::from_f(p[2 * i] - LsElem<DT>::to_f(h0)),
                          LsElem<DT>::from_f(p[2 * i + 1] - LsElem<DT>::to_f(h1)));
        l_run += p[2 * i] + p[2 * i + 1];
      }
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        // V^T fragment: lane (r, qg) holds dim 16 db + r of keys 32 cch + 8 qg + 0..7.
        const uint8_t* vp = sv_w + (32 * cch + 8 * qg) * LS_DEC_VPITCH + 2 * (16 * db + r);
        uint16_t e[8];
#pragma unroll
        for (int k = 0; k < 8; ++k) e[k] = *reinterpret_cast<const uint16_t*>(vp + k * LS_DEC_VPITCH);
        const ls_u32x4 vf = {ls_pack2(e[0], e[1]), ls_pack2(e[2], e[3]), ls_pack2(e[4], e[5]),
                             ls_pack2(e[6], e[7])};
        o[db] = LsElem<DT>::mfma(vf, phi, o[db]);
        o[db] = LsElem<DT>::mfma(vf, plo, o[db]);
      }
    }
    ls_dec_wave_sync();  // all reads of the page's V done before the next page overwrites it
  }
  l_run += ls_shfl_xor(l_run, 16);
  l_run += ls_shfl_xor(l_run, 32);
  // The wave's state into its LDS block: O [16][128], then m [16], l [16].
  float* st = reinterpret_cast<float*>(sv_w);
#pragma unroll
  for (int db = 0; db < 8; ++db)  // o[db][i]: head r, dim 16 db + 4 qg + i
    *reinterpret_cast<ls_f32x4*>(st + r * 128 + 16 * db + 4 * qg) = o[db];
  if (qg == 0) {
    st[16 * 128 + r] = m_run;
    st[16 * 128 + 16 + r] = l_run;
  }
  __syncthreads();
  // Merge the four waves: thread e-range of the 16 x 128 outputs.
  float* pp = part + (((int64_t)g * total_q + t) * n_splits + s) * LS_DEC_PART;
  for (int e = tid; e < 16 * 128; e += 256) {
    const int h = e >> 7, d = e & 127;
    float mw[4], M = -INFINITY;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      mw[i] = reinterpret_cast<const float*>(s_v[i])[16 * 128 + h];
      M = fmaxf(M, mw[i]);
    }
    float acc = 0.f, L = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (mw[i] == -INFINITY) continue;
      const float wt = __builtin_amdgcn_exp2f(mw[i] - M);
      const float* si = reinterpret_cast<const float*>(s_v[i]);
      acc += wt * si[h * 128 + d];
      L += wt * si[16 * 128 + 16 + h];
    }
    pp[h * 128 + d] = acc;
    if (d == 0) {
      pp[16 * 128 + h] = M;
      pp[16 * 128 + 16 + h] = L;
    }
  }
}

// out[t][g*gs + h][:] = sum_s 2^(m_s - M) O_s / sum_s 2^(m_s - M) l_s; rows
// without a visible key give zeros and lse = +inf.  One workgroup per (row,
// group, head), a thread per output dimension; the first wave forms the
// splits' normalised weights (one split per lane) in LDS.
template <int DT>
__global__ __launch_bounds__(128) void ls_decode_combine_kernel(
    const float* __restrict__ part, int64_t total_q, int gs, int D, int n_splits,
    uint16_t* __restrict__ out, float* __restrict__ lse) {
  const int64_t t = LS_BID_X;
  const int g = LS_BID_Y;
  const int h = LS_BID_Z;
  const int tid = LS_TID;
  const int G = gridDim.y;
  __shared__ float s_w[LS_DEC_MAX_SPLITS];
  __shared__ float s_lse;
  const float* pr = part + ((int64_t)g * total_q + t) * n_splits * LS_DEC_PART;
  if (tid < 64) {
    const float m = tid < n_splits ? pr[tid * LS_DEC_PART + 16 * 128 + h] : -INFINITY;
    const float l = tid < n_splits ? pr[tid * LS_DEC_PART + 16 * 128 + 16 + h] : 0.f;
    float M = m;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) M = fmaxf(M, ls_shfl_xor(M, o));
    const float wt = m == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m - M);
    float L = wt * l;
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += ls_shfl_xor(L, o);
    const float inv = L > 0.f ? 1.f / L : 0.f;
    if (tid < n_splits) s_w[tid] = wt * inv;
    if (tid == 0) s_lse = L > 0.f ? (M + __log2f(L)) * 0.69314718055994531f : INFINITY;
  }
  __syncthreads();
  for (int d = tid; d < D; d += 128) {
    float acc = 0.f;
    for (int sp = 0; sp < n_splits; ++sp) acc += s_w[sp] * pr[sp * LS_DEC_PART + h * 128 + d];
    out[(t * G + g) * (int64_t)gs * D + (int64_t)h * D + d] = LsElem<DT>::from_f(acc);
  }
  if (lse && tid == 0) lse[((int64_t)g * gs + h) * total_q + t] = s_lse;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
extern "C" int ls_kvcache_append(void* k_cache, void* v_cache, int64_t cache_batch_stride,
                                 int64_t cache_row_stride, const int32_t* cache_seqlens,
                                 const void* k_new, const void* v_new, int64_t new_row_stride,
                                 const int32_t* cu_seqlens_new, int64_t total_new, int32_t batch,
                                 int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                 void* kc_cache, int64_t kc_batch_stride, int64_t kc_row_stride,
                                 int64_t max_new_windows, int32_t kernel_size,
                                 int32_t kernel_stride, int32_t* cu_windows, void* stream) {
  LS_REQUIRE(batch >= 0 && total_new >= 0 && num_kv_heads > 0 && head_dim > 0, LS_ERR_INVALID,
             "ls_kvcache_append: bad sizes");
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "ls_kvcache_append: the cache is bf16 or fp16");
  LS_REQUIRE(head_dim % 8 == 0 && new_row_stride % 8 == 0 && cache_row_stride % 8 == 0 &&
                 cache_batch_stride % 8 == 0,
             LS_ERR_UNSUPPORTED, "ls_kvcache_append: head_dim and strides must be multiples of 8");
  LS_REQUIRE(cache_seqlens && cu_seqlens_new, LS_ERR_INVALID, "ls_kvcache_append: null lengths");
  hipStream_t s = (hipStream_t)stream;
  if (total_new > 0 && batch > 0) {
    LS_REQUIRE(k_cache && v_cache && k_new && v_new, LS_ERR_INVALID,
               "ls_kvcache_append: null tensor");
    LS_REQUIRE(ls_aligned16(k_cache) && ls_aligned16(v_cache) && ls_aligned16(k_new) &&
                   ls_aligned16(v_new),
               LS_ERR_UNSUPPORTED, "ls_kvcache_append: tensors must be 16-byte aligned");
    const int64_t threads = total_new * num_kv_heads * (head_dim / 8);
    hipLaunchKernelGGL(ls_cache_append_kernel, dim3((unsigned)((threads + 255) / 256)),
                       dim3(256), 0, s, (uint16_t*)k_cache, (uint16_t*)v_cache,
                       cache_batch_stride, cache_row_stride, cache_seqlens,
                       (const uint16_t*)k_new, (const uint16_t*)v_new, new_row_stride,
                       cu_seqlens_new, total_new, batch, num_kv_heads, head_dim);
    int rc = ls_check_launch("ls_cache_append_kernel");
    if (rc) return rc;
  }
  if (!kc_cache || batch == 0) return LS_OK;
  LS_REQUIRE(kernel_size > 0 && kernel_stride > 0, LS_ERR_INVALID,
             "ls_kvcache_append: kernel_size and kernel_stride must be positive");
  LS_REQUIRE(cu_windows, LS_ERR_INVALID, "ls_kvcache_append: null cu_windows");
  LS_REQUIRE(ls_aligned16(kc_cache) && kc_row_stride % 8 == 0 && kc_batch_stride % 8 == 0,
             LS_ERR_UNSUPPORTED, "ls_kvcache_append: compressed cache must be 16-byte aligned");
  hipLaunchKernelGGL(ls_cache_window_plan_kernel, dim3(1), dim3(64), 0, s, cache_seqlens,
                     cu_seqlens_new, batch, kernel_size, kernel_stride, cu_windows);
  int rc = ls_check_launch("ls_cache_window_plan_kernel");
  if (rc || max_new_windows <= 0) return rc;
  const int64_t threads = max_new_windows * num_kv_heads * (head_dim / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_cache_compress_kernel<LS_BF16>, grid, dim3(256), 0, s,
                       (const uint16_t*)k_cache, cache_batch_stride, cache_row_stride,
                       cache_seqlens, cu_windows, batch, num_kv_heads, head_dim, kernel_size,
                       kernel_stride, (uint16_t*)kc_cache, kc_batch_stride, kc_row_stride,
                       max_new_windows);
  else
    hipLaunchKernelGGL(ls_cache_compress_kernel<LS_F16>, grid, dim3(256), 0, s,
                       (const uint16_t*)k_cache, cache_batch_stride, cache_row_stride,
                       cache_seqlens, cu_windows, batch, num_kv_heads, head_dim, kernel_size,
                       kernel_stride, (uint16_t*)kc_cache, kc_batch_stride, kc_row_stride,
                       max_new_windows);
  return ls_check_launch("ls_cache_compress_kernel");
}

namespace {
struct SelWs {
  size_t x, part, pooled, total;
  int64_t ncpad;
  int n_chunks;
};
SelWs sel_ws(int64_t total_q, int G, int64_t max_kc, int64_t out_len) {
  SelWs w;
  w.n_chunks = (int)((max_kc + 63) / 64);
  w.ncpad = (int64_t)w.n_chunks * 64;
  size_t off = 0;
  w.x = off;
  off = ls_align256(off + 4 * (size_t)G * total_q * 16 * w.ncpad);
  w.part = off;
  off = ls_align256(off + 4 * (size_t)G * total_q * w.n_chunks * 32);
  w.pooled = off;
  off = ls_align256(off + 2 * (size_t)G * total_q * out_len);
  w.total = off;
  return w;
}
}  // namespace

extern "C" size_t ls_decode_select_workspace_size(int64_t total_q, int32_t batch,
                                                  int32_t num_kv_heads, int64_t max_kc,
                                                  int64_t out_len) {
  (void)batch;
  return sel_ws(total_q, num_kv_heads, max_kc, out_len).total;
}

extern "C" int ls_decode_select(const void* q, int64_t q_row_stride, const int32_t* cu_seqlens_q,
                                int64_t total_q, const void* kc_cache, int64_t kc_batch_stride,
                                int64_t kc_row_stride, const int32_t* cache_seqlens, int32_t batch,
                                int64_t max_kc, int32_t num_heads, int32_t num_kv_heads,
                                int32_t head_dim, int32_t dtype, float softmax_scale, int32_t topk,
                                int32_t block_size, int32_t kernel_size, int32_t kernel_stride,
                                int32_t init_blocks, int32_t local_blocks, int64_t out_len,
                                int32_t take, int32_t* topk_idx, void* ws, size_t ws_bytes,
                                void* stream) {
  LS_REQUIRE(batch > 0 && total_q >= 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             LS_ERR_INVALID, "ls_decode_select: bad sizes");
  const int gs = num_heads / num_kv_heads;
  LS_REQUIRE(head_dim == 128 && gs >= 1 && gs <= 16, LS_ERR_UNSUPPORTED,
             "ls_decode_select: head_dim 128 and at most 16 query heads per KV head");
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "ls_decode_select: bf16 or fp16 queries");
  LS_REQUIRE(block_size > 0 && kernel_stride > 0 && block_size % kernel_stride == 0 &&
                 kernel_size > 0,
             LS_ERR_INVALID, "ls_decode_select: bad page geometry");
  LS_REQUIRE(out_len >= 1 && take >= 1 && take <= out_len && take <= topk, LS_ERR_INVALID,
             "ls_decode_select: need 1 <= take <= min(topk, out_len)");
  LS_REQUIRE(out_len <= LS_DEC_TOPK_MAX_PAGES, LS_ERR_UNSUPPORTED,
             "ls_decode_select: at most %d pages per row (got %lld)", LS_DEC_TOPK_MAX_PAGES,
             (long long)out_len);
  LS_REQUIRE(max_kc >= 0 && total_q <= 0x7fffffffLL && num_kv_heads <= 65535, LS_ERR_INVALID,
             "ls_decode_select: bad sizes");
  LS_REQUIRE(q_row_stride % 8 == 0 && kc_row_stride == (int64_t)num_kv_heads * head_dim &&
                 kc_batch_stride % 8 == 0,
             LS_ERR_UNSUPPORTED,
             "ls_decode_select: query rows must be 16-byte aligned and compressed-cache rows dense");
  if (total_q == 0) return LS_OK;
  LS_REQUIRE(q && cu_seqlens_q && cache_seqlens && topk_idx && ws, LS_ERR_INVALID,
             "ls_decode_select: null pointer");
  LS_REQUIRE(max_kc == 0 || kc_cache, LS_ERR_INVALID, "ls_decode_select: null compressed cache");
  const int sp = block_size / kernel_stride;
  LS_REQUIRE(sp <= 256, LS_ERR_UNSUPPORTED,
             "ls_decode_select: at most 256 compressed keys per page (got %d)", sp);
  const SelWs L = sel_ws(total_q, num_kv_heads, max_kc, out_len);
  LS_REQUIRE(ws_bytes >= L.total, LS_ERR_WORKSPACE, "ls_decode_select: workspace %zu < %zu",
             ws_bytes, L.total);
  uint8_t* w = (uint8_t*)ws;
  float* x = (float*)(w + L.x);
  float* part = (float*)(w + L.part);
  uint16_t* pooled = (uint16_t*)(w + L.pooled);
  hipStream_t s = (hipStream_t)stream;
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  int rc;
  if (max_kc > 0) {
    const dim3 g1((unsigned)L.n_chunks, (unsigned)total_q, num_kv_heads);
    if (dtype == LS_BF16)
      hipLaunchKernelGGL(ls_stage1_chunk_kernel<LS_BF16>, g1, dim3(64), 0, s, (const uint16_t*)q,
                         q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)kc_cache,
                         kc_batch_stride, kc_row_stride, cache_seqlens, kernel_size,
                         kernel_stride, max_kc, gs, head_dim, scale_log2, L.ncpad, L.n_chunks, x,
                         part);
    else
      hipLaunchKernelGGL(ls_stage1_chunk_kernel<LS_F16>, g1, dim3(64), 0, s, (const uint16_t*)q,
                         q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)kc_cache,
                         kc_batch_stride, kc_row_stride, cache_seqlens, kernel_size,
                         kernel_stride, max_kc, gs, head_dim, scale_log2, L.ncpad, L.n_chunks, x,
                         part);
    rc = ls_check_launch("ls_stage1_chunk_kernel");
    if (rc) return rc;
  }
  const int ppb = 256 / sp;
  const dim3 g2((unsigned)((out_len + ppb - 1) / ppb), (unsigned)total_q, num_kv_heads);
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_stage1_pool_kernel<LS_BF16>, g2, dim3(256), 0, s, x, part, cu_seqlens_q,
                       batch, total_q, cache_seqlens, kernel_size, kernel_stride, max_kc, gs,
                       L.ncpad, L.n_chunks, sp, ppb, out_len, block_size, init_blocks,
                       local_blocks, pooled);
  else
    hipLaunchKernelGGL(ls_stage1_pool_kernel<LS_F16>, g2, dim3(256), 0, s, x, part, cu_seqlens_q,
                       batch, total_q, cache_seqlens, kernel_size, kernel_stride, max_kc, gs,
                       L.ncpad, L.n_chunks, sp, ppb, out_len, block_size, init_blocks,
                       local_blocks, pooled);
  rc = ls_check_launch("ls_stage1_pool_kernel");
  if (rc) return rc;
  // Rows of up to 8192 pages: one wave per row; longer rows: one workgroup
  // per row with the keys in LDS.
  if (out_len > 256 && out_len <= 4 * 64 * 16 && take <= 128) {
    // Four waves per row.
    const dim3 gr((unsigned)((int64_t)num_kv_heads * total_q));
    auto go = [&](auto nsw) {
      hipLaunchKernelGGL((ls_decode_topk_wg_kernel<decltype(nsw)::value>), gr, dim3(256), 0, s,
                         pooled, cu_seqlens_q, batch, total_q, num_kv_heads, cache_seqlens,
                         (int)out_len, block_size, take, topk_idx);
    };
    const int nsw = (int)((out_len + 255) / 256);
    if (nsw <= 2) go(std::integral_constant<int, 2>());
    else if (nsw <= 4) go(std::integral_constant<int, 4>());
    else if (nsw <= 8) go(std::integral_constant<int, 8>());
    else go(std::integral_constant<int, 16>());
    return ls_check_launch("ls_decode_topk_wg_kernel");
  }
  if (out_len <= 8192) {
    const dim3 gw((unsigned)(((int64_t)num_kv_heads * total_q + 3) / 4));
    auto go = [&](auto kpl) {
      hipLaunchKernelGGL((ls_decode_topk_wave_kernel<decltype(kpl)::value>), gw, dim3(256), 0, s,
                         pooled, cu_seqlens_q, batch, total_q, num_kv_heads, cache_seqlens,
                         (int)out_len, block_size, take, topk_idx);
    };
    if (out_len <= 256) go(std::integral_constant<int, 4>());
    else if (out_len <= 1024) go(std::integral_constant<int, 16>());
    else if (out_len <= 2048) go(std::integral_constant<int, 32>());
    else if (out_len <= 4096) go(std::integral_constant<int, 64>());
    else go(std::integral_constant<int, 128>());
    return ls_check_launch("ls_decode_topk_wave_kernel");
  }
  const size_t key_bytes = ((size_t)out_len * 2 + 3) & ~(size_t)3;
  hipLaunchKernelGGL(ls_decode_topk_kernel, dim3((unsigned)total_q, num_kv_heads), dim3(256),
                     key_bytes, s, pooled, cu_seqlens_q, batch, total_q, cache_seqlens,
                     (int)out_len, block_size, take, topk_idx);
  return ls_check_launch("ls_decode_topk_kernel");
}

extern "C" size_t ls_sparse_attn_kvcache_workspace_size(int64_t total_q, int32_t num_kv_heads,
                                                        int32_t n_splits) {
  return ls_align256(4 * (size_t)total_q * num_kv_heads * (n_splits > 0 ? n_splits : 1) *
                     LS_DEC_PART);
}

extern "C" int ls_sparse_attn_kvcache(const void* q, int64_t q_row_stride,
                                      const int32_t* cu_seqlens_q, int64_t total_q,
                                      const void* k_cache, const void* v_cache,
                                      int64_t cache_batch_stride, int64_t cache_row_stride,
                                      const int32_t* cache_seqlens, int32_t batch,
                                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                      int32_t dtype, const int32_t* topk_idx, int32_t topk,
                                      float softmax_scale, int32_t causal, int32_t n_splits,
                                      void* out, float* softmax_lse, void* ws, size_t ws_bytes,
                                      void* stream) {
  LS_REQUIRE(batch > 0 && total_q >= 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0,
             LS_ERR_INVALID, "ls_sparse_attn_kvcache: bad sizes");
  const int gs = num_heads / num_kv_heads;
  LS_REQUIRE(head_dim == 128 && gs >= 1 && gs <= 16, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_kvcache: head_dim 128 and at most 16 query heads per KV head");
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_kvcache: bf16 or fp16");
  LS_REQUIRE(topk >= 1 && n_splits >= 1 && n_splits <= LS_DEC_MAX_SPLITS, LS_ERR_INVALID,
             "ls_sparse_attn_kvcache: need topk >= 1 and 1 <= n_splits <= %d", LS_DEC_MAX_SPLITS);
  LS_REQUIRE(topk <= 64 * LS_DEC_ID_REGS, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_kvcache: at most %d plan ids per row (got %d)", 64 * LS_DEC_ID_REGS,
             topk);
  LS_REQUIRE(total_q <= 0x7fffffffLL && num_kv_heads <= 65535, LS_ERR_INVALID,
             "ls_sparse_attn_kvcache: too many rows or heads");
  LS_REQUIRE(q_row_stride % 8 == 0 && cache_row_stride % 8 == 0 && cache_batch_stride % 8 == 0,
             LS_ERR_UNSUPPORTED, "ls_sparse_attn_kvcache: strides must be multiples of 8");
  if (total_q == 0) return LS_OK;
  LS_REQUIRE(q && k_cache && v_cache && cu_seqlens_q && cache_seqlens && topk_idx && out && ws,
             LS_ERR_INVALID, "ls_sparse_attn_kvcache: null pointer");
  LS_REQUIRE(ls_aligned16(q) && ls_aligned16(k_cache) && ls_aligned16(v_cache), LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_kvcache: tensors must be 16-byte aligned");
  const size_t need = ls_sparse_attn_kvcache_workspace_size(total_q, num_kv_heads, n_splits);
  LS_REQUIRE(ws_bytes >= need, LS_ERR_WORKSPACE, "ls_sparse_attn_kvcache: workspace %zu < %zu",
             ws_bytes, need);
  // Four waves per split, ppw plan slots per wave.
  const int ppw = (topk + 4 * n_splits - 1) / (4 * n_splits);
  const int splits = (topk + 4 * ppw - 1) / (4 * ppw);
  hipStream_t s = (hipStream_t)stream;
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  float* part = (float*)ws;
  const dim3 grid((unsigned)splits, (unsigned)total_q, num_kv_heads);
  const dim3 cgrid((unsigned)total_q, num_kv_heads, gs);
  if (dtype == LS_BF16) {
    hipLaunchKernelGGL(ls_decode_attn_kernel<LS_BF16>, grid, dim3(256), 0, s, (const uint16_t*)q,
                       q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)k_cache,
                       (const uint16_t*)v_cache, cache_batch_stride, cache_row_stride,
                       cache_seqlens, gs, head_dim, topk_idx, topk, ppw, splits, scale_log2,
                       causal, part);
    int rc = ls_check_launch("ls_decode_attn_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(ls_decode_combine_kernel<LS_BF16>, cgrid, dim3(128), 0, s, part, total_q,
                       gs, head_dim, splits, (uint16_t*)out, softmax_lse);
  } else {
    hipLaunchKernelGGL(ls_decode_attn_kernel<LS_F16>, grid, dim3(256), 0, s, (const uint16_t*)q,
                       q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)k_cache,
                       (const uint16_t*)v_cache, cache_batch_stride, cache_row_stride,
                       cache_seqlens, gs, head_dim, topk_idx, topk, ppw, splits, scale_log2,
                       causal, part);
    int rc = ls_check_launch("ls_decode_attn_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(ls_decode_combine_kernel<LS_F16>, cgrid, dim3(128), 0, s, part, total_q,
                       gs, head_dim, splits, (uint16_t*)out, softmax_lse);
  }
  return ls_check_launch("ls_decode_combine_kernel");
}

extern "C" size_t ls_stage1_scores_workspace_size(int64_t total_q, int32_t num_kv_heads,
                                                  int64_t max_kc) {
  return sel_ws(total_q, num_kv_heads, max_kc, 0).total;
}

extern "C" int ls_stage1_scores(const void* q, int64_t q_row_stride, const int32_t* cu_seqlens_q,
                                int64_t total_q, const void* kc, int64_t kc_row_stride,
                                const int32_t* cu_seqlens_kc, int32_t batch, int64_t max_kc,
                                int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                int32_t dtype, float softmax_scale, void* out, int64_t out_cols,
                                void* ws, size_t ws_bytes, void* stream) {
  LS_REQUIRE(batch > 0 && total_q >= 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0 &&
                 max_kc >= 0 && out_cols >= 0,
             LS_ERR_INVALID, "ls_stage1_scores: bad sizes");
  const int gs = num_heads / num_kv_heads;
  LS_REQUIRE(head_dim == 128 && gs >= 1 && gs <= 16, LS_ERR_UNSUPPORTED,
             "ls_stage1_scores: head_dim 128 and at most 16 query heads per KV head");
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "ls_stage1_scores: bf16 or fp16 queries");
  LS_REQUIRE(total_q <= 0x7fffffffLL && num_kv_heads <= 65535, LS_ERR_INVALID,
             "ls_stage1_scores: bad sizes");
  LS_REQUIRE(q_row_stride % 8 == 0 && kc_row_stride % 8 == 0, LS_ERR_UNSUPPORTED,
             "ls_stage1_scores: query and key rows must be 16-byte aligned");
  if (total_q == 0 || out_cols == 0) return LS_OK;
  LS_REQUIRE(q && cu_seqlens_q && cu_seqlens_kc && out && ws && (max_kc == 0 || kc),
             LS_ERR_INVALID, "ls_stage1_scores: null pointer");
  const SelWs L = sel_ws(total_q, num_kv_heads, max_kc, 0);
  LS_REQUIRE(ws_bytes >= L.total, LS_ERR_WORKSPACE, "ls_stage1_scores: workspace %zu < %zu",
             ws_bytes, L.total);
  uint8_t* w = (uint8_t*)ws;
  float* x = (float*)(w + L.x);
  float* part = (float*)(w + L.part);
  hipStream_t s = (hipStream_t)stream;
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  int rc;
  if (max_kc > 0) {
    const dim3 g1((unsigned)L.n_chunks, (unsigned)total_q, num_kv_heads);
    if (dtype == LS_BF16)
      hipLaunchKernelGGL((ls_stage1_chunk_kernel<LS_BF16, true>), g1, dim3(64), 0, s,
                         (const uint16_t*)q, q_row_stride, cu_seqlens_q, batch, total_q,
                         (const uint16_t*)kc, (int64_t)0, kc_row_stride, cu_seqlens_kc, 0, 1,
                         max_kc, gs, head_dim, scale_log2, L.ncpad, L.n_chunks, x, part);
    else
      hipLaunchKernelGGL((ls_stage1_chunk_kernel<LS_F16, true>), g1, dim3(64), 0, s,
                         (const uint16_t*)q, q_row_stride, cu_seqlens_q, batch, total_q,
                         (const uint16_t*)kc, (int64_t)0, kc_row_stride, cu_seqlens_kc, 0, 1,
                         max_kc, gs, head_dim, scale_log2, L.ncpad, L.n_chunks, x, part);
    if ((rc = ls_check_launch("ls_stage1_chunk_kernel"))) return rc;
  }
  const dim3 g2((unsigned)total_q, num_kv_heads);
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_stage1_scores_kernel<LS_BF16>, g2, dim3(256), 0, s, x, part,
                       cu_seqlens_q, batch, total_q, cu_seqlens_kc, max_kc, gs, L.ncpad,
                       L.n_chunks, out_cols, (uint16_t*)out);
  else
    hipLaunchKernelGGL(ls_stage1_scores_kernel<LS_F16>, g2, dim3(256), 0, s, x, part,
                       cu_seqlens_q, batch, total_q, cu_seqlens_kc, max_kc, gs, L.ncpad,
                       L.n_chunks, out_cols, (uint16_t*)out);
  return ls_check_launch("ls_stage1_scores_kernel");
}
