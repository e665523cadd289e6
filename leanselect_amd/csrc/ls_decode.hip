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
#include "ls_common.h"

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
  auto add_rows = [&](int r0, int r1, float (&s)[8]) {
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
//   score[g][t][j] = sum_{h in g} softmax_j(scale * q[t][h] . kc[b][j][g])
// over the n_c(b) compressed keys of the sequence (no causal limit: the
// reference calls stage 1 with causal=False when decoding), rounded to the
// query dtype and then to bf16 (compressed_attention's .to(bfloat16)).
// Columns n_c(b) <= j < max_kc are written as 0.
//
// Pass 1 (one wave per 64-key chunk, row and group): S^T = Kc . Q^T on the
// 16x16x32 MFMA (keys are rows, the group's heads columns); the raw scores in
// base-2 units go to the workspace with each head's chunk maximum and
// sum of 2^(x - max).  Pass 2 (one workgroup per row and group): each head's
// log2-sum-exp from the chunk partials, then the group sums per key.
// ---------------------------------------------------------------------------
// cu_kc[b] = sum_{b' < b} n_c(b') over the sequences' current lengths;
// cache_lens[b] = len_b - len_q(b), the tokens before the sequence's rows.
__global__ void ls_decode_plan_kernel(const int32_t* __restrict__ cache_seqlens,
                                      const int32_t* __restrict__ cu_q, int batch, int ks,
                                      int stride, int32_t* __restrict__ cu_kc,
                                      int32_t* __restrict__ cache_lens) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t acc = 0;
  cu_kc[0] = 0;
  for (int b = 0; b < batch; ++b) {
    acc += (int32_t)ls_n_windows(cache_seqlens[b], ks, stride);
    cu_kc[b + 1] = acc;
    cache_lens[b] = cache_seqlens[b] - (cu_q[b + 1] - cu_q[b]);
  }
}

// x[g][t][h][j] (float, base-2 units, -inf past n_c), part[g][t][c][h] = (max, sum).
template <int DT>
__global__ __launch_bounds__(64) void ls_stage1_chunk_kernel(
    const uint16_t* __restrict__ q, int64_t qrs, const int32_t* __restrict__ cu_q, int batch,
    int64_t total_q, const uint16_t* __restrict__ kcc, int64_t kbs, int64_t krs,
    const int32_t* __restrict__ cu_kc, int gs, int D, float scale_log2, int64_t ncpad,
    int n_chunks, float* __restrict__ x, float* __restrict__ part) {
  const int c = LS_BID_X;
  const int64_t t = LS_BID_Y;
  const int g = LS_BID_Z;
  const int lane = LS_TID, r = lane & 15, qg = lane >> 4;
  const int b = ls_find_segment(cu_q, batch, t);
  const int nc = cu_kc[b + 1] - cu_kc[b];
  float* xrow = x + ((int64_t)g * total_q + t) * 16 * ncpad;
  float* prow = part + (((int64_t)g * total_q + t) * n_chunks + c) * 32;
  // Q^T fragments (B operand): lane (r, qg) holds head r, dims 32 ks + 8 qg + 0..7.
  ls_u32x4 qf[4];
  const bool head_ok = r < gs;
  const uint16_t* qrow = q + t * qrs + ((int64_t)g * gs + r) * D + 8 * qg;
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = head_ok ? ls_load16(qrow + 32 * ks) : ls_u32x4{0u, 0u, 0u, 0u};
  float m = -INFINITY;
  float sv[16];
#pragma unroll
  for (int kb = 0; kb < 4; ++kb) {
    const int j = 64 * c + 16 * kb + r;  // key row of this lane's A fragment
    ls_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    const bool key_ok = j < nc;
    const uint16_t* krow = kcc + (int64_t)b * kbs + (int64_t)j * krs + (int64_t)g * D + 8 * qg;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const ls_u32x4 kf = key_ok ? ls_load16(krow + 32 * ks) : ls_u32x4{0u, 0u, 0u, 0u};
      acc = LsElem<DT>::mfma(kf, qf[ks], acc);
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

template <int DT>
__global__ __launch_bounds__(256) void ls_stage1_finish_kernel(
    const float* __restrict__ x, const float* __restrict__ part, const int32_t* __restrict__ cu_q,
    int batch, int64_t total_q, const int32_t* __restrict__ cu_kc, int gs, int64_t ncpad,
    int n_chunks, int64_t max_kc, uint16_t* __restrict__ score) {
  const int64_t t = LS_BID_X;
  const int g = LS_BID_Y;
  const int tid = LS_TID;
  __shared__ float s_lse[16];
  const int b = ls_find_segment(cu_q, batch, t);
  const int nc = cu_kc[b + 1] - cu_kc[b];
  const int nch = (nc + 63) / 64;
  const float* prow = part + ((int64_t)g * total_q + t) * n_chunks * 32;
  {
    // Sixteen consecutive threads per head (four heads per wave) reduce the
    // head's chunk partials: each a strided share, then butterfly shuffles.
    const int h = tid >> 4, part = tid & 15;
    float M = -INFINITY;
    if (h < gs)
      for (int c = part; c < nch; c += 16) M = fmaxf(M, prow[c * 32 + 2 * h]);
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) M = fmaxf(M, ls_shfl_xor(M, o));
    float L = 0.f;
    if (h < gs && M != -INFINITY)
      for (int c = part; c < nch; c += 16) {
        const float mc = prow[c * 32 + 2 * h];
        if (mc != -INFINITY) L += prow[c * 32 + 2 * h + 1] * __builtin_amdgcn_exp2f(mc - M);
      }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) L += ls_shfl_xor(L, o);
    if (h < gs && part == 0) s_lse[h] = M + __log2f(L);
  }
  __syncthreads();
  const float* xrow = x + ((int64_t)g * total_q + t) * 16 * ncpad;
  uint16_t* orow = score + ((int64_t)g * total_q + t) * max_kc;
  for (int64_t j = tid; j < max_kc; j += 256) {
    uint16_t o = 0;
    if (j < nc) {
      float s = 0.f;
      for (int h = 0; h < gs; ++h) s += __builtin_amdgcn_exp2f(xrow[(int64_t)h * ncpad + j] - s_lse[h]);
      if constexpr (DT == LS_F16)
        o = ls_f32_to_bf16(ls_f16_to_f32(ls_f32_to_f16(s)));
      else
        o = ls_f32_to_bf16(s);
    }
    orow[j] = o;
  }
}

// ---------------------------------------------------------------------------
// Decode top-k over pooled page scores pooled[g][t][out_len] (bf16, forced
// pages +inf, pages past the row's own -inf): the `take` best pages (ties to
// the lower page), ascending, ids past the row's page q_idx replaced by -1
// (they sort last, so the list is the kept ids then -1 padding).  One
// workgroup per (row, group); keys (value << 16 | (65535 - page)) are unique
// and their take-th largest is found by an 8-bit radix select in four passes.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void ls_decode_topk_kernel(
    const uint16_t* __restrict__ pooled, const int32_t* __restrict__ cu_q, int batch,
    int64_t total_q, const int32_t* __restrict__ cache_lens, int out_len, int block_size,
    int take, int32_t* __restrict__ ids) {
  const int64_t t = LS_BID_X;
  const int g = LS_BID_Y;
  const int tid = LS_TID;
  __shared__ uint32_t s_hist[256];
  __shared__ uint32_t s_sel[2];  // prefix found so far, keys still needed above it
  __shared__ int32_t s_cnt[256];
  const uint16_t* row = pooled + ((int64_t)g * total_q + t) * out_len;
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t q_idx = ((int64_t)cache_lens[b] + (t - cu_q[b])) / block_size;
  auto key_of = [&](int p) -> uint32_t {
    return (ls_order_key16(row[p]) << 16) | (uint32_t)(65535 - p);
  };
  if (tid == 0) {
    s_sel[0] = 0u;
    s_sel[1] = (uint32_t)take;
  }
  for (int pass = 3; pass >= 0; --pass) {
    s_hist[tid] = 0u;
    __syncthreads();
    const uint32_t prefix = s_sel[0];
    const uint32_t hi_mask = pass == 3 ? 0u : (0xffffffffu << (8 * (pass + 1)));
    for (int p = tid; p < out_len; p += 256) {
      const uint32_t k = key_of(p);
      if ((k & hi_mask) == (prefix & hi_mask)) atomicAdd(&s_hist[(k >> (8 * pass)) & 255u], 1u);
    }
    __syncthreads();
    if (tid == 0) {
      uint32_t need = s_sel[1], acc = 0u;
      int d = 255;
      for (; d > 0; --d) {
        if (acc + s_hist[d] >= need) break;
        acc += s_hist[d];
      }
      s_sel[0] = prefix | ((uint32_t)d << (8 * pass));
      s_sel[1] = need - acc;
    }
    __syncthreads();
  }
  const uint32_t T = s_sel[0];  // the take-th largest key
  // Ordered compaction of the kept pages (key >= T, page <= q_idx).
  const int per = (out_len + 255) / 256;
  const int p0 = tid * per, p1 = min(out_len, p0 + per);
  int cnt = 0;
  for (int p = p0; p < p1; ++p) cnt += (key_of(p) >= T && p <= q_idx) ? 1 : 0;
  s_cnt[tid] = cnt;
  __syncthreads();
  for (int off = 1; off < 256; off <<= 1) {  // inclusive scan
    const int v = tid >= off ? s_cnt[tid - off] : 0;
    __syncthreads();
    s_cnt[tid] += v;
    __syncthreads();
  }
  int pos = s_cnt[tid] - cnt;
  const int kept = s_cnt[255];
  int32_t* orow = ids + ((int64_t)g * total_q + t) * take;
  for (int p = p0; p < p1; ++p)
    if (key_of(p) >= T && p <= q_idx) orow[pos++] = p;
  for (int i = kept + tid; i < take; i += 256) orow[i] = -1;
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
  for (int ks = 0; ks < 4; ++ks)
    qf[ks] = head_ok ? ls_load16(qrow + 32 * ks) : ls_u32x4{0u, 0u, 0u, 0u};
  float m_run = -INFINITY, l_run = 0.f;
  ls_f32x4 o[8];
#pragma unroll
  for (int db = 0; db < 8; ++db) o[db] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
  const int32_t* idrow = topk_idx + ((int64_t)g * total_q + t) * topk;
  const uint16_t* kseq = kc_ + (int64_t)b * cbs + (int64_t)g * D;
  const uint16_t* vseq = vc_ + (int64_t)b * cbs + (int64_t)g * D;
  const int slot0 = (4 * s + w) * ppw, slot1 = min(topk, slot0 + ppw);
  for (int slot = slot0; slot < slot1; ++slot) {
    const int id = idrow[slot];
    if (id < 0 || (int64_t)id >= n_pages || 64LL * id >= limit) continue;
    // Skip a repeated id (the reference forms a page bitmask, so each page counts once).
    bool dup = false;
    for (int j0 = 0; j0 < slot; j0 += 64) {
      const int j = j0 + lane;
      dup |= __ballot(j < slot && idrow[j] == id) != 0ull;
    }
    if (dup) continue;
    const int64_t key0 = 64LL * id;
    const int64_t nvis = min((int64_t)64, limit - key0);  // visible keys of this page (> 0)
    // Stage V (keys past nvis as zeros) into the wave's LDS, rows of 128 values.
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int ci = it * 64 + lane, kr = ci >> 4, c16 = ci & 15;
      ls_u32x4 v = {0u, 0u, 0u, 0u};
      if (kr < nvis) v = ls_load16(vseq + (key0 + kr) * crs + 8 * c16);
      uint32_t* dst = reinterpret_cast<uint32_t*>(sv_w + kr * LS_DEC_VPITCH + 16 * c16);
      dst[0] = v[0];
      dst[1] = v[1];
      dst[2] = v[2];
      dst[3] = v[3];
    }
    // Scores: key block kb = 2 c + nb, MFMA row R holds key 32 c + 8 (R / 4) + 4 nb + R % 4.
    float sv[16];
    float pm = -INFINITY;
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int cch = kb >> 1, nb = kb & 1;
      const int krow = 32 * cch + 8 * (r >> 2) + 4 * nb + (r & 3);
      const bool kin = krow < nvis;
      const uint16_t* kp = kseq + (key0 + krow) * crs + 8 * qg;
      ls_f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const ls_u32x4 kf = kin ? ls_load16(kp + 32 * ks) : ls_u32x4{0u, 0u, 0u, 0u};
        acc = LsElem<DT>::mfma(kf, qf[ks], acc);
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = 32 * cch + 8 * qg + 4 * nb + i;  // row 4 qg + i of block kb
        const float v = key < nvis ? acc[i] * scale_log2 : -INFINITY;
        sv[4 * kb + i] = v;
        pm = fmaxf(pm, v);
      }
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
// without a visible key give zeros and lse = +inf.  The splits' weights are
// formed once per head in LDS; each output is then a sum of independent loads.
template <int DT>
__global__ __launch_bounds__(256) void ls_decode_combine_kernel(
    const float* __restrict__ part, int64_t total_q, int gs, int D, int n_splits,
    uint16_t* __restrict__ out, float* __restrict__ lse) {
  const int64_t t = LS_BID_X;
  const int g = LS_BID_Y;
  const int tid = LS_TID;
  const int G = gridDim.y;
  __shared__ float s_w[LS_DEC_MAX_SPLITS][16];
  __shared__ float s_m[LS_DEC_MAX_SPLITS][16];
  __shared__ float s_l[LS_DEC_MAX_SPLITS][16];
  __shared__ float s_lse[16];
  const float* pr = part + ((int64_t)g * total_q + t) * n_splits * LS_DEC_PART;
  for (int i = tid; i < n_splits * 16; i += 256) {
    const int sp = i >> 4, h = i & 15;
    s_m[sp][h] = pr[sp * LS_DEC_PART + 16 * 128 + h];
    s_l[sp][h] = pr[sp * LS_DEC_PART + 16 * 128 + 16 + h];
  }
  __syncthreads();
  if (tid < 16) {
    float M = -INFINITY;
    for (int sp = 0; sp < n_splits; ++sp) M = fmaxf(M, s_m[sp][tid]);
    float L = 0.f;
    for (int sp = 0; sp < n_splits; ++sp) {
      const float wt = s_m[sp][tid] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s_m[sp][tid] - M);
      s_w[sp][tid] = wt;
      L += wt * s_l[sp][tid];
    }
    const float inv = L > 0.f ? 1.f / L : 0.f;
    for (int sp = 0; sp < n_splits; ++sp) s_w[sp][tid] *= inv;
    s_lse[tid] = L > 0.f ? (M + __log2f(L)) * 0.69314718055994531f : INFINITY;
  }
  __syncthreads();
  for (int e = tid; e < gs * 128; e += 256) {
    const int h = e >> 7, d = e & 127;
    float acc = 0.f;
    for (int sp = 0; sp < n_splits; ++sp) acc += s_w[sp][h] * pr[sp * LS_DEC_PART + h * 128 + d];
    out[(t * G + g) * (int64_t)gs * D + (int64_t)h * D + d] = LsElem<DT>::from_f(acc);
    if (lse && d == 0) lse[((int64_t)g * gs + h) * total_q + t] = s_lse[h];
  }
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
  size_t cu_kc, cache_lens, x, part, score, pooled, total;
  int64_t ncpad;
  int n_chunks;
};
SelWs sel_ws(int64_t total_q, int batch, int G, int64_t max_kc, int64_t out_len) {
  SelWs w;
  w.n_chunks = (int)((max_kc + 63) / 64);
  w.ncpad = (int64_t)w.n_chunks * 64;
  size_t off = 0;
  w.cu_kc = off;
  off = ls_align256(off + 4 * (size_t)(batch + 1));
  w.cache_lens = off;
  off = ls_align256(off + 4 * (size_t)(batch + 1));
  w.x = off;
  off = ls_align256(off + 4 * (size_t)G * total_q * 16 * w.ncpad);
  w.part = off;
  off = ls_align256(off + 4 * (size_t)G * total_q * w.n_chunks * 32);
  w.score = off;
  off = ls_align256(off + 2 * (size_t)G * total_q * max_kc);
  w.pooled = off;
  off = ls_align256(off + 2 * (size_t)G * total_q * out_len);
  w.total = off;
  return w;
}
}  // namespace

extern "C" size_t ls_decode_select_workspace_size(int64_t total_q, int32_t batch,
                                                  int32_t num_kv_heads, int64_t max_kc,
                                                  int64_t out_len) {
  return sel_ws(total_q, batch, num_kv_heads, max_kc, out_len).total;
}

extern "C" int ls_page_maxpool_varlen(const void* input, const int32_t* cu_seqlens_q,
                                      const int32_t* cu_seqlens_k, const int32_t* cache_lens,
                                      int32_t batch, int32_t num_heads, int64_t total_q,
                                      int64_t max_seqlen_k, int64_t out_len, int32_t local_blocks,
                                      int32_t init_blocks, int32_t block_size, int32_t stride,
                                      int32_t dtype, void* out, void* stream);

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
  LS_REQUIRE(out_len >= 1 && out_len <= 65535 && take >= 1 && take <= out_len && take <= topk,
             LS_ERR_INVALID, "ls_decode_select: need 1 <= take <= min(topk, out_len), out_len < 65536");
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
  const SelWs L = sel_ws(total_q, batch, num_kv_heads, max_kc, out_len);
  LS_REQUIRE(ws_bytes >= L.total, LS_ERR_WORKSPACE, "ls_decode_select: workspace %zu < %zu",
             ws_bytes, L.total);
  uint8_t* w = (uint8_t*)ws;
  int32_t* cu_kc = (int32_t*)(w + L.cu_kc);
  int32_t* cache_lens = (int32_t*)(w + L.cache_lens);
  float* x = (float*)(w + L.x);
  float* part = (float*)(w + L.part);
  uint16_t* score = (uint16_t*)(w + L.score);
  uint16_t* pooled = (uint16_t*)(w + L.pooled);
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(ls_decode_plan_kernel, dim3(1), dim3(64), 0, s, cache_seqlens, cu_seqlens_q,
                     batch, kernel_size, kernel_stride, cu_kc, cache_lens);
  int rc = ls_check_launch("ls_decode_plan_kernel");
  if (rc) return rc;
  const float scale_log2 = softmax_scale * 1.4426950408889634f;
  if (max_kc > 0) {
    const dim3 g1((unsigned)L.n_chunks, (unsigned)total_q, num_kv_heads);
    const dim3 g2((unsigned)total_q, num_kv_heads);
    if (dtype == LS_BF16) {
      hipLaunchKernelGGL(ls_stage1_chunk_kernel<LS_BF16>, g1, dim3(64), 0, s, (const uint16_t*)q,
                         q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)kc_cache,
                         kc_batch_stride, kc_row_stride, cu_kc, gs, head_dim, scale_log2, L.ncpad,
                         L.n_chunks, x, part);
      rc = ls_check_launch("ls_stage1_chunk_kernel");
      if (rc) return rc;
      hipLaunchKernelGGL(ls_stage1_finish_kernel<LS_BF16>, g2, dim3(256), 0, s, x, part,
                         cu_seqlens_q, batch, total_q, cu_kc, gs, L.ncpad, L.n_chunks, max_kc,
                         score);
    } else {
      hipLaunchKernelGGL(ls_stage1_chunk_kernel<LS_F16>, g1, dim3(64), 0, s, (const uint16_t*)q,
                         q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)kc_cache,
                         kc_batch_stride, kc_row_stride, cu_kc, gs, head_dim, scale_log2, L.ncpad,
                         L.n_chunks, x, part);
      rc = ls_check_launch("ls_stage1_chunk_kernel");
      if (rc) return rc;
      hipLaunchKernelGGL(ls_stage1_finish_kernel<LS_F16>, g2, dim3(256), 0, s, x, part,
                         cu_seqlens_q, batch, total_q, cu_kc, gs, L.ncpad, L.n_chunks, max_kc,
                         score);
    }
    rc = ls_check_launch("ls_stage1_finish_kernel");
    if (rc) return rc;
  }
  rc = ls_page_maxpool_varlen(score, cu_seqlens_q, cu_kc, cache_lens, batch, num_kv_heads,
                              total_q, max_kc, out_len, local_blocks, init_blocks, block_size,
                              kernel_stride, LS_BF16, pooled, stream);
  if (rc) return rc;
  hipLaunchKernelGGL(ls_decode_topk_kernel, dim3((unsigned)total_q, num_kv_heads), dim3(256), 0,
                     s, pooled, cu_seqlens_q, batch, total_q, cache_lens, (int)out_len,
                     block_size, take, topk_idx);
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
  const dim3 cgrid((unsigned)total_q, num_kv_heads);
  if (dtype == LS_BF16) {
    hipLaunchKernelGGL(ls_decode_attn_kernel<LS_BF16>, grid, dim3(256), 0, s, (const uint16_t*)q,
                       q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)k_cache,
                       (const uint16_t*)v_cache, cache_batch_stride, cache_row_stride,
                       cache_seqlens, gs, head_dim, topk_idx, topk, ppw, splits, scale_log2,
                       causal, part);
    int rc = ls_check_launch("ls_decode_attn_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(ls_decode_combine_kernel<LS_BF16>, cgrid, dim3(256), 0, s, part, total_q,
                       gs, head_dim, splits, (uint16_t*)out, softmax_lse);
  } else {
    hipLaunchKernelGGL(ls_decode_attn_kernel<LS_F16>, grid, dim3(256), 0, s, (const uint16_t*)q,
                       q_row_stride, cu_seqlens_q, batch, total_q, (const uint16_t*)k_cache,
                       (const uint16_t*)v_cache, cache_batch_stride, cache_row_stride,
                       cache_seqlens, gs, head_dim, topk_idx, topk, ppw, splits, scale_log2,
                       causal, part);
    int rc = ls_check_launch("ls_decode_attn_kernel");
    if (rc) return rc;
    hipLaunchKernelGGL(ls_decode_combine_kernel<LS_F16>, cgrid, dim3(256), 0, s, part, total_q,
                       gs, head_dim, splits, (uint16_t*)out, softmax_lse);
  }
  return ls_check_launch("ls_decode_combine_kernel");
}
