// Block-sparse causal attention over per-token page plans (a10).
//
// Contract: infllmv2_attn_varlen_func(..., topk_idx=)
// (third_party/infllmv2/paper1.patch:1993-2100; called from
// leanselect/models/minicpm.py:3216-3244): for query row t and KV group g the
// keys are those of the valid ids in topk_idx[g, t, :] (each page once) with
// j <= t + len_k - len_q when causal; all H/G heads of the group share the plan.
//
// Design (one wave per (token, group, 16-head tile)):
//   * the plan row is turned into an ascending, duplicate-free page list with
//     an LDS bitmap (ids past the causal frontier are dropped);
//   * S^T = K . Q^T on v_mfma_f32_16x16x32: keys are MFMA rows, the 16 heads of
//     the group are columns, so each lane owns one head and the online-softmax
//     row statistics need only two cross-lane steps;
//   * K rows are permuted inside each 32-key chunk so that lane group q ends up
//     with the 8 contiguous keys base+8q..base+8q+7; P^T then feeds the second
//     MFMA (O^T = V^T . P^T) straight from registers as its B operand and V^T
//     is read as 16-byte rows of a transposed, page-aligned copy of V built by
//     ls_vt_kernel (zero-filled past each sequence end);
//   * float32 softmax in base 2; P . V runs on the fp16 MFMA (P in [0, 1]
//     keeps 10 mantissa bits instead of bf16's 7; V is staged to fp16 with an
//     exact per-page power-of-two scale that moves onto P), output rounded once.
#include "ls_common.h"

#define LS_ATTN_MAX_PAGES 8192
#define LS_ATTN_MAX_TAKE 256

__device__ __forceinline__ void ls_wave_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

__device__ __forceinline__ int ls_wave_excl_scan(int v, int lane, int* total) {
  int x = v;
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const int y = __shfl_up(x, d, LS_WAVE);
    if (lane >= d) x += y;
  }
  *total = __shfl(x, 63, LS_WAVE);
  return x - v;
}

// pg_off[b] = sum_{b' < b} ceil(len_k(b') / 64): page-aligned start of each
// sequence in the transposed V copy (in pages).
__global__ void ls_attn_plan_kernel(const int32_t* __restrict__ cu_k, int batch,
                                    int32_t* __restrict__ pg_off) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t acc = 0;
  pg_off[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int len = cu_k[b + 1] - cu_k[b];
    acc += len > 0 ? (len + 63) / 64 : 0;
    pg_off[b + 1] = acc;
  }
}

// vt[g][d][64 * pg_off[b] + j] = fp16(v[cu_k[b] + j][g][d] * 2^-e)  (0 for j >= len_k(b)),
// vexp[g * n_pages + pg_off[b] + p] = e: the smallest e >= 0 (at most 15) that keeps
// the page's scaled values within +-32768, so they are finite in fp16 (e = 0 for
// ordinary activations; bf16 values are then exact in fp16 down to 2^-14).
// One workgroup transposes one 64-key page of one group through LDS.
template <int DT, int D>
__global__ __launch_bounds__(256) void ls_vt_kernel(const uint16_t* __restrict__ v,
                                                    int64_t v_rs, const int32_t* __restrict__ cu_k,
                                                    const int32_t* __restrict__ pg_off,
                                                    int batch, int64_t lpad, int64_t n_pages,
                                                    uint16_t* __restrict__ vt,
                                                    int32_t* __restrict__ vexp) {
  constexpr int PITCH = D + 2;
  __shared__ uint16_t tile[64 * PITCH];
  __shared__ float wave_max[4];
  const int64_t tile_id = blockIdx.x;
  if (tile_id >= pg_off[batch]) return;
  const int g = blockIdx.y;
  const int b = ls_find_segment(pg_off, batch, tile_id);
  const int p = (int)(tile_id - pg_off[b]);
  const int lk = cu_k[b + 1] - cu_k[b];
  const int64_t krow0 = (int64_t)cu_k[b] + 64LL * p;
  constexpr int CH = D / 8;  // 16-byte chunks per row
  float mx = 0.f;
  for (int c = threadIdx.x; c < 64 * CH; c += 256) {
    const int key = c / CH, d0 = (c % CH) * 8;
    ls_u32x4 val = {0u, 0u, 0u, 0u};
    if (64 * p + key < lk) val = ls_load16(v + (krow0 + key) * v_rs + (int64_t)g * D + d0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t lo = (uint16_t)(val[i] & 0xffffu), hi = (uint16_t)(val[i] >> 16);
      mx = fmaxf(mx, fmaxf(fabsf(LsElem<DT>::to_f(lo)), fabsf(LsElem<DT>::to_f(hi))));
      tile[key * PITCH + d0 + 2 * i] = lo;
      tile[key * PITCH + d0 + 2 * i + 1] = hi;
    }
  }
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, LS_WAVE));
  if ((threadIdx.x & 63) == 0) wave_max[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
  int e = 0;
  while (e < 15 && mx * __builtin_ldexpf(1.f, -e) > 32768.f) ++e;
  const float scale = __builtin_ldexpf(1.f, -e);
  if (threadIdx.x == 0) vexp[(int64_t)g * n_pages + pg_off[b] + p] = e;
  const int64_t col0 = 64LL * (pg_off[b] + p);
  for (int c = threadIdx.x; c < D * 8; c += 256) {
    const int d = c / 8, k0 = (c % 8) * 8;
    ls_u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = ls_pack2(ls_f32_to_f16(LsElem<DT>::to_f(tile[(k0 + 2 * i) * PITCH + d]) * scale),
                      ls_f32_to_f16(LsElem<DT>::to_f(tile[(k0 + 2 * i + 1) * PITCH + d]) * scale));
    *reinterpret_cast<ls_u32x4*>(vt + ((int64_t)g * D + d) * lpad + col0 + k0) = o;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void ls_attn_kernel(
    const uint16_t* __restrict__ qg, int64_t q_rs, const uint16_t* __restrict__ kg,
    int64_t k_rs, const uint16_t* __restrict__ vt, int64_t lpad,
    const int32_t* __restrict__ vexp, int64_t n_pages,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
    const int32_t* __restrict__ pg_off, int batch, int64_t total_q, int G, int gs,
    const int32_t* __restrict__ topk_idx, int take, float scale_log2, int causal,
    uint16_t* __restrict__ out, float* __restrict__ lse) {
  constexpr int D = 128;
  __shared__ uint32_t s_bits[4][LS_ATTN_MAX_PAGES / 32];
  __shared__ int32_t s_list[4][LS_ATTN_MAX_TAKE];
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int64_t t = (int64_t)blockIdx.x * 4 + w;
  if (t >= total_q) return;
  const int g = blockIdx.y;
  const int head = blockIdx.z * 16 + r;  // head within the group
  const bool head_ok = head < gs;

  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t tr = t - cu_q[b];
  const int lq = cu_q[b + 1] - cu_q[b];
  const int lk = cu_k[b + 1] - cu_k[b];
  const int64_t kstart = cu_k[b];
  const int64_t vbase = 64LL * pg_off[b];
  int64_t jmax = lk - 1;
  if (causal) jmax = min(jmax, tr + (int64_t)(lk - lq));

  // ---- page list: ascending, unique, inside [0, jmax / 64] ----
  int n_list = 0;
  if (jmax >= 0) {
    // The host bounds max_seqlen_k; the clamp keeps the LDS bitmap in range
    // even when a caller understates it.
    const int last_page = (int)min(jmax / 64, (int64_t)LS_ATTN_MAX_PAGES - 1);
    const int nwords = last_page / 32 + 1;
    uint32_t* bits = s_bits[w];
    for (int i = lane; i < nwords; i += 64) bits[i] = 0u;
    ls_wave_sync();
    const int32_t* ids = topk_idx + ((int64_t)g * total_q + t) * take;
    for (int i = lane; i < take; i += 64) {
      const int p = ids[i];
      if (p >= 0 && p <= last_page) atomicOr(&bits[p >> 5], 1u << (p & 31));
    }
    ls_wave_sync();
    for (int w0 = 0; w0 < nwords; w0 += 64) {
      const int i = w0 + lane;
      uint32_t word = i < nwords ? bits[i] : 0u;
      int tot;
      int pos = n_list + ls_wave_excl_scan(__popc(word), lane, &tot);
      while (word) {
        const int bit = __ffs(word) - 1;
        word &= word - 1;
        s_list[w][pos++] = i * 32 + bit;
      }
      n_list += tot;
    }
    ls_wave_sync();
  }

  // ---- Q^T fragments (B operand): head r, channels 32ks + 8q .. +7 ----
  ls_u32x4 qf[4];
  {
    const uint16_t* qrow = qg + t * q_rs + ((int64_t)g * gs + (head_ok ? head : 0)) * D + 8 * q;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[ks] = ls_load16(qrow + 32 * ks);
      if (!head_ok) qf[ks] = ls_u32x4{0u, 0u, 0u, 0u};
    }
  }

  float m_run = -INFINITY, l_run = 0.f;
  ls_f32x4 o[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) o[i] = ls_f32x4{0.f, 0.f, 0.f, 0.f};

  const uint16_t* kgrp = kg + (int64_t)g * D + 8 * q;
  const uint16_t* vgrp = vt + ((int64_t)g * D + r) * lpad + vbase + 8 * q;
  // Row of the K fragment for MFMA row r: keys base + 8(r/4) + 4nb + r%4.
  const int krow_off = 8 * (r >> 2) + (r & 3);

  const int32_t* vexp_seq = vexp + (int64_t)g * n_pages + pg_off[b];
  for (int pi = 0; pi < n_list; ++pi) {
    const int page = s_list[w][pi];
    const float p_scale = __builtin_ldexpf(1.f, vexp_seq[page]);
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int64_t base = 64LL * page + 32 * c;
      if (base > jmax) break;
      ls_u32x4 kf0[4], kf1[4];
      {
        const int64_t k0 = min(base + krow_off, (int64_t)lk - 1);
        const int64_t k1 = min(base + krow_off + 4, (int64_t)lk - 1);
        const uint16_t* p0 = kgrp + (kstart + k0) * k_rs;
        const uint16_t* p1 = kgrp + (kstart + k1) * k_rs;
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          kf0[ks] = ls_load16(p0 + 32 * ks);
          kf1[ks] = ls_load16(p1 + 32 * ks);
        }
      }
      ls_u32x4 vf[8];
#pragma unroll
      for (int db = 0; db < 8; ++db) vf[db] = ls_load16(vgrp + (int64_t)16 * db * lpad + base);

      ls_f32x4 s0 = {0.f, 0.f, 0.f, 0.f}, s1 = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        s0 = LsElem<DT>::mfma(kf0[ks], qf[ks], s0);
        s1 = LsElem<DT>::mfma(kf1[ks], qf[ks], s1);
      }
      // Lane (r, q) now holds head r's scores of keys base + 8q + 0..7.
      float sv[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        sv[i] = s0[i] * scale_log2;
        sv[4 + i] = s1[i] * scale_log2;
      }
      const int64_t key0 = base + 8 * q;
#pragma unroll
      for (int i = 0; i < 8; ++i)
        if (key0 + i > jmax) sv[i] = -INFINITY;
      float cm = fmaxf(fmaxf(fmaxf(sv[0], sv[1]), fmaxf(sv[2], sv[3])),
                       fmaxf(fmaxf(sv[4], sv[5]), fmaxf(sv[6], sv[7])));
      cm = fmaxf(cm, ls_shfl_xor(cm, 16));
      cm = fmaxf(cm, ls_shfl_xor(cm, 32));
      const float m_new = fmaxf(m_run, cm);
      if (m_new == -INFINITY) continue;
      const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
      float pv[8], lsum = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        pv[i] = __builtin_amdgcn_exp2f(sv[i] - m_new);
        lsum += pv[i];
      }
      l_run = l_run * alpha + lsum;
      m_run = m_new;
      // P * V on the fp16 MFMA: P in [0, 1] keeps 10 mantissa bits; the page's
      // power-of-two V scale moves onto P exactly.
      ls_u32x4 pf;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pf[i] = ls_pack2(ls_f32_to_f16(pv[2 * i] * p_scale), ls_f32_to_f16(pv[2 * i + 1] * p_scale));
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        o[db] *= alpha;
        o[db] = LsElem<LS_F16>::mfma(vf[db], pf, o[db]);
      }
    }
  }

  float l_tot = l_run + ls_shfl_xor(l_run, 16);
  l_tot += ls_shfl_xor(l_tot, 32);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (head_ok) {
    uint16_t* orow = out + (t * G * gs + (int64_t)g * gs + head) * D + 4 * q;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      uint32_t lo = ls_pack2(LsElem<DT>::from_f(o[db][0] * inv), LsElem<DT>::from_f(o[db][1] * inv));
      uint32_t hi = ls_pack2(LsElem<DT>::from_f(o[db][2] * inv), LsElem<DT>::from_f(o[db][3] * inv));
      *reinterpret_cast<uint2*>(orow + 16 * db) = make_uint2(lo, hi);
    }
    if (lse && q == 0)
      lse[((int64_t)g * gs + head) * total_q + t] =
          l_tot > 0.f ? m_run * 0.69314718055994531f + __logf(l_tot) : INFINITY;
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {
struct AttnWs {
  size_t vt, pg, vexp, total;
  int64_t lpad, n_pages;
};
AttnWs attn_ws(int64_t total_k, int batch, int G, int D, int eb) {
  AttnWs L;
  L.n_pages = (total_k + 63) / 64 + batch;
  L.lpad = L.n_pages * 64;
  size_t off = 0;
  L.vt = off; off += ls_align256((size_t)G * D * L.lpad * eb);
  L.pg = off; off += ls_align256((size_t)(batch + 1) * 4);
  L.vexp = off; off += ls_align256((size_t)G * L.n_pages * 4);
  L.total = off;
  return L;
}
}  // namespace

extern "C" size_t ls_sparse_attn_workspace_size(int64_t total_k, int32_t batch,
                                                int32_t num_kv_heads, int32_t head_dim,
                                                int32_t max_seqlen_k, int32_t dtype) {
  (void)max_seqlen_k;
  return attn_ws(total_k, batch, num_kv_heads, head_dim, (int)ls_dtype_bytes(dtype)).total;
}

extern "C" int ls_sparse_attn_varlen(const void* q, int64_t q_row_stride, const void* k,
                                     int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                     const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                     int32_t batch, int64_t total_q, int64_t total_k,
                                     int32_t max_seqlen_q, int32_t max_seqlen_k,
                                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                     int32_t dtype, const int32_t* topk_idx, int32_t take,
                                     int32_t block_size, float softmax_scale, int32_t causal,
                                     void* out, float* lse, void* workspace,
                                     size_t workspace_bytes, void* stream) {
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen: only bf16 and fp16 are supported (dtype %d)", dtype);
  LS_REQUIRE(head_dim == 128, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen: head_dim must be 128 (got %d)", head_dim);
  LS_REQUIRE(block_size == 64, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen: block_size must be 64 (got %d)", block_size);
  LS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0, LS_ERR_INVALID,
             "ls_sparse_attn_varlen: num_heads must be a positive multiple of num_kv_heads");
  LS_REQUIRE(batch >= 0 && total_q >= 0 && total_k >= 0 && take >= 0, LS_ERR_INVALID,
             "ls_sparse_attn_varlen: bad sizes");
  LS_REQUIRE(take <= LS_ATTN_MAX_TAKE, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen: at most %d ids per row (got %d)", LS_ATTN_MAX_TAKE, take);
  LS_REQUIRE((int64_t)max_seqlen_k <= 64LL * LS_ATTN_MAX_PAGES, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen: max_seqlen_k above %d", 64 * LS_ATTN_MAX_PAGES);
  (void)max_seqlen_q;
  if (total_q == 0 || batch == 0) return LS_OK;
  LS_REQUIRE(q && k && v && out && cu_seqlens_q && cu_seqlens_k && (take == 0 || topk_idx),
             LS_ERR_INVALID, "ls_sparse_attn_varlen: null pointer");
  LS_REQUIRE(ls_aligned16(q) && ls_aligned16(k) && ls_aligned16(v) && ls_aligned16(out) &&
                 q_row_stride % 8 == 0 && k_row_stride % 8 == 0 && v_row_stride % 8 == 0,
             LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen: tensors must be 16-byte aligned with row strides %% 8 == 0");
  const AttnWs L = attn_ws(total_k, batch, num_kv_heads, head_dim, 2);
  LS_REQUIRE(workspace && workspace_bytes >= L.total, LS_ERR_WORKSPACE,
             "ls_sparse_attn_varlen: workspace needs %zu bytes", L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  uint16_t* vt = (uint16_t*)(ws + L.vt);
  int32_t* pg = (int32_t*)(ws + L.pg);
  int32_t* vexp = (int32_t*)(ws + L.vexp);
  hipLaunchKernelGGL(ls_attn_plan_kernel, dim3(1), dim3(64), 0, s, cu_seqlens_k, batch, pg);
  int rc = ls_check_launch("ls_attn_plan_kernel");
  if (rc) return rc;
  if (total_k > 0) {
    const dim3 vgrid((unsigned)((total_k + 63) / 64 + batch), num_kv_heads);
    if (dtype == LS_BF16)
      hipLaunchKernelGGL((ls_vt_kernel<LS_BF16, 128>), vgrid, dim3(256), 0, s, (const uint16_t*)v,
                         v_row_stride, cu_seqlens_k, pg, batch, L.lpad, L.n_pages, vt, vexp);
    else
      hipLaunchKernelGGL((ls_vt_kernel<LS_F16, 128>), vgrid, dim3(256), 0, s, (const uint16_t*)v,
                         v_row_stride, cu_seqlens_k, pg, batch, L.lpad, L.n_pages, vt, vexp);
    if ((rc = ls_check_launch("ls_vt_kernel"))) return rc;
  }
  const int gs = num_heads / num_kv_heads;
  const float scale = softmax_scale > 0.f ? softmax_scale : 1.0f / sqrtf((float)head_dim);
  const float scale_log2 = scale * 1.4426950408889634f;
  const dim3 grid((unsigned)((total_q + 3) / 4), num_kv_heads, (gs + 15) / 16);
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_attn_kernel<LS_BF16>, grid, dim3(256), 0, s, (const uint16_t*)q,
                       q_row_stride, (const uint16_t*)k, k_row_stride, vt, L.lpad, vexp, L.n_pages, cu_seqlens_q,
                       cu_seqlens_k, pg, batch, total_q, num_kv_heads, gs, topk_idx, take,
                       scale_log2, causal, (uint16_t*)out, lse);
  else
    hipLaunchKernelGGL(ls_attn_kernel<LS_F16>, grid, dim3(256), 0, s, (const uint16_t*)q,
                       q_row_stride, (const uint16_t*)k, k_row_stride, vt, L.lpad, vexp, L.n_pages, cu_seqlens_q,
                       cu_seqlens_k, pg, batch, total_q, num_kv_heads, gs, topk_idx, take,
                       scale_log2, causal, (uint16_t*)out, lse);
  return ls_check_launch("ls_attn_kernel");
}
