// Producer and consumer kernels around the LeanSelect attention layer in a
// MiniCPM4.1 decoder (leanselect/models/minicpm.py:3562-3630): RMSNorm, the
// scaled residual add fused with the next RMSNorm, in-place rotary embedding
// of the packed QKV projection output, SiLU-gated FFN activation and the
// scaled token embedding.  All are HBM-bound elementwise or row reductions:
// 16-byte loads and stores, float32 arithmetic, and the reference's rounding
// points (each torch op that returns a 16-bit tensor rounds once, RNE).
// Every product and sum rounds separately, as in the reference's torch
// expressions: this file is built with -ffp-contract=off (no fused
// multiply-adds).
#include <type_traits>

#include "ls_common.h"

namespace {

__device__ __forceinline__ void ls_unpack8(const ls_u32x4& v, float (&f)[8], bool bf16) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t lo = (uint16_t)(v[i] & 0xffffu), hi = (uint16_t)(v[i] >> 16);
    f[2 * i] = bf16 ? ls_bf16_to_f32(lo) : ls_f16_to_f32(lo);
    f[2 * i + 1] = bf16 ? ls_bf16_to_f32(hi) : ls_f16_to_f32(hi);
  }
}

template <int DT>
__device__ __forceinline__ ls_u32x4 ls_pack8(const float (&f)[8]) {
  ls_u32x4 v;
#pragma unroll
  for (int i = 0; i < 4; ++i)
    v[i] = ls_pack2(LsElem<DT>::from_f(f[2 * i]), LsElem<DT>::from_f(f[2 * i + 1]));
  return v;
}

template <int DT>
__device__ __forceinline__ float ls_round(float x) {
  return LsElem<DT>::to_f(LsElem<DT>::from_f(x));
}

}  // namespace

// ---------------------------------------------------------------------------
// RMSNorm (rms_layernorm, minicpm.py:772-788), one wave per row:
//   var = mean(float(x)^2);  n = round(float(x) * (1 / sqrt(var + eps)));
//   out = round(float(n) * float(w)).
// With ADD, the row is first the new residual (minicpm.py:3616-3625):
//   x = round(float(res) + float(round(float(h) * c)))   (written back to res).
// A lane holds 8-element chunks lane*8 + 512*i of the row in registers, NC of
// them (the row's chunk count over 64, rounded up to a power of two).  All of
// a row's loads are issued before any is used (indices past the row are
// clamped into it and their values not used), so their latencies overlap.
// ---------------------------------------------------------------------------
#define LS_NORM_MAX_CHUNKS 16  // hidden <= 64 lanes * 8 * 16 = 8192

template <int DT, bool ADD, int NC>
__global__ __launch_bounds__(256) void ls_rmsnorm_kernel(
    uint16_t* __restrict__ x, int64_t xs, const uint16_t* __restrict__ h, int64_t hs, float c,
    const uint16_t* __restrict__ w, int64_t n_rows, int hidden, float eps,
    uint16_t* __restrict__ out, int64_t os) {
  static_assert(NC >= 1 && NC <= LS_NORM_MAX_CHUNKS, "chunks per lane");
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  constexpr bool BF = DT == LS_BF16;
  const int nch = hidden / 8;
  uint16_t* xr = x + row * xs;
  ls_u32x4 v[NC], hv[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int ch = min(lane + 64 * i, nch - 1);
    v[i] = ls_load16(xr + 8 * ch);
    if constexpr (ADD) hv[i] = ls_load16(h + row * hs + 8 * ch);
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    if (lane + 64 * i >= nch) break;
    float f[8];
    ls_unpack8(v[i], f, BF);
    if constexpr (ADD) {
      float g[8];
      ls_unpack8(hv[i], g, BF);
#pragma unroll
      for (int j = 0; j < 8; ++j) f[j] = ls_round<DT>(__fadd_rn(f[j], ls_round<DT>(__fmul_rn(g[j], c))));
      v[i] = ls_pack8<DT>(f);
      *reinterpret_cast<ls_u32x4*>(xr + 8 * (lane + 64 * i)) = v[i];
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) ss = __fadd_rn(ss, __fmul_rn(f[j], f[j]));
  }
  ls_u32x4 wv[NC];
#pragma unroll
  for (int i = 0; i < NC; ++i) wv[i] = ls_load16(w + 8 * min(lane + 64 * i, nch - 1));
#pragma unroll
  for (int d = 32; d >= 1; d >>= 1) ss += __shfl_xor(ss, d, 64);
  const float rs = 1.f / sqrtf(__fadd_rn(__fmul_rn(ss, 1.f / (float)hidden), eps));
  uint16_t* orow = out + row * os;
#pragma unroll
  for (int i = 0; i < NC; ++i) {
    const int ch = lane + 64 * i;
    if (ch >= nch) break;
    float f[8], wf[8];
    ls_unpack8(v[i], f, BF);
    ls_unpack8(wv[i], wf, BF);
#pragma unroll
    for (int j = 0; j < 8; ++j) f[j] = __fmul_rn(ls_round<DT>(__fmul_rn(f[j], rs)), wf[j]);
    *reinterpret_cast<ls_u32x4*>(orow + 8 * ch) = ls_pack8<DT>(f);
  }
}

// ---------------------------------------------------------------------------
// Rotary embedding in place (apply_rotary_pos_emb, minicpm.py:1027-1070):
//   out = round(float(x) * cos[p] + rotate_half(float(x)) * sin[p]),
// products and sum each rounded to float32 (no fused multiply-add), with
// rotate_half(x) = (-x[64:], x[:64]).  One wave per row: lane l owns the
// pair chunks d = 8 (l & 7) .. +7 and d + 64 of heads (l >> 3) + 8 j, so its
// 32 table entries are loaded once per row.  Query heads start at column 0,
// key heads at column k_off, each head_dim (128) wide.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void ls_rope_kernel(
    uint16_t* __restrict__ x, int64_t xs, const int32_t* __restrict__ pos, int64_t n_rows,
    int n_q, int n_k, int64_t k_off, const float* __restrict__ cosb,
    const float* __restrict__ sinb, int64_t table_rows) {
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= n_rows) return;
  constexpr bool BF = DT == LS_BF16;
  const int c = lane & 7;
  int64_t p = pos[row];
  p = p < 0 ? 0 : (p >= table_rows ? table_rows - 1 : p);  // the host checks the range
  const float* cr = cosb + p * 128 + 8 * c;
  const float* sr = sinb + p * 128 + 8 * c;
  float c1[8], c2[8], s1[8], s2[8];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const ls_f32x4 a = *reinterpret_cast<const ls_f32x4*>(cr + 4 * i);
    const ls_f32x4 b = *reinterpret_cast<const ls_f32x4*>(cr + 64 + 4 * i);
    const ls_f32x4 e = *reinterpret_cast<const ls_f32x4*>(sr + 4 * i);
    const ls_f32x4 f = *reinterpret_cast<const ls_f32x4*>(sr + 64 + 4 * i);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c1[4 * i + j] = a[j];
      c2[4 * i + j] = b[j];
      s1[4 * i + j] = e[j];
      s2[4 * i + j] = f[j];
    }
  }
  uint16_t* xr = x + row * xs;
  const int heads = n_q + n_k;
  for (int hd = lane >> 3; hd < heads; hd += 8) {
    uint16_t* base = xr + (hd < n_q ? (int64_t)hd * 128 : k_off + (int64_t)(hd - n_q) * 128) + 8 * c;
    float x1[8], x2[8], y1[8], y2[8];
    ls_unpack8(ls_load16(base), x1, BF);
    ls_unpack8(ls_load16(base + 64), x2, BF);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      y1[j] = __fadd_rn(__fmul_rn(x1[j], c1[j]), __fmul_rn(-x2[j], s1[j]));
      y2[j] = __fadd_rn(__fmul_rn(x2[j], c2[j]), __fmul_rn(x1[j], s2[j]));
    }
    *reinterpret_cast<ls_u32x4*>(base) = ls_pack8<DT>(y1);
    *reinterpret_cast<ls_u32x4*>(base + 64) = ls_pack8<DT>(y2);
  }
}

// ---------------------------------------------------------------------------
// Rotary embedding of the key heads fused with the compressed keys
// (producer-side compression: the mean of 32 post-RoPE key rows at stride 16,
// CompressK.forward, minicpm.py:1158-1185, formed while the rows are rotated
// instead of re-reading them).  Window a of a sequence is the sum of its half
// windows a and a + 1 (16 rows each), so:
//   ls_rope_k_half_kernel  one workgroup per 16-row half window of one
//     sequence, one thread per (key head, rotation pair d / d + 64): rotates
//     the rows in place exactly as ls_rope_kernel and sums the rounded results
//     in float32 in row order into hsum[half][head][128];
//   ls_k_atoms_kernel      kc[atom][head][d] = round((hsum[a][head][d] +
//     hsum[a + 1][head][d]) / 32): the same sums, in the same order, as
//     ls_compress_half_kernel forms from the rotated rows.
// hw_off[b] = sum_{b' < b} ceil(len(b') / 16) (first half window of each
// sequence); cu_out[b] as ls_compress_k_varlen.
// ---------------------------------------------------------------------------
__global__ void ls_rope_k_plan_kernel(const int32_t* __restrict__ cu, int batch,
                                      int32_t* __restrict__ hw_off, int32_t* __restrict__ cu_out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t h = 0, a = 0;
  hw_off[0] = 0;
  cu_out[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int len = cu[b + 1] - cu[b];
    h += len > 0 ? (len + 15) / 16 : 0;
    a += len >= 32 ? (len - 32) / 16 + 1 : 0;
    hw_off[b + 1] = h;
    cu_out[b + 1] = a;
  }
}

template <int DT>
__global__ __launch_bounds__(1024) void ls_rope_k_half_kernel(
    uint16_t* __restrict__ x, int64_t xs, const int32_t* __restrict__ pos,
    const int32_t* __restrict__ cu, const int32_t* __restrict__ hw_off, int batch, int n_k,
    int64_t k_off, const float* __restrict__ cosb, const float* __restrict__ sinb,
    int64_t table_rows, float* __restrict__ hsum) {
  const int64_t hw = blockIdx.x;
  if (hw >= hw_off[batch]) return;
  const int b = ls_find_segment(hw_off, batch, hw);
  const int64_t r0 = (int64_t)cu[b] + 16 * (hw - hw_off[b]);
  const int rows = (int)min((int64_t)16, (int64_t)cu[b + 1] - r0);
  const int hd = threadIdx.x >> 6, d = threadIdx.x & 63;
  float s1 = 0.f, s2 = 0.f;
  for (int r = 0; r < rows; ++r) {
    const int64_t row = r0 + r;
    int64_t p = pos[row];
    p = p < 0 ? 0 : (p >= table_rows ? table_rows - 1 : p);
    uint16_t* xr = x + row * xs + k_off + (int64_t)hd * 128;
    const float x1 = LsElem<DT>::to_f(xr[d]), x2 = LsElem<DT>::to_f(xr[d + 64]);
    const float y1 = __fadd_rn(__fmul_rn(x1, cosb[p * 128 + d]), __fmul_rn(-x2, sinb[p * 128 + d]));
    const float y2 = __fadd_rn(__fmul_rn(x2, cosb[p * 128 + 64 + d]), __fmul_rn(x1, sinb[p * 128 + 64 + d]));
    const uint16_t o1 = LsElem<DT>::from_f(y1), o2 = LsElem<DT>::from_f(y2);
    xr[d] = o1;
    xr[d + 64] = o2;
    s1 += LsElem<DT>::to_f(o1);
    s2 += LsElem<DT>::to_f(o2);
  }
  float* hs = hsum + (hw * n_k + hd) * 128;
  hs[d] = s1;
  hs[d + 64] = s2;
}

template <int DT>
__global__ __launch_bounds__(256) void ls_k_atoms_kernel(
    const float* __restrict__ hsum, const int32_t* __restrict__ hw_off,
    const int32_t* __restrict__ cu_out, int batch, int n_k, int64_t total_atoms,
    uint16_t* __restrict__ kc) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t per_atom = (int64_t)n_k * 128;
  const int64_t atom = i / per_atom;
  if (atom >= total_atoms || atom >= cu_out[batch]) return;
  const int e = (int)(i - atom * per_atom);
  const int b = ls_find_segment(cu_out, batch, atom);
  const int64_t h = hw_off[b] + (atom - cu_out[b]);
  const float v = (hsum[h * per_atom + e] + hsum[(h + 1) * per_atom + e]) / 32.f;
  kc[atom * per_atom + e] = LsElem<DT>::from_f(v);
}

// ---------------------------------------------------------------------------
// SiLU-gated activation (MiniCPMMLP.forward, minicpm.py:1098-1130:
// act_fn(gate_proj(x)) * up_proj(x)) on one [n, 2 I] GEMM output holding gate
// columns [0, I) and up columns [I, 2 I):
//   out = round(float(round(g / (1 + exp(-g)))) * float(u)).
// One thread per 8 outputs.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void ls_silu_mul_kernel(const uint16_t* __restrict__ gu,
                                                          int64_t gs, int64_t n_rows, int inter,
                                                          uint16_t* __restrict__ out, int64_t os) {
  const int per_row = inter / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n_rows * per_row) return;
  constexpr bool BF = DT == LS_BF16;
  const int64_t row = i / per_row;
  const int ch = (int)(i % per_row);
  float g[8], u[8];
  ls_unpack8(ls_load16(gu + row * gs + 8 * ch), g, BF);
  ls_unpack8(ls_load16(gu + row * gs + inter + 8 * ch), u, BF);
#pragma unroll
  for (int j = 0; j < 8; ++j)
    g[j] = __fmul_rn(ls_round<DT>(g[j] / __fadd_rn(1.f, expf(-g[j]))), u[j]);
  *reinterpret_cast<ls_u32x4*>(out + row * os + 8 * ch) = ls_pack8<DT>(g);
}

// ---------------------------------------------------------------------------
// Scaled token embedding (MiniCPMModel.forward, minicpm.py:3773-3774):
//   out[n] = round(float(table[ids[n]]) * scale).  One thread per 8 outputs.
// ---------------------------------------------------------------------------
template <int DT>
__global__ __launch_bounds__(256) void ls_embed_kernel(const int32_t* __restrict__ ids, int64_t n,
                                                       const uint16_t* __restrict__ table,
                                                       int64_t vocab, int hidden, float scale,
                                                       uint16_t* __restrict__ out) {
  const int per_row = hidden / 8;
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (i >= n * per_row) return;
  constexpr bool BF = DT == LS_BF16;
  const int64_t row = i / per_row;
  const int ch = (int)(i % per_row);
  int64_t id = ids[row];
  id = id < 0 ? 0 : (id >= vocab ? vocab - 1 : id);  // the host checks the range
  float f[8];
  ls_unpack8(ls_load16(table + id * hidden + 8 * ch), f, BF);
#pragma unroll
  for (int j = 0; j < 8; ++j) f[j] = __fmul_rn(f[j], scale);
  *reinterpret_cast<ls_u32x4*>(out + row * hidden + 8 * ch) = ls_pack8<DT>(f);
}

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
namespace {

int ls_model_dtype(int dtype, const char* who) {
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "%s: bf16 or fp16 only (got dtype %d)", who, dtype);
  return LS_OK;
}

template <bool ADD>
int launch_norm(int dtype, uint16_t* x, int64_t xs, const uint16_t* h, int64_t hs, float c,
                const uint16_t* w, int64_t n, int hidden, float eps, uint16_t* out, int64_t os,
                hipStream_t s) {
  const dim3 grid((unsigned)((n + 3) / 4));
  const int per_lane = (hidden / 8 + 63) / 64;
  auto go = [&](auto nc) {
    constexpr int NC = decltype(nc)::value;
    if (dtype == LS_BF16)
      hipLaunchKernelGGL((ls_rmsnorm_kernel<LS_BF16, ADD, NC>), grid, dim3(256), 0, s, x, xs, h,
                         hs, c, w, n, hidden, eps, out, os);
    else
      hipLaunchKernelGGL((ls_rmsnorm_kernel<LS_F16, ADD, NC>), grid, dim3(256), 0, s, x, xs, h,
                         hs, c, w, n, hidden, eps, out, os);
  };
  if (per_lane <= 1) go(std::integral_constant<int, 1>());
  else if (per_lane <= 2) go(std::integral_constant<int, 2>());
  else if (per_lane <= 4) go(std::integral_constant<int, 4>());
  else if (per_lane <= 8) go(std::integral_constant<int, 8>());
  else go(std::integral_constant<int, LS_NORM_MAX_CHUNKS>());
  return ls_check_launch("ls_rmsnorm_kernel");
}

int check_norm(const char* who, int64_t n, int hidden, int64_t xs, int64_t os, int dtype) {
  if (int rc = ls_model_dtype(dtype, who)) return rc;
  LS_REQUIRE(n >= 0 && hidden > 0 && hidden % 8 == 0 && hidden <= 64 * 8 * LS_NORM_MAX_CHUNKS,
             LS_ERR_UNSUPPORTED, "%s: hidden must be a multiple of 8 up to %d (got %d)", who,
             64 * 8 * LS_NORM_MAX_CHUNKS, hidden);
  LS_REQUIRE(xs >= hidden && os >= hidden && xs % 8 == 0 && os % 8 == 0, LS_ERR_INVALID,
             "%s: row strides must be >= hidden and multiples of 8", who);
  return LS_OK;
}

}  // namespace

extern "C" int ls_rmsnorm(const void* x, int64_t x_row_stride, const void* weight, int64_t n_rows,
                          int32_t hidden, float eps, int32_t dtype, void* out,
                          int64_t out_row_stride, void* stream) {
  if (int rc = check_norm("ls_rmsnorm", n_rows, hidden, x_row_stride, out_row_stride, dtype))
    return rc;
  if (n_rows == 0) return LS_OK;
  LS_REQUIRE(ls_aligned16(x) && ls_aligned16(weight) && ls_aligned16(out), LS_ERR_UNSUPPORTED,
             "ls_rmsnorm: tensors must be 16-byte aligned");
  return launch_norm<false>(dtype, (uint16_t*)x, x_row_stride, nullptr, 0, 0.f,
                            (const uint16_t*)weight, n_rows, hidden, eps, (uint16_t*)out,
                            out_row_stride, (hipStream_t)stream);
}

extern "C" int ls_add_rmsnorm(void* residual, int64_t res_row_stride, const void* h,
                              int64_t h_row_stride, float h_scale, const void* weight,
                              int64_t n_rows, int32_t hidden, float eps, int32_t dtype, void* out,
                              int64_t out_row_stride, void* stream) {
  if (int rc = check_norm("ls_add_rmsnorm", n_rows, hidden, res_row_stride, out_row_stride, dtype))
    return rc;
  LS_REQUIRE(h_row_stride >= hidden && h_row_stride % 8 == 0, LS_ERR_INVALID,
             "ls_add_rmsnorm: h row stride must be >= hidden and a multiple of 8");
  if (n_rows == 0) return LS_OK;
  LS_REQUIRE(ls_aligned16(residual) && ls_aligned16(h) && ls_aligned16(weight) &&
                 ls_aligned16(out),
             LS_ERR_UNSUPPORTED, "ls_add_rmsnorm: tensors must be 16-byte aligned");
  return launch_norm<true>(dtype, (uint16_t*)residual, res_row_stride, (const uint16_t*)h,
                           h_row_stride, h_scale, (const uint16_t*)weight, n_rows, hidden, eps,
                           (uint16_t*)out, out_row_stride, (hipStream_t)stream);
}

extern "C" int ls_rope_inplace(void* x, int64_t row_stride, const int32_t* positions,
                               int64_t n_rows, int32_t n_q_heads, int32_t n_k_heads,
                               int64_t k_col_offset, int32_t head_dim, const float* cos_table,
                               const float* sin_table, int64_t table_rows, int32_t dtype,
                               void* stream) {
  if (int rc = ls_model_dtype(dtype, "ls_rope_inplace")) return rc;
  LS_REQUIRE(head_dim == 128, LS_ERR_UNSUPPORTED, "ls_rope_inplace: head_dim must be 128 (got %d)",
             head_dim);
  LS_REQUIRE(n_rows >= 0 && n_q_heads >= 0 && n_k_heads >= 0 && table_rows > 0, LS_ERR_INVALID,
             "ls_rope_inplace: bad sizes");
  LS_REQUIRE(row_stride % 8 == 0 && k_col_offset % 8 == 0 &&
                 row_stride >= (int64_t)n_q_heads * head_dim &&
                 row_stride >= k_col_offset + (int64_t)n_k_heads * head_dim,
             LS_ERR_INVALID, "ls_rope_inplace: heads must lie inside the row (stride %lld)",
             (long long)row_stride);
  LS_REQUIRE(n_k_heads == 0 || k_col_offset >= (int64_t)n_q_heads * head_dim, LS_ERR_INVALID,
             "ls_rope_inplace: key heads must not overlap the query heads");
  if (n_rows == 0 || n_q_heads + n_k_heads == 0) return LS_OK;
  LS_REQUIRE(ls_aligned16(x) && ls_aligned16(cos_table) && ls_aligned16(sin_table),
             LS_ERR_UNSUPPORTED, "ls_rope_inplace: tensors must be 16-byte aligned");
  const dim3 grid((unsigned)((n_rows + 3) / 4));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_rope_kernel<LS_BF16>, grid, dim3(256), 0, s, (uint16_t*)x, row_stride,
                       positions, n_rows, n_q_heads, n_k_heads, k_col_offset, cos_table,
                       sin_table, table_rows);
  else
    hipLaunchKernelGGL(ls_rope_kernel<LS_F16>, grid, dim3(256), 0, s, (uint16_t*)x, row_stride,
                       positions, n_rows, n_q_heads, n_k_heads, k_col_offset, cos_table,
                       sin_table, table_rows);
  return ls_check_launch("ls_rope_kernel");
}

extern "C" int ls_silu_mul(const void* gate_up, int64_t gu_row_stride, int64_t n_rows,
                           int32_t inter, int32_t dtype, void* out, int64_t out_row_stride,
                           void* stream) {
  if (int rc = ls_model_dtype(dtype, "ls_silu_mul")) return rc;
  LS_REQUIRE(n_rows >= 0 && inter > 0 && inter % 8 == 0, LS_ERR_UNSUPPORTED,
             "ls_silu_mul: intermediate size must be a positive multiple of 8 (got %d)", inter);
  LS_REQUIRE(gu_row_stride >= 2LL * inter && gu_row_stride % 8 == 0 && out_row_stride >= inter &&
                 out_row_stride % 8 == 0,
             LS_ERR_INVALID, "ls_silu_mul: bad row strides");
  if (n_rows == 0) return LS_OK;
  LS_REQUIRE(ls_aligned16(gate_up) && ls_aligned16(out), LS_ERR_UNSUPPORTED,
             "ls_silu_mul: tensors must be 16-byte aligned");
  const int64_t threads = n_rows * (inter / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_silu_mul_kernel<LS_BF16>, grid, dim3(256), 0, s,
                       (const uint16_t*)gate_up, gu_row_stride, n_rows, inter, (uint16_t*)out,
                       out_row_stride);
  else
    hipLaunchKernelGGL(ls_silu_mul_kernel<LS_F16>, grid, dim3(256), 0, s,
                       (const uint16_t*)gate_up, gu_row_stride, n_rows, inter, (uint16_t*)out,
                       out_row_stride);
  return ls_check_launch("ls_silu_mul_kernel");
}

extern "C" int ls_embed_scale(const int32_t* ids, int64_t n, const void* table, int64_t vocab,
                              int32_t hidden, float scale, int32_t dtype, void* out,
                              void* stream) {
  if (int rc = ls_model_dtype(dtype, "ls_embed_scale")) return rc;
  LS_REQUIRE(n >= 0 && vocab > 0 && hidden > 0 && hidden % 8 == 0, LS_ERR_UNSUPPORTED,
             "ls_embed_scale: hidden must be a positive multiple of 8 (got %d)", hidden);
  if (n == 0) return LS_OK;
  LS_REQUIRE(ls_aligned16(table) && ls_aligned16(out), LS_ERR_UNSUPPORTED,
             "ls_embed_scale: tensors must be 16-byte aligned");
  const int64_t threads = n * (hidden / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipStream_t s = (hipStream_t)stream;
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_embed_kernel<LS_BF16>, grid, dim3(256), 0, s, ids, n,
                       (const uint16_t*)table, vocab, hidden, scale, (uint16_t*)out);
  else
    hipLaunchKernelGGL(ls_embed_kernel<LS_F16>, grid, dim3(256), 0, s, ids, n,
                       (const uint16_t*)table, vocab, hidden, scale, (uint16_t*)out);
  return ls_check_launch("ls_embed_kernel");
}

extern "C" size_t ls_rope_k_compress_workspace_size(int64_t n_rows, int32_t batch,
                                                    int32_t n_k_heads, int32_t head_dim) {
  (void)head_dim;
  const int64_t halves = (n_rows > 0 ? n_rows : 0) / 16 + (batch > 0 ? batch : 0);
  return ls_align256((size_t)(batch + 1) * 4) +
         ls_align256((size_t)halves * (n_k_heads > 0 ? n_k_heads : 0) * 128 * 4);
}

extern "C" int ls_rope_k_compress(void* x, int64_t row_stride, const int32_t* positions,
                                  const int32_t* cu_seqlens, int32_t batch, int64_t n_rows,
                                  int32_t n_k_heads, int64_t k_col_offset, int32_t head_dim,
                                  const float* cos_table, const float* sin_table,
                                  int64_t table_rows, int32_t dtype, void* kc_out,
                                  int64_t total_atoms, int32_t* cu_out, void* workspace,
                                  size_t workspace_bytes, void* stream) {
  if (int rc = ls_model_dtype(dtype, "ls_rope_k_compress")) return rc;
  LS_REQUIRE(head_dim == 128, LS_ERR_UNSUPPORTED,
             "ls_rope_k_compress: head_dim must be 128 (got %d)", head_dim);
  LS_REQUIRE(n_rows >= 0 && batch >= 0 && n_k_heads > 0 && n_k_heads <= 16 && table_rows > 0 &&
                 total_atoms >= 0,
             LS_ERR_INVALID, "ls_rope_k_compress: bad sizes");
  LS_REQUIRE(k_col_offset >= 0 && row_stride >= k_col_offset + (int64_t)n_k_heads * head_dim,
             LS_ERR_INVALID, "ls_rope_k_compress: key heads must lie inside the row");
  LS_REQUIRE(cu_seqlens && cu_out, LS_ERR_INVALID, "ls_rope_k_compress: null cu_seqlens");
  const size_t need = ls_rope_k_compress_workspace_size(n_rows, batch, n_k_heads, head_dim);
  LS_REQUIRE(workspace && workspace_bytes >= need, LS_ERR_WORKSPACE,
             "ls_rope_k_compress: workspace needs %zu bytes", need);
  hipStream_t s = (hipStream_t)stream;
  int32_t* hw_off = (int32_t*)workspace;
  float* hsum = (float*)((char*)workspace + ls_align256((size_t)(batch + 1) * 4));
  hipLaunchKernelGGL(ls_rope_k_plan_kernel, dim3(1), dim3(64), 0, s, cu_seqlens, batch, hw_off,
                     cu_out);
  if (int rc = ls_check_launch("ls_rope_k_plan_kernel")) return rc;
  if (n_rows == 0 || batch == 0) return LS_OK;
  LS_REQUIRE(x && positions && cos_table && sin_table && (total_atoms == 0 || kc_out),
             LS_ERR_INVALID, "ls_rope_k_compress: null tensor");
  const int64_t halves = n_rows / 16 + batch;
  const dim3 hgrid((unsigned)halves), hblock((unsigned)(64 * n_k_heads));
  const dim3 agrid((unsigned)((total_atoms * n_k_heads * 128 + 255) / 256));
  if (dtype == LS_BF16) {
    hipLaunchKernelGGL(ls_rope_k_half_kernel<LS_BF16>, hgrid, hblock, 0, s, (uint16_t*)x,
                       row_stride, positions, cu_seqlens, hw_off, batch, n_k_heads, k_col_offset,
                       cos_table, sin_table, table_rows, hsum);
    if (int rc = ls_check_launch("ls_rope_k_half_kernel")) return rc;
    if (total_atoms > 0)
      hipLaunchKernelGGL(ls_k_atoms_kernel<LS_BF16>, agrid, dim3(256), 0, s, hsum, hw_off, cu_out,
                         batch, n_k_heads, total_atoms, (uint16_t*)kc_out);
  } else {
    hipLaunchKernelGGL(ls_rope_k_half_kernel<LS_F16>, hgrid, hblock, 0, s, (uint16_t*)x,
                       row_stride, positions, cu_seqlens, hw_off, batch, n_k_heads, k_col_offset,
                       cos_table, sin_table, table_rows, hsum);
    if (int rc = ls_check_launch("ls_rope_k_half_kernel")) return rc;
    if (total_atoms > 0)
      hipLaunchKernelGGL(ls_k_atoms_kernel<LS_F16>, agrid, dim3(256), 0, s, hsum, hw_off, cu_out,
                         batch, n_k_heads, total_atoms, (uint16_t*)kc_out);
  }
  return ls_check_launch("ls_k_atoms_kernel");
}
