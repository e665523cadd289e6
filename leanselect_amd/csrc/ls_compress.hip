// Compressed keys: mean of kernel_size-token windows at kernel_stride,
// per packed sequence.  HBM-bound; each thread owns 8 consecutive channels of
// one (atom, kv-head) and sums in float32 in token order.  For windows of two
// strides (the 32/16 geometry) each half-window sum is read once and shared by
// the two windows that contain it (ls_compress_half_kernel); other geometries
// sum each window directly (ls_compress_kernel).
//
// Follows CompressK.forward + calc_chunks_with_stride
// (leanselect/models/minicpm.py:1158-1185, 711-750).
#include "ls_common.h"

// cu_out[b] = sum_{b' < b} n_atoms(b'); n_atoms = (len - ks) / stride + 1, or 0
// when len < ks.  One thread: batch sizes are small and this runs once.
__global__ void ls_compress_plan_kernel(const int32_t* __restrict__ cu_k, int batch, int ks,
                                        int stride, int32_t* __restrict__ cu_out) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  int32_t acc = 0;
  cu_out[0] = 0;
  for (int b = 0; b < batch; ++b) {
    int len = cu_k[b + 1] - cu_k[b];
    int n = len >= ks ? (len - ks) / stride + 1 : 0;
    acc += n;
    cu_out[b + 1] = acc;
  }
}

template <int DT>
__global__ __launch_bounds__(256) void ls_compress_kernel(
    const typename LsElem<DT>::T* __restrict__ k, int64_t k_row_stride,
    const int32_t* __restrict__ cu_k, const int32_t* __restrict__ cu_out, int batch, int G,
    int D, int ks, int stride, typename LsElem<DT>::T* __restrict__ out, int64_t total_atoms) {
  typedef typename LsElem<DT>::T T;
  const int d8_per_row = D / 8;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t per_atom = (int64_t)G * d8_per_row;
  const int64_t atom = idx / per_atom;
  if (atom >= total_atoms || atom >= (int64_t)cu_out[batch]) return;
  const int rem = (int)(idx - atom * per_atom);
  const int g = rem / d8_per_row;
  const int d0 = (rem - g * d8_per_row) * 8;
  const int b = ls_find_segment(cu_out, batch, atom);
  const int64_t tok0 = (int64_t)cu_k[b] + (atom - cu_out[b]) * (int64_t)stride;

  float acc[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) acc[i] = 0.f;
  const T* src = k + tok0 * k_row_stride + (int64_t)g * D + d0;
  for (int t = 0; t < ks; ++t) {
    const T* row = src + (int64_t)t * k_row_stride;
    if constexpr (DT == LS_F32) {
      ls_u32x4 a = ls_load16(row);
      ls_u32x4 c = ls_load16(row + 4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[i] += __uint_as_float(a[i]);
        acc[4 + i] += __uint_as_float(c[i]);
      }
    } else {
      ls_u32x4 a = ls_load16(row);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] += LsElem<DT>::to_f((uint16_t)(a[i] & 0xffffu));
        acc[2 * i + 1] += LsElem<DT>::to_f((uint16_t)(a[i] >> 16));
      }
    }
  }
  const float n_win = (float)ks;  // mean = sum / window length, as torch.mean
  T* dst = out + atom * per_atom * 8 + (int64_t)g * D + d0;
  if constexpr (DT == LS_F32) {
    ls_u32x4 a, c;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      a[i] = __float_as_uint(acc[i] / n_win);
      c[i] = __float_as_uint(acc[4 + i] / n_win);
    }
    *reinterpret_cast<ls_u32x4*>(dst) = a;
    *reinterpret_cast<ls_u32x4*>(dst + 4) = c;
  } else {
    ls_u32x4 a;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      a[i] = ls_pack2(LsElem<DT>::from_f(acc[2 * i] / n_win),
                      LsElem<DT>::from_f(acc[2 * i + 1] / n_win));
    *reinterpret_cast<ls_u32x4*>(dst) = a;
  }
}

// Windows of 2 * stride tokens (the 32/16 geometry): window a is the sum of
// the half windows [a*stride, (a+1)*stride) and [(a+1)*stride, (a+2)*stride),
// so each half-window sum is read from HBM once and shared by the two windows
// that contain it.  A block holds APB consecutive windows of one KV head,
// D/8 threads per window (8 channels each); a thread sums the first half of
// its window (float32, token order) into LDS and takes the second half from
// the next window's thread when that window is in the same block and
// sequence (otherwise it sums it itself).  mean = (first + second) / ks.
template <int DT>
__global__ __launch_bounds__(256) void ls_compress_half_kernel(
    const typename LsElem<DT>::T* __restrict__ k, int64_t k_row_stride,
    const int32_t* __restrict__ cu_k, const int32_t* __restrict__ cu_out, int batch, int G,
    int D, int stride, typename LsElem<DT>::T* __restrict__ out, int64_t total_atoms) {
  typedef typename LsElem<DT>::T T;
  __shared__ float s_half[256 * 8];
  const int tpa = D / 8;            // threads per window
  const int apb = 256 / tpa;        // windows per block
  const int tid = threadIdx.x;
  const int i = tid / tpa, j = tid - i * tpa;
  const int g = blockIdx.y;
  const int64_t n_atoms = min(total_atoms, (int64_t)cu_out[batch]);
  const int64_t atom = (int64_t)blockIdx.x * apb + i;
  const bool live = atom < n_atoms;
  int b = 0;
  int64_t tok0 = 0;
  float acc[8];
#pragma unroll
  for (int c = 0; c < 8; ++c) acc[c] = 0.f;
  auto add_rows = [&](int64_t first, float (&sum)[8]) {
    const T* src = k + first * k_row_stride + (int64_t)g * D + 8 * j;
    for (int t = 0; t < stride; ++t) {
      const T* row = src + (int64_t)t * k_row_stride;
      if constexpr (DT == LS_F32) {
        ls_u32x4 a = ls_load16(row);
        ls_u32x4 c = ls_load16(row + 4);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sum[e] += __uint_as_float(a[e]);
          sum[4 + e] += __uint_as_float(c[e]);
        }
      } else {
        ls_u32x4 a = ls_load16(row);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          sum[2 * e] += LsElem<DT>::to_f((uint16_t)(a[e] & 0xffffu));
          sum[2 * e + 1] += LsElem<DT>::to_f((uint16_t)(a[e] >> 16));
        }
      }
    }
  };
  if (live) {
    b = ls_find_segment(cu_out, batch, atom);
    tok0 = (int64_t)cu_k[b] + (atom - cu_out[b]) * (int64_t)stride;
    add_rows(tok0, acc);
  }
#pragma unroll
  for (int c = 0; c < 8; ++c) s_half[tid * 8 + c] = acc[c];
  __syncthreads();
  if (!live) return;
  float second[8];
  const bool shared = i + 1 < apb && atom + 1 < cu_out[b + 1];
  if (shared) {
#pragma unroll
    for (int c = 0; c < 8; ++c) second[c] = s_half[(tid + tpa) * 8 + c];
  } else {
#pragma unroll
    for (int c = 0; c < 8; ++c) second[c] = 0.f;
    add_rows(tok0 + stride, second);
  }
  const float n_win = (float)(2 * stride);  // mean = sum / window length, as torch.mean
  T* dst = out + (atom * G + g) * (int64_t)D + 8 * j;
  if constexpr (DT == LS_F32) {
    ls_u32x4 a, c;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      a[e] = __float_as_uint((acc[e] + second[e]) / n_win);
      c[e] = __float_as_uint((acc[4 + e] + second[4 + e]) / n_win);
    }
    *reinterpret_cast<ls_u32x4*>(dst) = a;
    *reinterpret_cast<ls_u32x4*>(dst + 4) = c;
  } else {
    ls_u32x4 a;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      a[e] = ls_pack2(LsElem<DT>::from_f((acc[2 * e] + second[2 * e]) / n_win),
                      LsElem<DT>::from_f((acc[2 * e + 1] + second[2 * e + 1]) / n_win));
    *reinterpret_cast<ls_u32x4*>(dst) = a;
  }
}

extern "C" int ls_compress_k_varlen(const void* k, int64_t k_row_stride,
                                    const int32_t* cu_seqlens_k, int32_t batch,
                                    int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                    int32_t kernel_size, int32_t kernel_stride, void* out,
                                    int64_t total_atoms, int32_t* cu_out, void* stream) {
  LS_REQUIRE(batch >= 0 && num_kv_heads > 0 && head_dim > 0, LS_ERR_INVALID,
             "ls_compress_k_varlen: bad sizes");
  LS_REQUIRE(kernel_size > 0 && kernel_stride > 0, LS_ERR_INVALID,
             "ls_compress_k_varlen: kernel_size and kernel_stride must be positive");
  LS_REQUIRE(dtype == LS_F32 || dtype == LS_BF16 || dtype == LS_F16, LS_ERR_INVALID,
             "ls_compress_k_varlen: unknown dtype %d", dtype);
  LS_REQUIRE(head_dim % 8 == 0 && k_row_stride % 8 == 0, LS_ERR_UNSUPPORTED,
             "ls_compress_k_varlen: head_dim and row stride must be multiples of 8");
  LS_REQUIRE(cu_seqlens_k && cu_out, LS_ERR_INVALID, "ls_compress_k_varlen: null cu_seqlens");
  LS_REQUIRE(total_atoms == 0 || (k && out), LS_ERR_INVALID, "ls_compress_k_varlen: null tensor");
  LS_REQUIRE(total_atoms == 0 || (ls_aligned16(k) && ls_aligned16(out)), LS_ERR_UNSUPPORTED,
             "ls_compress_k_varlen: tensors must be 16-byte aligned");
  hipStream_t s = (hipStream_t)stream;
  hipLaunchKernelGGL(ls_compress_plan_kernel, dim3(1), dim3(64), 0, s, cu_seqlens_k, batch,
                     kernel_size, kernel_stride, cu_out);
  int rc = ls_check_launch("ls_compress_plan_kernel");
  if (rc) return rc;
  if (total_atoms == 0 || batch == 0) return LS_OK;
  const int tpa = head_dim / 8;
  if (kernel_size == 2 * kernel_stride && tpa <= 256 && 256 % tpa == 0) {
    const int apb = 256 / tpa;
    const dim3 hgrid((unsigned)((total_atoms + apb - 1) / apb), num_kv_heads);
#define LS_HALF_ARGS hgrid, dim3(256), 0, s
    switch (dtype) {
      case LS_BF16:
        hipLaunchKernelGGL(ls_compress_half_kernel<LS_BF16>, LS_HALF_ARGS, (const uint16_t*)k,
                           k_row_stride, cu_seqlens_k, cu_out, batch, num_kv_heads, head_dim,
                           kernel_stride, (uint16_t*)out, total_atoms);
        break;
      case LS_F16:
        hipLaunchKernelGGL(ls_compress_half_kernel<LS_F16>, LS_HALF_ARGS, (const uint16_t*)k,
                           k_row_stride, cu_seqlens_k, cu_out, batch, num_kv_heads, head_dim,
                           kernel_stride, (uint16_t*)out, total_atoms);
        break;
      default:
        hipLaunchKernelGGL(ls_compress_half_kernel<LS_F32>, LS_HALF_ARGS, (const float*)k,
                           k_row_stride, cu_seqlens_k, cu_out, batch, num_kv_heads, head_dim,
                           kernel_stride, (float*)out, total_atoms);
        break;
    }
#undef LS_HALF_ARGS
    return ls_check_launch("ls_compress_half_kernel");
  }
  const int64_t threads = total_atoms * num_kv_heads * (head_dim / 8);
  const dim3 grid((unsigned)((threads + 255) / 256));
  switch (dtype) {
    case LS_BF16:
      hipLaunchKernelGGL(ls_compress_kernel<LS_BF16>, grid, dim3(256), 0, s,
                         (const uint16_t*)k, k_row_stride, cu_seqlens_k, cu_out, batch,
                         num_kv_heads, head_dim, kernel_size, kernel_stride, (uint16_t*)out,
                         total_atoms);
      break;
    case LS_F16:
      hipLaunchKernelGGL(ls_compress_kernel<LS_F16>, grid, dim3(256), 0, s,
                         (const uint16_t*)k, k_row_stride, cu_seqlens_k, cu_out, batch,
                         num_kv_heads, head_dim, kernel_size, kernel_stride, (uint16_t*)out,
                         total_atoms);
      break;
    default:
      hipLaunchKernelGGL(ls_compress_kernel<LS_F32>, grid, dim3(256), 0, s, (const float*)k,
                         k_row_stride, cu_seqlens_k, cu_out, batch, num_kv_heads, head_dim,
                         kernel_size, kernel_stride, (float*)out, total_atoms);
      break;
  }
  return ls_check_launch("ls_compress_kernel");
}
