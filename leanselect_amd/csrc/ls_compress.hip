// Compressed keys: mean of kernel_size-token windows at kernel_stride,
// per packed sequence.  HBM-bound; each thread owns 8 consecutive channels of
// one (atom, kv-head) and sums its window in float32 in token order.
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
