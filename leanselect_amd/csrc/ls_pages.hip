// Page geometry kernels behind leanselect/pages.py's hot-path helpers.
//   ls_pool_atoms_to_pages  pool_atoms_to_pages(reduce="max")  leanselect/pages.py:146-187
//   ls_forced_page_mask     forced_page_mask                   leanselect/pages.py:222-240
// Both are bandwidth-bound elementwise maps (one thread per output element).
#include "ls_common.h"

template <int DT>
__global__ __launch_bounds__(256) void ls_pool_kernel(const typename LsElem<DT>::T* __restrict__ in,
                                                      int64_t rows, int64_t n_atoms,
                                                      int64_t row_stride, int64_t n_pages, int s,
                                                      typename LsElem<DT>::T* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= rows * n_pages) return;
  const int64_t r = i / n_pages, p = i % n_pages;
  const typename LsElem<DT>::T* row = in + r * row_stride;
  float best = -INFINITY;
  const int64_t a_lo = p * s - 1 < 0 ? 0 : p * s - 1;
  const int64_t a_hi = p * s + s < n_atoms ? p * s + s : n_atoms;
  for (int64_t a = a_lo; a < a_hi; ++a) best = fmaxf(best, LsElem<DT>::to_f(row[a]));
  out[i] = LsElem<DT>::from_f(best);
}

__global__ __launch_bounds__(256) void ls_forced_kernel(const int64_t* __restrict__ pos,
                                                        int64_t n, int64_t num_pages,
                                                        int block_size, int init_blocks,
                                                        int local_blocks,
                                                        uint8_t* __restrict__ out) {
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n * num_pages) return;
  const int64_t qi = i / num_pages, p = i % num_pages;
  const int64_t x = pos[qi];
  // Floor division, as torch's // on int64.
  const int64_t qp = x >= 0 ? x / block_size : -((-x + block_size - 1) / block_size);
  out[i] = (uint8_t)(p < init_blocks || (qp >= p && qp <= p + local_blocks));
}

extern "C" int ls_pool_atoms_to_pages(const void* atom_scores, int64_t rows, int64_t n_atoms,
                                      int64_t row_stride, int32_t dtype, int64_t n_pages,
                                      int32_t pool_stride, void* out, void* stream) {
  LS_REQUIRE(rows >= 0 && n_atoms > 0 && n_pages >= 0 && pool_stride > 0, LS_ERR_INVALID,
             "ls_pool_atoms_to_pages: bad sizes");
  LS_REQUIRE(dtype == LS_F32 || dtype == LS_BF16 || dtype == LS_F16, LS_ERR_INVALID,
             "ls_pool_atoms_to_pages: unknown dtype %d", dtype);
  const int64_t n = rows * n_pages;
  if (n == 0) return LS_OK;
  LS_REQUIRE(atom_scores && out, LS_ERR_INVALID, "ls_pool_atoms_to_pages: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const dim3 grid((unsigned)((n + 255) / 256));
  if (dtype == LS_BF16)
    hipLaunchKernelGGL(ls_pool_kernel<LS_BF16>, grid, dim3(256), 0, s, (const uint16_t*)atom_scores,
                       rows, n_atoms, row_stride, n_pages, pool_stride, (uint16_t*)out);
  else if (dtype == LS_F16)
    hipLaunchKernelGGL(ls_pool_kernel<LS_F16>, grid, dim3(256), 0, s, (const uint16_t*)atom_scores,
                       rows, n_atoms, row_stride, n_pages, pool_stride, (uint16_t*)out);
  else
    hipLaunchKernelGGL(ls_pool_kernel<LS_F32>, grid, dim3(256), 0, s, (const float*)atom_scores,
                       rows, n_atoms, row_stride, n_pages, pool_stride, (float*)out);
  return ls_check_launch("ls_pool_kernel");
}

extern "C" int ls_forced_page_mask(const int64_t* positions, int64_t n, int64_t num_pages,
                                   int32_t block_size, int32_t init_blocks, int32_t local_blocks,
                                   uint8_t* out, void* stream) {
  LS_REQUIRE(n >= 0 && num_pages >= 0 && block_size > 0, LS_ERR_INVALID,
             "ls_forced_page_mask: bad sizes");
  const int64_t total = n * num_pages;
  if (total == 0) return LS_OK;
  LS_REQUIRE(positions && out, LS_ERR_INVALID, "ls_forced_page_mask: null pointer");
  hipLaunchKernelGGL(ls_forced_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     (hipStream_t)stream, positions, n, num_pages, block_size, init_blocks,
                     local_blocks, out);
  return ls_check_launch("ls_forced_kernel");
}
