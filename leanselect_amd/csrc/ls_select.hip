// LeanSelect prefill selection on gfx950.
//
//   fused weights  q_fused / kv_fused          leanselect/selector.py:144-158
//   q~ = Q . q_fused summed over the GQA group leanselect/selector.py:160-177   (MFMA GEMM)
//   k~ = Kc . kv_fused                         leanselect/selector.py:179-190   (MFMA GEMM)
//   page score = max over a 5-atom window of   leanselect/selector.py:203-214,
//                round(q~ . k~)                leanselect/pages.py:146-187       (MFMA + in-register pool)
//   visibility, forced pages, top-k            leanselect/models/minicpm.py:3094-3142
//
// Rounding follows the reference: fused weights, q~, k~ and atom scores are
// rounded to the activation dtype; a page score is the max of rounded atom
// scores (rounding is monotone, so the max is rounded once).
#include "ls_common.h"
#include "ls_nosa_internal.h"
#include "ls_topk_row.h"

// ---------------------------------------------------------------------------
// Fused weights
// ---------------------------------------------------------------------------

// Reference layout: q_fused[h][d][r*RD + j] = head_mix[h][r] * q_proj[r][d][j].
template <int DT>
__global__ __launch_bounds__(256) void ls_fuse_ref_kernel(
    const float* __restrict__ mix, const float* __restrict__ proj, int heads, int R, int D,
    int RD, typename LsElem<DT>::T* __restrict__ out) {
  const int64_t F = (int64_t)R * RD;
  const int64_t n = (int64_t)heads * D * F;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int f = (int)(i % F);
  const int d = (int)((i / F) % D);
  const int h = (int)(i / (F * D));
  const int r = f / RD, j = f % RD;
  out[i] = LsElem<DT>::from_f(mix[h * R + r] * proj[((int64_t)r * D + d) * RD + j]);
}

// GEMM layout: wt[g][f][s*D + d] = mix[g*gs + s][r] * proj[r][d][j] with f = r*RD + j,
// i.e. the fused weights of one group transposed so the reduction index is
// contiguous.  `heads = G * gs`.
template <int DT>
__global__ __launch_bounds__(256) void ls_fuse_t_kernel(
    const float* __restrict__ mix, const float* __restrict__ proj, int G, int gs, int R, int D,
    int RD, typename LsElem<DT>::T* __restrict__ wt) {
  const int64_t F = (int64_t)R * RD;
  const int64_t K = (int64_t)gs * D;
  const int64_t n = (int64_t)G * F * K;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= n) return;
  const int k = (int)(i % K);
  const int f = (int)((i / K) % F);
  const int g = (int)(i / (K * F));
  const int s = k / D, d = k % D;
  const int r = f / RD, j = f % RD;
  wt[i] = LsElem<DT>::from_f(mix[(g * gs + s) * R + r] * proj[((int64_t)r * D + d) * RD + j]);
}

// ---------------------------------------------------------------------------
// Projection GEMM: out[g][m][f] = sum_k A[m*lda + g*gk + k] * wt[g][f][k].
// 16-bit inputs on v_mfma_f32_16x16x32; each wave owns 32 rows x F columns.
// Operand layout of the 16x16x32 MFMA (lane l, q = l / 16):
//   A: row l%16, reduction slots 8q..8q+7;  B: column l%16, the same slots;
//   D: rows 4q..4q+3, column l%16.
// ---------------------------------------------------------------------------
template <int DT, int FB>
__global__ __launch_bounds__(256) void ls_proj_mfma_kernel(
    const uint16_t* __restrict__ A, int64_t lda, int64_t gk, int64_t M, int K,
    const uint16_t* __restrict__ wt, uint16_t* __restrict__ out) {
  constexpr int F = FB * 16;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int g = blockIdx.y;
  const int64_t m0 = (int64_t)blockIdx.x * 128 + w * 32;
  if (m0 >= M) return;
  const uint16_t* Ag = A + g * gk;
  const uint16_t* Wg = wt + (int64_t)g * F * K;
  const int64_t row0 = min(m0 + r, M - 1), row1 = min(m0 + 16 + r, M - 1);
  const uint16_t* a0p = Ag + row0 * lda + 8 * q;
  const uint16_t* a1p = Ag + row1 * lda + 8 * q;
  const uint16_t* bp = Wg + (int64_t)r * K + 8 * q;

  ls_f32x4 acc0[FB], acc1[FB];
#pragma unroll
  for (int c = 0; c < FB; ++c) {
    acc0[c] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
    acc1[c] = acc0[c];
  }
  for (int k0 = 0; k0 < K; k0 += 32) {
    const ls_u32x4 a0 = ls_load16(a0p + k0);
    const ls_u32x4 a1 = ls_load16(a1p + k0);
#pragma unroll
    for (int c = 0; c < FB; ++c) {
      const ls_u32x4 b = ls_load16(bp + (int64_t)c * 16 * K + k0);
      acc0[c] = LsElem<DT>::mfma(a0, b, acc0[c]);
      acc1[c] = LsElem<DT>::mfma(a1, b, acc1[c]);
    }
  }
  uint16_t* og = out + (int64_t)g * M * F;
#pragma unroll
  for (int c = 0; c < FB; ++c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t ma = m0 + 4 * q + i, mb = m0 + 16 + 4 * q + i;
      if (ma < M) og[ma * F + c * 16 + r] = LsElem<DT>::from_f(acc0[c][i]);
      if (mb < M) og[mb * F + c * 16 + r] = LsElem<DT>::from_f(acc1[c][i]);
    }
  }
}

// Projection GEMM for long A (the q~ projection streams every query row once):
// a workgroup owns 128 rows x F columns, the weight tile of each 128-wide K
// step is staged once in LDS (double buffered, 16-byte chunks XOR-swizzled by
// column) and shared by the four waves, and each wave prefetches its next A
// step while the MFMAs of the current one run.  In slice ks of a K step, lane
// group q takes k = 32ks + 8q .. +7 (both operands), so the four lanes of a
// row read 64 contiguous bytes per load instruction.
// Requires K % 128 == 0.
template <int DT, int FB>
__global__ __launch_bounds__(256, 2) void ls_proj_tile_kernel(
    const uint16_t* __restrict__ A, int64_t lda, int64_t gk, int64_t M, int K,
    const uint16_t* __restrict__ wt, uint16_t* __restrict__ out, int G) {
  constexpr int F = FB * 16;
  constexpr int NB = F * 16 / 256;  // 16-byte weight chunks per thread per K step
  __shared__ ls_u32x4 sB[2][F * 16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  // The groups of one 128-row tile are neighbouring workgroups, so the halves
  // of each row are read close together in time.
  const int g = (int)(blockIdx.x % (unsigned)G);
  const int64_t m0 = (int64_t)(blockIdx.x / (unsigned)G) * 128 + w * 32;
  const uint16_t* Ag = A + g * gk;
  const uint16_t* Wg = wt + (int64_t)g * F * K;
  const uint16_t* a0p = Ag + min(m0 + r, M - 1) * lda + 8 * q;
  const uint16_t* a1p = Ag + min(m0 + 16 + r, M - 1) * lda + 8 * q;
  const int nk = K / 128;

  ls_u32x4 breg[NB];
  auto load_b = [&](int kt) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = tid + 256 * j, f = i >> 4, ch = i & 15;
      breg[j] = ls_load16(Wg + (int64_t)f * K + 128 * kt + 8 * ch);
    }
  };
  auto store_b = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = tid + 256 * j, f = i >> 4, ch = i & 15;
      sB[buf][f * 16 + (ch ^ (f & 15))] = breg[j];
    }
  };
  ls_u32x4 a0[4], a1[4];
  auto load_a = [&](int kt) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      a0[ks] = ls_load16(a0p + 128 * kt + 32 * ks);
      a1[ks] = ls_load16(a1p + 128 * kt + 32 * ks);
    }
  };

  ls_f32x4 acc0[FB], acc1[FB];
#pragma unroll
  for (int c = 0; c < FB; ++c) {
    acc0[c] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
    acc1[c] = acc0[c];
  }
  load_b(0);
  load_a(0);
  store_b(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    ls_u32x4 c0[4], c1[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      c0[ks] = a0[ks];
      c1[ks] = a1[ks];
    }
    if (kt + 1 < nk) {
      load_b(kt + 1);
      load_a(kt + 1);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int c = 0; c < FB; ++c) {
        const ls_u32x4 b = sB[buf][(16 * c + r) * 16 + ((4 * ks + q) ^ r)];
        acc0[c] = LsElem<DT>::mfma(c0[ks], b, acc0[c]);
        acc1[c] = LsElem<DT>::mfma(c1[ks], b, acc1[c]);
      }
    }
    if (kt + 1 < nk) store_b(buf ^ 1);
    __syncthreads();
  }
  if (m0 >= M) return;
  uint16_t* og = out + (int64_t)g * M * F;
#pragma unroll
  for (int c = 0; c < FB; ++c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t ma = m0 + 4 * q + i, mb = m0 + 16 + 4 * q + i;
      if (ma < M) og[ma * F + c * 16 + r] = LsElem<DT>::from_f(acc0[c][i]);
      if (mb < M) og[mb * F + c * 16 + r] = LsElem<DT>::from_f(acc1[c][i]);
    }
  }
}

// Rotary embedding of the query heads fused with the q~ projection
// (producer-side: the rotated rows feed the projection's MFMAs from registers,
// so the projection does not read the queries a second time).  Rotation as
// apply_rotary_pos_emb (leanselect/models/minicpm.py:1027-1070):
//   y[d] = round(x[d] cos[p][d] - x[d + 64] sin[p][d]),
//   y[d + 64] = round(x[d + 64] cos[p][d + 64] + x[d] sin[p][d + 64])  (d < 64)
// with every product and sum rounded to float32 (no fused multiply-add), the
// rotated values written back in place, and the projection computed exactly as
// ls_proj_tile_kernel computes it (same K-step and slice order), so q~ is
// bit-identical to rotating first and projecting after.  A workgroup owns 128
// rows (eight waves of 16, sharing each K step's weight tile in LDS) of one KV
// group; in slice ks of a K step (one head) lane
// group q holds dims 32 ks + 8 q .. +7, so the rotation pairs (ks, ks + 2) sit
// in the same lane, and each lane keeps its row's 64 rotary coefficients.
__device__ __forceinline__ void ls_rope_pair(float x1, float x2, float c1, float c2, float s1,
                                             float s2, float& y1, float& y2) {
#pragma clang fp contract(off)
  y1 = x1 * c1 + (-x2) * s1;
  y2 = x2 * c2 + x1 * s2;
}

#define LS_RP_WAVES 8  // waves (16 rows each) per workgroup of the fused rotary projection

template <int DT, int FB>
__global__ __launch_bounds__(64 * LS_RP_WAVES, 1) void ls_rope_proj_kernel(
    uint16_t* __restrict__ A, int64_t lda, int gs, int64_t M, const int32_t* __restrict__ pos,
    const float* __restrict__ cosb, const float* __restrict__ sinb, int64_t table_rows,
    const uint16_t* __restrict__ wt, uint16_t* __restrict__ out) {
  constexpr int F = FB * 16;
  constexpr int NT = 64 * LS_RP_WAVES;
  constexpr int NB = F * 16 / NT;  // 16-byte weight chunks per thread per K step
  static_assert(NB * NT == F * 16, "weight tile must split evenly over the threads");
  __shared__ ls_u32x4 sB[2][F * 16];
  const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
  const int r = lane & 15, q = lane >> 4;
  const int g = blockIdx.y;
  const int64_t m0 = (int64_t)blockIdx.x * (16 * LS_RP_WAVES) + w * 16;  // the wave's first row
  const int64_t row = m0 + r;                             // this lane's A row
  const bool row_ok = row < M;
  const int64_t rowc = row_ok ? row : M - 1;
  const int K = gs * 128, nk = gs;
  uint16_t* ap = A + rowc * lda + (int64_t)g * K + 8 * q;
  const uint16_t* Wg = wt + (int64_t)g * F * K;

  int64_t p = pos[rowc];
  p = p < 0 ? 0 : (p >= table_rows ? table_rows - 1 : p);  // the host checks the range
  float c1[2][8], c2[2][8], s1[2][8], s2[2][8];
#pragma unroll
  for (int h = 0; h < 2; ++h) {
    const int64_t d0 = p * 128 + 32 * h + 8 * q;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const ls_f32x4 a = *reinterpret_cast<const ls_f32x4*>(cosb + d0 + 4 * i);
      const ls_f32x4 b = *reinterpret_cast<const ls_f32x4*>(cosb + d0 + 64 + 4 * i);
      const ls_f32x4 e = *reinterpret_cast<const ls_f32x4*>(sinb + d0 + 4 * i);
      const ls_f32x4 f = *reinterpret_cast<const ls_f32x4*>(sinb + d0 + 64 + 4 * i);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        c1[h][4 * i + j] = a[j];
        c2[h][4 * i + j] = b[j];
        s1[h][4 * i + j] = e[j];
        s2[h][4 * i + j] = f[j];
      }
    }
  }

  ls_u32x4 breg[NB];
  auto load_b = [&](int kt) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = tid + NT * j, f = i >> 4, ch = i & 15;
      breg[j] = ls_load16(Wg + (int64_t)f * K + 128 * kt + 8 * ch);
    }
  };
  auto store_b = [&](int buf) {
#pragma unroll
    for (int j = 0; j < NB; ++j) {
      const int i = tid + NT * j, f = i >> 4, ch = i & 15;
      sB[buf][f * 16 + (ch ^ (f & 15))] = breg[j];
    }
  };
  ls_u32x4 a[4];  // the row's slices of the next K step (in flight while one is rotated)
  auto load_a = [&](int kt) {
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) a[ks] = ls_load16(ap + 128 * kt + 32 * ks);
  };

  ls_f32x4 acc[FB];
#pragma unroll
  for (int c = 0; c < FB; ++c) acc[c] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
  load_b(0);
  load_a(0);
  store_b(0);
  __syncthreads();
  for (int kt = 0; kt < nk; ++kt) {
    const int buf = kt & 1;
    ls_u32x4 x[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) x[ks] = a[ks];
    if (kt + 1 < nk) {
      load_b(kt + 1);
      load_a(kt + 1);
    }
    // Rotate the head's slices (pairs ks, ks + 2) and write them back.
    ls_u32x4 y[4];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        float lo1, hi1, lo2, hi2;
        const float xa0 = LsElem<DT>::to_f((uint16_t)(x[h][e] & 0xffffu));
        const float xa1 = LsElem<DT>::to_f((uint16_t)(x[h][e] >> 16));
        const float xb0 = LsElem<DT>::to_f((uint16_t)(x[h + 2][e] & 0xffffu));
        const float xb1 = LsElem<DT>::to_f((uint16_t)(x[h + 2][e] >> 16));
        ls_rope_pair(xa0, xb0, c1[h][2 * e], c2[h][2 * e], s1[h][2 * e], s2[h][2 * e], lo1, lo2);
        ls_rope_pair(xa1, xb1, c1[h][2 * e + 1], c2[h][2 * e + 1], s1[h][2 * e + 1],
                     s2[h][2 * e + 1], hi1, hi2);
        y[h][e] = ls_pack2(LsElem<DT>::from_f(lo1), LsElem<DT>::from_f(hi1));
        y[h + 2][e] = ls_pack2(LsElem<DT>::from_f(lo2), LsElem<DT>::from_f(hi2));
      }
    }
    if (row_ok) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        *reinterpret_cast<ls_u32x4*>(ap + 128 * kt + 32 * ks) = y[ks];
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
      for (int c = 0; c < FB; ++c) {
        const ls_u32x4 b = sB[buf][(16 * c + r) * 16 + ((4 * ks + q) ^ r)];
        acc[c] = LsElem<DT>::mfma(y[ks], b, acc[c]);
      }
    }
    if (kt + 1 < nk) store_b(buf ^ 1);
    __syncthreads();
  }
  if (m0 >= M) return;
  uint16_t* og = out + (int64_t)g * M * F;
#pragma unroll
  for (int c = 0; c < FB; ++c) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int64_t mo = m0 + 4 * q + i;
      if (mo < M) og[mo * F + c * 16 + r] = LsElem<DT>::from_f(acc[c][i]);
    }
  }
}

// float32 projection on the vector ALU (the reference's float32 path).
__global__ __launch_bounds__(256) void ls_proj_f32_kernel(
    const float* __restrict__ A, int64_t lda, int64_t gk, int64_t M, int K, int F,
    const float* __restrict__ wt, float* __restrict__ out) {
  const int g = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * F) return;
  const int64_t m = i / F;
  const int f = (int)(i % F);
  const float* a = A + m * lda + g * gk;
  const float* b = wt + ((int64_t)g * F + f) * K;
  float acc = 0.f;
  for (int k = 0; k < K; ++k) acc = fmaf(a[k], b[k], acc);
  out[(int64_t)g * M * F + i] = acc;
}

// ---------------------------------------------------------------------------
// Selection plan: blk_off[b] = sum_{b' < b} ceil(len_q(b') / block_size).
// ---------------------------------------------------------------------------
__global__ void ls_select_plan_kernel(const int32_t* __restrict__ cu_q, int batch, int bs,
                                      int32_t* __restrict__ blk_off) {
  if (threadIdx.x != 0 || blockIdx.x != 0) return;
  // blk_off[0..batch]: query blocks before each sequence; then sb_off[0..batch]
  // (at blk_off + batch + 1): groups of four query blocks before each sequence.
  int32_t* sb_off = blk_off + batch + 1;
  int32_t acc = 0, acc4 = 0;
  blk_off[0] = 0;
  sb_off[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int len = cu_q[b + 1] - cu_q[b];
    const int nb = len > 0 ? (len + bs - 1) / bs : 0;
    acc += nb;
    acc4 += (nb + 3) / 4;
    blk_off[b + 1] = acc;
    sb_off[b + 1] = acc4;
  }
}

// ---------------------------------------------------------------------------
// Page scores on MFMA.  One workgroup = one 64-token query block of one KV
// group; the block's atom range is split into four contiguous quarters, one
// per wave, and every wave scores all 64 tokens (four 16-token MFMA column
// blocks), so each k~ fragment is read once per workgroup and feeds four
// MFMAs.  Atoms are the MFMA rows and tokens the columns: after one 16-atom
// step lane l (q = l/16) holds the four atoms 16j+4q..16j+4q+3 of page 4j+q
// for token l%16; the fifth atom of the window (16j+4q-1) is the last atom of
// the lane group below, one rotate away, or the carry from the previous step
// for q == 0.
//
// Modes (LS_SCORE_*): SELECT: per sequence, only the non-forced visible pages
// [init_blocks, qp - local_blocks - 1] of the block are scored, into the
// scratch rows P[g][t][*].  ALL: per sequence, every page whose window holds
// an atom (p <= A_b / 4, below the page-column count), causal or not (the NOSA
// shortlist ranks them all).  FULL: a single sequence, every page, out[g][n][*].
// ---------------------------------------------------------------------------
#define LS_SCORE_FULL 0
#define LS_SCORE_SELECT 1
#define LS_SCORE_ALL 2

template <int DT, int KS, int MODE>
__global__ __launch_bounds__(256, KS <= 4 ? 3 : 2) void ls_score_mfma_kernel(
    const uint16_t* __restrict__ qt, int64_t Nq, const uint16_t* __restrict__ kt, int64_t Na,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_a,
    const int32_t* __restrict__ blk_off, int batch, int64_t n_blk_launch, int init_blocks,
    int local_blocks, int64_t full_seq_len, uint16_t* __restrict__ out, int64_t out_stride) {
  constexpr int F = KS * 32;
  // Each wave stages 16 steps of its scores (64 tokens x 64 pages) here and
  // then writes whole 128-byte row segments; rows are padded to 68 halves so
  // the per-step 16-bit writes of the sixteen token rows hit distinct banks.
  constexpr int SP = 68;
  __shared__ __align__(16) uint16_t s_out[4][64 * SP];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int g = blockIdx.y;

  int64_t tq0, tq_end, a0, n_atoms;
  int p_lo, p_hi;
  if constexpr (MODE != LS_SCORE_FULL) {
    const int64_t ir = n_blk_launch - 1 - (int64_t)blockIdx.x;  // longest rows first
    if (ir >= blk_off[batch]) return;
    const int b = ls_find_segment(blk_off, batch, ir);
    const int qb = (int)(ir - blk_off[b]);
    tq0 = (int64_t)cu_q[b] + (int64_t)64 * qb;
    tq_end = min(tq0 + 64, (int64_t)cu_q[b + 1]);
    a0 = cu_a[b];
    n_atoms = (int64_t)cu_a[b + 1] - a0;
    if constexpr (MODE == LS_SCORE_SELECT) {
      p_lo = init_blocks;
      // (Clamped to the row's columns: a max_seqlen_q below a sequence's
      // length then gives wrong pages, never a write outside the row.)
      p_hi = (int)min((int64_t)(qb - local_blocks - 1), out_stride - 1);
    } else {  // full_seq_len carries the page-column count in this mode
      p_lo = 0;
      p_hi = (int)min(n_atoms / 4, full_seq_len - 1);
    }
  } else {
    tq0 = 64LL * blockIdx.x;
    tq_end = min(tq0 + 64, Nq);
    a0 = 0;
    n_atoms = Na;
    p_lo = 0;
    p_hi = (int)((full_seq_len + 63) / 64) - 1;
  }
  if (n_atoms <= 0 || p_lo > p_hi) return;

  // This wave's share of the block's 16-atom steps.
  const int j_lo = p_lo >> 2, j_hi = p_hi >> 2;
  const int n_j = j_hi - j_lo + 1;
  const int jw_lo = j_lo + (n_j * w) / 4, jw_hi = j_lo + (n_j * (w + 1)) / 4 - 1;
  if (jw_lo > jw_hi) return;

  // q~^T fragments (B operand) of the four 16-token column blocks.
  ls_u32x4 qf[4][KS];
  int64_t tok[4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    tok[tb] = min(tq0 + 16 * tb + r, tq_end - 1);
    const uint16_t* qrow = qt + ((int64_t)g * Nq + tok[tb]) * F + 8 * q;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[tb][ks] = ls_load16(qrow + 32 * ks);
  }

  // Pages this wave writes, and whether 4-page pieces of a row may be stored
  // as one 8-byte word.
  const int pa = max(p_lo, 4 * jw_lo), pb = min(p_hi, 4 * jw_hi + 3);
  const bool wide = (out_stride & 3) == 0 && ((uintptr_t)out & 7) == 0;
  uint16_t* const so = s_out[w];
  // Writes the staged steps of batch jb (pages 64 jb .. 64 jb + 63) that fall
  // in [pa, pb] for the block's valid tokens: lane (token 4 it + lane / 16,
  // piece lane % 16) stores pages 64 jb + 4 piece .. + 3.
  auto flush = [&](int jb) {
    const int pg0 = 64 * jb;
    const int fa = max(pa, pg0), fb = min(pb, pg0 + 63);
    if (fa > fb) return;
    const int pc = lane & 15, pp = pg0 + 4 * pc;
    const bool full = wide && pp >= fa && pp + 3 <= fb;
    const bool part = !full && pp <= fb && pp + 3 >= fa;
#pragma unroll 4
    for (int it = 0; it < 16; ++it) {
      const int tk = 4 * it + (lane >> 4);
      if (tq0 + tk >= tq_end || !(full || part)) continue;
      const uint2 v = *reinterpret_cast<const uint2*>(so + tk * SP + 4 * pc);
      uint16_t* dst = out + ((int64_t)g * Nq + tq0 + tk) * out_stride + pp;
      if (full) {
        *reinterpret_cast<uint2*>(dst) = v;
      } else {
        const uint16_t h[4] = {(uint16_t)(v.x & 0xffffu), (uint16_t)(v.x >> 16),
                               (uint16_t)(v.y & 0xffffu), (uint16_t)(v.y >> 16)};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (pp + i >= fa && pp + i <= fb) dst[i] = h[i];
      }
    }
  };

  const uint16_t* kbase = kt + ((int64_t)g * Na + a0) * F + 8 * q;
  float carry[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  const int j_first = jw_lo > 0 ? jw_lo - 1 : 0;  // one step early primes the carry
  const int n_at = (int)n_atoms;
  auto load_k = [&](ls_u32x4 (&kf)[KS], int j) {
    const uint16_t* kp = kbase + (int64_t)min(16 * j + r, n_at - 1) * F;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[ks] = ls_load16(kp + 32 * ks);
  };
  // Prefetch distance in steps: two where a third fragment buffer fits in the
  // register budget, one for the widest routers.
  constexpr int PD = KS <= 6 ? 2 : 1;
  // One 16-atom step on k~ fragments kc, prefetching the fragments of step
  // j + PD into kn.  The prefetch is unconditional (load_k clamps its rows, so
  // steps past the end reread the last atom): a branch around it would make
  // the compiler's wait counting conservative, and every step would then wait
  // for the stores of the previous ones.
  auto step = [&](int j, const ls_u32x4 (&kc)[KS], ls_u32x4 (&kn)[KS]) {
    load_k(kn, j + PD);
    ls_f32x4 acc[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      acc[tb] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc[tb] = LsElem<DT>::mfma(kc[ks], qf[tb][ks], acc[tb]);
    }
    const int atom0 = 16 * j + 4 * q;
    if (16 * j + 15 >= n_at) {  // uniform: only the last step has atoms past the end
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (atom0 + i >= n_at) acc[tb][i] = -INFINITY;
    }
    // Atom 4q - 1 of each page comes from the lane group below; the four
    // cross-lane reads are issued together, so their latencies overlap.
    float rot[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) rot[tb] = ls_shfl(acc[tb][3], (lane - 16) & 63);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const float m4 = ls_fmax_nan(ls_fmax_nan(acc[tb][0], acc[tb][1]), ls_fmax_nan(acc[tb][2], acc[tb][3]));
      const float prev = q == 0 ? carry[tb] : rot[tb];
      carry[tb] = rot[tb];
      so[(16 * tb + r) * SP + 4 * (j & 15) + q] = LsElem<DT>::from_f(ls_canon_nan(ls_fmax_nan(m4, prev)));
    }
    if ((j & 15) == 15 || j == jw_hi) flush(j >> 4);
  };
  // PD + 1 fragment buffers used in turn (no register copies between steps).
  int j = j_first;
  if constexpr (PD == 2) {
    ls_u32x4 kA[KS], kB[KS], kC[KS];
    load_k(kA, j_first);
    load_k(kB, j_first + 1);
    for (; j + 2 <= jw_hi; j += 3) {
      step(j, kA, kC);
      step(j + 1, kB, kA);
      step(j + 2, kC, kB);
    }
    if (j <= jw_hi) step(j, kA, kC);
    if (j + 1 <= jw_hi) step(j + 1, kB, kA);
  } else {
    ls_u32x4 kA[KS], kB[KS];
    load_k(kA, j_first);
    for (; j + 1 <= jw_hi; j += 2) {
      step(j, kA, kB);
      step(j + 1, kB, kA);
    }
    if (j <= jw_hi) step(j, kA, kB);
  }
}

// Page scores on MFMA for router widths of 128 and 256 (KS 4 and 8), with the
// k~ panel shared through LDS.  One workgroup = four consecutive 64-token query
// blocks of one sequence and KV group, one per wave; all four walk the same
// 16-atom steps (a wave past its own last page only keeps staging), so each
// step's 16 k~ rows are read from global memory once per workgroup, by direct
// global->LDS loads, four steps per batch, double buffered.  In LDS, 16-byte
// chunk c of row R sits at position c ^ (R & 15), so the sixteen lanes of an
// MFMA operand read hit distinct bank groups.  Scoring, the five-atom page max
// and the staged row writes are those of ls_score_mfma_kernel, per wave.
template <int DT, int KS, int MODE>
__global__ __launch_bounds__(256, KS <= 4 ? 3 : 2) void ls_score_panel_kernel(
    const uint16_t* __restrict__ qt, int64_t Nq, const uint16_t* __restrict__ kt, int64_t Na,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_a,
    const int32_t* __restrict__ sb_off, int batch, int64_t n_sb_launch, int init_blocks,
    int local_blocks, int64_t full_seq_len, uint16_t* __restrict__ out, int64_t out_stride) {
  static_assert(KS == 4 || KS == 8, "the chunk swizzle needs 16 or 32 chunks per row");
  constexpr int F = KS * 32;
  constexpr int ROWB = F * 2;          // bytes of one k~ row
  constexpr int STEPB = 16 * ROWB;     // one 16-atom step
  constexpr int NSTEP = 4;             // steps per staged batch
  constexpr int BATCHB = NSTEP * STEPB;
  constexpr int SP = 68;
  __shared__ __align__(16) uint8_t s_k[2][BATCHB];
  __shared__ __align__(16) uint16_t s_out[4][64 * SP];
  __shared__ int s_jhi[4];
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int r = lane & 15, q = lane >> 4;
  const int g = blockIdx.y;

  int64_t tq0, tq_end, a0, n_atoms;
  int p_lo, p_hi;
  if constexpr (MODE != LS_SCORE_FULL) {
    const int64_t isb = n_sb_launch - 1 - (int64_t)blockIdx.x;  // longest rows first
    if (isb >= sb_off[batch]) return;
    const int b = ls_find_segment(sb_off, batch, isb);
    const int qb = 4 * (int)(isb - sb_off[b]) + w;
    tq0 = (int64_t)cu_q[b] + (int64_t)64 * qb;
    tq_end = min(tq0 + 64, (int64_t)cu_q[b + 1]);
    a0 = cu_a[b];
    n_atoms = (int64_t)cu_a[b + 1] - a0;
    if constexpr (MODE == LS_SCORE_SELECT) {
      p_lo = init_blocks;
      // (Clamped to the row's columns: a max_seqlen_q below a sequence's
      // length then gives wrong pages, never a write outside the row.)
      p_hi = (int)min((int64_t)(qb - local_blocks - 1), out_stride - 1);
    } else {  // full_seq_len carries the page-column count in this mode
      p_lo = 0;
      p_hi = (int)min(n_atoms / 4, full_seq_len - 1);
    }
  } else {
    tq0 = 64LL * (4LL * blockIdx.x + w);
    tq_end = min(tq0 + 64, Nq);
    a0 = 0;
    n_atoms = Na;
    p_lo = 0;
    p_hi = (int)((full_seq_len + 63) / 64) - 1;
  }
  // p_lo, a0 and n_atoms are the same for the four waves.
  const bool active = tq0 < tq_end && n_atoms > 0 && p_lo <= p_hi;
  const int jw_hi = active ? (p_hi >> 2) : -1;
  if (lane == 0) s_jhi[w] = jw_hi;
  __syncthreads();
  const int j_hi = max(max(s_jhi[0], s_jhi[1]), max(s_jhi[2], s_jhi[3]));
  if (j_hi < 0) return;  // no wave has a page to score (uniform)
  const int j_lo = p_lo >> 2;
  const int j_first = j_lo > 0 ? j_lo - 1 : 0;  // one step early primes the carry
  const int n_at = (int)n_atoms;

  // q~^T fragments (B operand) of the wave's four 16-token column blocks.
  ls_u32x4 qf[4][KS];
  int64_t tok[4];
#pragma unroll
  for (int tb = 0; tb < 4; ++tb) {
    tok[tb] = active ? min(tq0 + 16 * tb + r, tq_end - 1) : 0;
    const uint16_t* qrow = qt + ((int64_t)g * Nq + tok[tb]) * F + 8 * q;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[tb][ks] = active ? ls_load16(qrow + 32 * ks) : ls_u32x4{0u, 0u, 0u, 0u};
  }

  // Staged score rows, written as whole 128-byte segments (see ls_score_mfma_kernel).
  const int pa = p_lo, pb = p_hi;
  const bool wide = (out_stride & 3) == 0 && ((uintptr_t)out & 7) == 0;
  uint16_t* const so = s_out[w];
  auto flush = [&](int jb) {
    const int pg0 = 64 * jb;
    const int fa = max(pa, pg0), fb = min(pb, pg0 + 63);
    if (fa > fb) return;
    const int pc = lane & 15, pp = pg0 + 4 * pc;
    const bool full = wide && pp >= fa && pp + 3 <= fb;
    const bool part = !full && pp <= fb && pp + 3 >= fa;
    // All sixteen staged pieces are read first, so their LDS latencies overlap.
    uint2 vs[16];
#pragma unroll
    for (int it = 0; it < 16; ++it)
      vs[it] = *reinterpret_cast<const uint2*>(so + (4 * it + (lane >> 4)) * SP + 4 * pc);
#pragma unroll
    for (int it = 0; it < 16; ++it) {
      const int tk = 4 * it + (lane >> 4);
      if (tq0 + tk >= tq_end || !(full || part)) continue;
      const uint2 v = vs[it];
      uint16_t* dst = out + ((int64_t)g * Nq + tq0 + tk) * out_stride + pp;
      if (full) {
        *reinterpret_cast<uint2*>(dst) = v;
      } else {
        const uint16_t h[4] = {(uint16_t)(v.x & 0xffffu), (uint16_t)(v.x >> 16),
                               (uint16_t)(v.y & 0xffffu), (uint16_t)(v.y >> 16)};
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (pp + i >= fa && pp + i <= fb) dst[i] = h[i];
      }
    }
  };

  // Batch of steps jb .. jb + NSTEP - 1 into buffer buf: 1 KB per load, lane l
  // of load i covering batch bytes 1024 i + 16 l (row R, position c), from
  // logical chunk c ^ (R & 15) of atom 16 jb + R (clamped to the last atom).
  const uint8_t* kg = reinterpret_cast<const uint8_t*>(kt + ((int64_t)g * Na + a0) * F);
  const uint32_t sk0 = (uint32_t)(uintptr_t)(ls_lds_void*)&s_k[0][0];
  auto stage = [&](int jb, int buf) {
#pragma unroll
    for (int i = w; i < BATCHB / 1024; i += 4) {
      const int byte = 1024 * i + 16 * lane;
      const int row = byte / ROWB, pos = (byte % ROWB) / 16;
      const int atom = min(16 * jb + row, n_at - 1);
      const int chunk = pos ^ (row & 15);
      ls_dma16(kg, (uint32_t)(atom * ROWB + 16 * chunk), sk0 + (uint32_t)(buf * BATCHB + 1024 * i));
    }
  };

  float carry[4] = {-INFINITY, -INFINITY, -INFINITY, -INFINITY};
  auto read_k = [&](ls_u32x4 (&kf)[KS], const uint8_t* kb) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      kf[ks] = *reinterpret_cast<const ls_u32x4*>(kb + r * ROWB + 16 * ((4 * ks + q) ^ r));
  };
  auto step_mfma = [&](const ls_u32x4 (&kf)[KS], ls_f32x4 (&acc)[4]) {
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      acc[tb] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc[tb] = LsElem<DT>::mfma(kf[ks], qf[tb][ks], acc[tb]);
    }
  };
  // The page maxima of step j from its scores acc (atoms past the end are
  // masked when `tail`), staged in LDS.
  auto step_epi = [&](int j, ls_f32x4 (&acc)[4], bool tail) {
    const int atom0 = 16 * j + 4 * q;
    if (tail) {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (atom0 + i >= n_at) acc[tb][i] = -INFINITY;
    }
    float rot[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) rot[tb] = ls_shfl(acc[tb][3], (lane - 16) & 63);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const float m4 = ls_fmax_nan(ls_fmax_nan(acc[tb][0], acc[tb][1]), ls_fmax_nan(acc[tb][2], acc[tb][3]));
      const float prev = q == 0 ? carry[tb] : rot[tb];
      carry[tb] = rot[tb];
      so[(16 * tb + r) * SP + 4 * (j & 15) + q] = LsElem<DT>::from_f(ls_canon_nan(ls_fmax_nan(m4, prev)));
    }
  };
  auto step = [&](int j, const ls_u32x4 (&kf)[KS]) {
    ls_f32x4 acc[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      acc[tb] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) acc[tb] = LsElem<DT>::mfma(kf[ks], qf[tb][ks], acc[tb]);
    }
    const int atom0 = 16 * j + 4 * q;
    if (16 * j + 15 >= n_at) {  // uniform: only the last step has atoms past the end
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int i = 0; i < 4; ++i)
          if (atom0 + i >= n_at) acc[tb][i] = -INFINITY;
    }
    // Atom 4q - 1 of each page comes from the lane group below; the four
    // cross-lane reads are issued together, so their latencies overlap.
    float rot[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) rot[tb] = ls_shfl(acc[tb][3], (lane - 16) & 63);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      const float m4 = ls_fmax_nan(ls_fmax_nan(acc[tb][0], acc[tb][1]), ls_fmax_nan(acc[tb][2], acc[tb][3]));
      const float prev = q == 0 ? carry[tb] : rot[tb];
      carry[tb] = rot[tb];
      so[(16 * tb + r) * SP + 4 * (j & 15) + q] = LsElem<DT>::from_f(ls_canon_nan(ls_fmax_nan(m4, prev)));
    }
  };

  // Batches start at multiples of NSTEP, so a 64-page block (16 steps) always
  // ends on a batch's last step and is written out after it.
  const int jb0 = j_first & ~(NSTEP - 1);
  stage(jb0, 0);
  int buf = 0;
  for (int jb = jb0; jb <= j_hi; jb += NSTEP, buf ^= 1) {
    // This batch has landed (every wave waited for its own loads), and every
    // wave is done with the other buffer, which the next batch may overwrite.
    LS_WAIT_VMCNT(0);
    __syncthreads();
    if (jb + NSTEP <= j_hi) stage(jb + NSTEP, buf ^ 1);
    // Each step's k~ fragments are read from LDS while the step before it
    // computes (two fragment sets used in turn).
    ls_u32x4 kf[2][KS];
    read_k(kf[0], &s_k[buf][0]);
    if (jb >= j_first && jb + NSTEP - 1 <= jw_hi && 16 * (jb + NSTEP) <= n_at) {
      // Every step of the batch is the wave's and has all its atoms: branch
      // free, with step st + 1's MFMAs issued before step st's maxima, so the
      // vector work overlaps the matrix core.
      ls_f32x4 acc[2][4];
      step_mfma(kf[0], acc[0]);
      read_k(kf[1], &s_k[buf][STEPB]);
#pragma unroll
      for (int st = 0; st < NSTEP; ++st) {
        if (st + 1 < NSTEP) step_mfma(kf[(st + 1) & 1], acc[(st + 1) & 1]);
        if (st + 2 < NSTEP) read_k(kf[st & 1], &s_k[buf][(st + 2) * STEPB]);
        step_epi(jb + st, acc[st & 1], false);
      }
    } else {
#pragma unroll
      for (int st = 0; st < NSTEP; ++st) {
        const int j = jb + st;
        if (st + 1 < NSTEP) read_k(kf[(st + 1) & 1], &s_k[buf][(st + 1) * STEPB]);
        if (j >= j_first && j <= jw_hi) step(j, kf[st & 1]);
      }
    }
    // The wave's last step, or a block's last step, was in this batch.
    const int jl = min(jb + NSTEP - 1, jw_hi);
    if (jl >= jb && jl >= j_first && ((jl & 15) == 15 || jl == jw_hi)) flush(jl >> 4);
  }
}

// float32 page scores on the vector ALU: one thread per (group, token, page).
// General pooling stride s = block_size / kernel_stride.
template <int MODE>
__global__ __launch_bounds__(256) void ls_score_f32_kernel(
    const float* __restrict__ qt, int64_t Nq, const float* __restrict__ kt, int64_t Na, int F,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_a, int batch,
    int init_blocks, int local_blocks, int block_size, int s, int64_t full_seq_len,
    int64_t n_pages_cols, float* __restrict__ out, int64_t out_stride) {
  const int g = blockIdx.y;
  const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= Nq * n_pages_cols) return;
  const int64_t t = i / n_pages_cols;
  const int p = (int)(i % n_pages_cols);
  int64_t a0, n_atoms;
  if constexpr (MODE == LS_SCORE_SELECT) {
    const int b = ls_find_segment(cu_q, batch, t);
    const int qp = (int)((t - cu_q[b]) / block_size);
    if (p < init_blocks || p > qp - local_blocks - 1) return;
    a0 = cu_a[b];
    n_atoms = (int64_t)cu_a[b + 1] - a0;
  } else if constexpr (MODE == LS_SCORE_ALL) {
    const int b = ls_find_segment(cu_q, batch, t);
    a0 = cu_a[b];
    n_atoms = (int64_t)cu_a[b + 1] - a0;
    if ((int64_t)p > n_atoms / s) return;
  } else {
    if (p >= (full_seq_len + block_size - 1) / block_size) return;
    a0 = 0;
    n_atoms = Na;
  }
  if (n_atoms <= 0) return;
  const float* qrow = qt + ((int64_t)g * Nq + t) * F;
  float best = -INFINITY;
  for (int64_t a = (int64_t)p * s - 1; a < (int64_t)p * s + s; ++a) {
    if (a < 0 || a >= n_atoms) continue;
    const float* krow = kt + ((int64_t)g * Na + a0 + a) * F;
    float acc = 0.f;
    for (int f = 0; f < F; ++f) acc = fmaf(qrow[f], krow[f], acc);
    best = ls_fmax_nan(best, acc);
  }
  out[((int64_t)g * Nq + t) * out_stride + p] = ls_canon_nan(best);
}


// Number of NaN keys (keys above rule.hi) among the cn candidate scores at
// P[base ..] of one row; every lane of the wave calls it and gets the count.
template <bool KEY32>
__device__ __forceinline__ int ls_count_nan_keys(const void* __restrict__ P, int64_t base, int cn,
                                                 int lane, const LsInvalidKeys& rule) {
  int n = 0;
  for (int c0 = 0; c0 < cn; c0 += 64) {
    const int c = c0 + lane;
    uint32_t k = 0u;
    if (c < cn) {
      if constexpr (KEY32) k = ls_order_key32(((const uint32_t*)P)[base + c]);
      else k = ls_order_key16(((const uint16_t*)P)[base + c]);
    }
    n += __popcll(__ballot(k > rule.hi));
  }
  return n;
}

// Selection of one row in the reference's order (minicpm.py:3124-3141): the
// visible pages are ranked by score with the forced pages at +inf, and
// torch.topk ranks NaN above +inf; the chosen pages with a NaN or -inf score
// become -1.  Rows therefore normally hold the forced pages (sink pages, then
// the local window) plus the top kk of the other visible pages, written in
// page order; NaN scores (canonical, keys above rule.hi) displace forced pages
// only when there are more of them than kk, in which case the forced pages
// keep the slots left after the NaN ones (the lowest forced pages first, as
// the ties at +inf resolve to the lower page) and the others become -1.
// With bf16 set (bf16 page scores) long rows try ls_topk_select16_bf16 first.
// At least six waves per SIMD: the rows' latency chains (row setup, loads,
// stores) overlap across waves.
template <int KPL, bool KEY32>
__global__ __launch_bounds__(256, 6) void ls_topk_kernel(
    const void* __restrict__ P, int64_t p_stride, const int32_t* __restrict__ cu_q,
    const int32_t* __restrict__ cu_a, int batch, int64_t total_q, int G, int take,
    int init_blocks, int local_blocks, int block_size, LsInvalidKeys rule, int bf16,
    int32_t* __restrict__ topk_idx) {
  __shared__ uint32_t s_scr[4][320];  // per-wave gather space of the k-th key search
  const int lane = threadIdx.x & 63;
  // The wave index is uniform: keep the row and everything derived from it scalar.
  // (Grid: x = groups of four query rows, y = KV group.)
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int g = blockIdx.y;
  const int64_t t = (int64_t)blockIdx.x * 4 + wv;
  if (t >= total_q) return;
  const int64_t row = (int64_t)g * total_q + t;
  int32_t* orow = topk_idx + row * take;
  uint32_t* const scr = s_scr[wv];
  const int b = ls_find_segment(cu_q, batch, t);
  const int64_t tr = t - cu_q[b];
  const int lq = cu_q[b + 1] - cu_q[b];
  const int n_atoms = cu_a[b + 1] - cu_a[b];
  if (n_atoms <= 0) {
    for (int i = lane; i < take; i += 64) orow[i] = -1;
    return;
  }
  const int qp = (int)(tr / block_size);
  const int n_pages = (lq + block_size - 1) / block_size;
  const int take_b = min(take, n_pages);
  const int n_valid = min(take_b, qp + 1);
  const int lo_end = min(init_blocks, qp + 1);
  const int hi_start = max(qp - local_blocks, lo_end);
  const int n_forced = lo_end + (qp + 1 - hi_start);
  // (Clamped to the row's columns, as the scoring is.)
  const int cn = (int)max((int64_t)0, min((int64_t)(hi_start - lo_end), p_stride - lo_end));
  const int64_t base = row * p_stride + lo_end;
  if (n_forced >= n_valid) {
    // The budget holds forced pages only: the first n_valid of them in page
    // order, after any NaN-scored other pages (emitted as -1).
    const int n_nan = cn > 0 ? ls_count_nan_keys<KEY32>(P, base, cn, lane, rule) : 0;
    const int n_keep = max(0, n_valid - n_nan);
    for (int i = lane; i < take; i += 64)
      orow[i] = i >= n_keep ? -1 : (i < lo_end ? i : hi_start + (i - lo_end));
    return;
  }
  const int kk = n_valid - n_forced;

  // One pass over the row's slots: sink pages [0, lo_end), the local pages
  // [hi_pos, n_valid) and -1 past n_valid; the selection writes the rest.
  const int hi_pos = lo_end + kk;
  for (int i = lane; i < take; i += 64) {
    if (i < lo_end || i >= hi_pos)
      orow[i] = i < lo_end ? i : (i < n_valid ? hi_start + (i - hi_pos) : -1);
  }

  // Candidates in registers, NS slots of 64; the row's slot count is uniform,
  // so the branch picks one straight-line body per wave.
  auto select = [&]() -> uint32_t {
    if constexpr (!KEY32) {
      uint32_t T;
      if (bf16 && ls_topk_select16_bf16<KPL>((const uint16_t*)P + base, cn, kk, lo_end, lane,
                                               orow, scr, INT32_MAX, rule, T))
        return T;
      return ls_topk_select16<KPL>(P, base, cn, kk, lo_end, lane, orow, scr, INT32_MAX, rule);
    } else {
      const int n_slots = (cn + 63) >> 6;
#define LS_TOPK32_CASE(N)                                                                      \
      if (n_slots <= (N) || KPL <= (N))                                                        \
        return ls_topk_row<(KPL < (N) ? KPL : (N)), true>(P, base, cn, kk, lo_end, lane, orow, \
                                                          scr, INT32_MAX, rule);
      LS_TOPK32_CASE(1)
      LS_TOPK32_CASE(2)
      LS_TOPK32_CASE(4)
      LS_TOPK32_CASE(8)
      LS_TOPK32_CASE(16)
      LS_TOPK32_CASE(32)
      LS_TOPK32_CASE(64)
#undef LS_TOPK32_CASE
      return ls_topk_row<KPL, true>(P, base, cn, kk, lo_end, lane, orow, scr, INT32_MAX, rule);
    }
  };
  const uint32_t T = select();
  if (T > rule.hi) {
    // The kk-th key is NaN: kk or more NaN-scored pages, all chosen (as -1).
    // Beyond kk of them they displace forced pages from the end of the page
    // order.  (Rare; the forced pages written above are rewritten once their
    // stores have completed.)
    const int n_nan = ls_count_nan_keys<KEY32>(P, base, cn, lane, rule);
    const int n_keep = max(0, n_valid - n_nan);
    if (n_keep < n_forced) {
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
      for (int f = n_keep + lane; f < n_forced; f += 64)
        orow[f < lo_end ? f : hi_pos + (f - lo_end)] = -1;
    }
  }
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {

struct WsLayout {
  size_t wq, wk, qt, kt, blk, p, total;
  int64_t p_stride;
};

WsLayout ws_layout(int64_t total_q, int64_t total_atoms, int batch, int H, int G, int D, int F,
                   int max_pages, int eb) {
  WsLayout L;
  size_t off = 0;
  L.wq = off; off += ls_align256((size_t)H * D * F * eb);
  L.wk = off; off += ls_align256((size_t)G * D * F * eb);
  L.qt = off; off += ls_align256((size_t)G * total_q * F * eb);
  L.kt = off; off += ls_align256((size_t)G * total_atoms * F * eb);
  L.blk = off; off += ls_align256((size_t)(batch + 1) * 2 * 4);
  L.p_stride = ((int64_t)max_pages + 63) & ~(int64_t)63;
  L.p = off; off += ls_align256((size_t)G * total_q * L.p_stride * eb);
  L.total = off;
  return L;
}

// The NOSA selection adds the per-sequence CIS page offsets and the CIS page
// scores cpg[g][*] (at most total_atoms / 4 + batch pages per group).
struct NosaWsLayout {
  WsLayout L;
  size_t pg, cpg, order, total;
  int64_t cpg_stride, n_blk;
};

NosaWsLayout nosa_ws_layout(int64_t total_q, int64_t total_atoms, int batch, int H, int G, int D,
                            int F, int out_len, int eb) {
  NosaWsLayout N;
  N.L = ws_layout(total_q, total_atoms, batch, H, G, D, F, out_len, eb);
  size_t off = N.L.total;
  N.pg = off; off += ls_align256((size_t)(batch + 2) * 4);
  N.cpg_stride = (total_atoms / 4 + batch + 63) & ~(int64_t)63;
  N.cpg = off; off += ls_align256((size_t)G * N.cpg_stride * 4);
  // The query blocks' stage-2 page orders (64-row blocks: block_size 64).
  N.n_blk = (total_q + 63) / 64 + batch;
  N.order = off; off += ls_align256(ls_nosa_order_bytes(N.n_blk, G, LS_NOSA_ORDER_STRIDE));
  N.total = off;
  return N;
}

int check_dims(const char* who, int H, int G, int D, int R, int RD, int dtype) {
  LS_REQUIRE(H > 0 && G > 0 && D > 0 && R > 0 && RD > 0, LS_ERR_INVALID, "%s: bad sizes", who);
  LS_REQUIRE(H % G == 0, LS_ERR_INVALID, "%s: num_heads must be divisible by num_kv_heads", who);
  LS_REQUIRE(R <= H, LS_ERR_INVALID, "%s: router_heads cannot exceed num_heads", who);
  LS_REQUIRE(dtype == LS_F32 || dtype == LS_BF16 || dtype == LS_F16, LS_ERR_INVALID,
             "%s: unknown dtype %d", who, dtype);
  if (dtype != LS_F32) {
    const int F = R * RD;
    LS_REQUIRE(D % 32 == 0 && F % 32 == 0 && F <= 256, LS_ERR_UNSUPPORTED,
               "%s: 16-bit path needs head_dim %% 32 == 0 and router width in {32..256} "
               "step 32 (got D=%d F=%d)", who, D, F);
  }
  return LS_OK;
}

template <int DT>
int launch_fuse_t(const float* mix, const float* proj, int G, int gs, int R, int D, int RD,
                  void* wt, hipStream_t s) {
  const int64_t n = (int64_t)G * gs * D * R * RD;
  hipLaunchKernelGGL(ls_fuse_t_kernel<DT>, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s,
                     mix, proj, G, gs, R, D, RD, (typename LsElem<DT>::T*)wt);
  return ls_check_launch("ls_fuse_t_kernel");
}

int fuse_t(int dtype, const float* mix, const float* proj, int G, int gs, int R, int D, int RD,
           void* wt, hipStream_t s) {
  switch (dtype) {
    case LS_BF16: return launch_fuse_t<LS_BF16>(mix, proj, G, gs, R, D, RD, wt, s);
    case LS_F16: return launch_fuse_t<LS_F16>(mix, proj, G, gs, R, D, RD, wt, s);
    default: return launch_fuse_t<LS_F32>(mix, proj, G, gs, R, D, RD, wt, s);
  }
}

template <int DT>
int launch_proj16(const void* A, int64_t lda, int64_t gk, int64_t M, int K, int F, int G,
                  const void* wt, void* out, hipStream_t s) {
  const dim3 grid((unsigned)((M + 127) / 128), G);
  const uint16_t* a = (const uint16_t*)A;
  const uint16_t* w = (const uint16_t*)wt;
  uint16_t* o = (uint16_t*)out;
  if (K % 128 == 0 && F % 64 == 0 && F <= 128) {  // LDS-staged weight tiles
    const dim3 tgrid((unsigned)((M + 127) / 128 * G));
    if (F == 64)
      hipLaunchKernelGGL((ls_proj_tile_kernel<DT, 4>), tgrid, dim3(256), 0, s, a, lda, gk, M, K, w, o, G);
    else
      hipLaunchKernelGGL((ls_proj_tile_kernel<DT, 8>), tgrid, dim3(256), 0, s, a, lda, gk, M, K, w, o, G);
    return ls_check_launch("ls_proj_tile_kernel");
  }
  switch (F / 16) {
    case 2: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 2>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    case 4: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 4>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    case 6: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 6>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    case 8: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 8>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    case 10: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 10>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    case 12: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 12>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    case 14: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 14>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    case 16: hipLaunchKernelGGL((ls_proj_mfma_kernel<DT, 16>), grid, dim3(256), 0, s, a, lda, gk, M, K, w, o); break;
    default: return ls_fail(LS_ERR_UNSUPPORTED, "projection: router width %d unsupported", F);
  }
  return ls_check_launch("ls_proj_mfma_kernel");
}

// out[g][m][:] = A-rows . wt[g]; K = reduction length; A rows lda apart, group g at g*gk.
int project(int dtype, const void* A, int64_t lda, int64_t gk, int64_t M, int K, int F, int G,
            const void* wt, void* out, hipStream_t s) {
  if (M == 0) return LS_OK;
  if (dtype == LS_F32) {
    const dim3 grid((unsigned)((M * F + 255) / 256), G);
    hipLaunchKernelGGL(ls_proj_f32_kernel, grid, dim3(256), 0, s, (const float*)A, lda, gk, M,
                       K, F, (const float*)wt, (float*)out);
    return ls_check_launch("ls_proj_f32_kernel");
  }
  LS_REQUIRE(ls_aligned16(A) && lda % 8 == 0 && gk % 8 == 0, LS_ERR_UNSUPPORTED,
             "projection: 16-bit inputs must be 16-byte aligned with row strides %% 8 == 0");
  if (dtype == LS_BF16) return launch_proj16<LS_BF16>(A, lda, gk, M, K, F, G, wt, out, s);
  return launch_proj16<LS_F16>(A, lda, gk, M, K, F, G, wt, out, s);
}

template <int DT, int MODE>
int launch_score16(int F, dim3 grid, hipStream_t s, const void* qt, int64_t Nq, const void* kt,
                   int64_t Na, const int32_t* cu_q, const int32_t* cu_a, const int32_t* blk,
                   int batch, int64_t n_launch, int init_blocks, int local_blocks,
                   int64_t full_len, void* out, int64_t out_stride) {
  const uint16_t* qp = (const uint16_t*)qt;
  const uint16_t* kp = (const uint16_t*)kt;
  uint16_t* op = (uint16_t*)out;
  if (F == 128 || F == 256) {
    // Four query blocks per workgroup sharing the k~ panel through LDS.
    const int32_t* sb = MODE != LS_SCORE_FULL ? blk + batch + 1 : nullptr;
    const int64_t n_sb = MODE != LS_SCORE_FULL ? (Nq + 255) / 256 + batch : ((Nq + 63) / 64 + 3) / 4;
    const dim3 pgrid((unsigned)n_sb, grid.y);
    if (F == 128)
      hipLaunchKernelGGL((ls_score_panel_kernel<DT, 4, MODE>), pgrid, dim3(256), 0, s, qp, Nq, kp,
                         Na, cu_q, cu_a, sb, batch, n_sb, init_blocks, local_blocks, full_len, op,
                         out_stride);
    else
      hipLaunchKernelGGL((ls_score_panel_kernel<DT, 8, MODE>), pgrid, dim3(256), 0, s, qp, Nq, kp,
                         Na, cu_q, cu_a, sb, batch, n_sb, init_blocks, local_blocks, full_len, op,
                         out_stride);
    return ls_check_launch("ls_score_panel_kernel");
  }
  switch (F / 32) {
#define LS_SCORE_CASE(KSV)                                                                   \
  case KSV:                                                                                  \
    hipLaunchKernelGGL((ls_score_mfma_kernel<DT, KSV, MODE>), grid, dim3(256), 0, s, qp, Nq, \
                       kp, Na, cu_q, cu_a, blk, batch, n_launch, init_blocks, local_blocks,    \
                       full_len, op, out_stride);                                            \
    break;
    LS_SCORE_CASE(1)
    LS_SCORE_CASE(2)
    LS_SCORE_CASE(3)
    LS_SCORE_CASE(4)
    LS_SCORE_CASE(5)
    LS_SCORE_CASE(6)
    LS_SCORE_CASE(7)
    LS_SCORE_CASE(8)
#undef LS_SCORE_CASE
    default: return ls_fail(LS_ERR_UNSUPPORTED, "score: router width %d unsupported", F);
  }
  return ls_check_launch("ls_score_mfma_kernel");
}

template <int MODE>
int score(int dtype, int F, const void* qt, int64_t Nq, const void* kt, int64_t Na,
          const int32_t* cu_q, const int32_t* cu_a, const int32_t* blk, int batch,
          int64_t n_blk_launch, int init_blocks, int local_blocks, int block_size,
          int kernel_stride, int64_t full_len, int64_t n_page_cols, void* out,
          int64_t out_stride, int G, hipStream_t s) {
  if (Nq == 0) return LS_OK;
  if (dtype == LS_F32) {
    const int64_t n = Nq * n_page_cols;
    const dim3 grid((unsigned)((n + 255) / 256), G);
    hipLaunchKernelGGL(ls_score_f32_kernel<MODE>, grid, dim3(256), 0, s, (const float*)qt, Nq,
                       (const float*)kt, Na, F, cu_q, cu_a, batch, init_blocks, local_blocks,
                       block_size, block_size / kernel_stride, full_len, n_page_cols,
                       (float*)out, out_stride);
    return ls_check_launch("ls_score_f32_kernel");
  }
  LS_REQUIRE(block_size == 64 && kernel_stride == 16, LS_ERR_UNSUPPORTED,
             "score: the 16-bit path supports block_size 64 with kernel_stride 16 "
             "(got %d/%d)", block_size, kernel_stride);
  const dim3 grid(MODE != LS_SCORE_FULL ? (unsigned)n_blk_launch : (unsigned)((Nq + 63) / 64), G);
  if (dtype == LS_BF16)
    return launch_score16<LS_BF16, MODE>(F, grid, s, qt, Nq, kt, Na, cu_q, cu_a, blk, batch,
                                           n_blk_launch, init_blocks, local_blocks, full_len,
                                           out, out_stride);
  return launch_score16<LS_F16, MODE>(F, grid, s, qt, Nq, kt, Na, cu_q, cu_a, blk, batch,
                                        n_blk_launch, init_blocks, local_blocks, full_len, out,
                                        out_stride);
}

// The invalid-key rule of the prefill selection for score dtype dt: canonical
// NaN keys lie above +inf's key, and -inf's key marks -inf.
LsInvalidKeys prefill_rule(int dt) {
  LsInvalidKeys r;
  if (dt == LS_F32) {
    r.hi = ls_order_key32(0x7f800000u);
    r.ninf = ls_order_key32(0xff800000u);
  } else {
    r.hi = ls_order_key16(dt == LS_BF16 ? 0x7f80u : 0x7c00u);
    r.ninf = ls_order_key16(dt == LS_BF16 ? 0xff80u : 0xfc00u);
  }
  return r;
}

template <int KPL, bool KEY32>
void launch_topk_kpl(dim3 grid, hipStream_t s, const void* P, int64_t ps, const int32_t* cu_q,
                     const int32_t* cu_a, int batch, int64_t total_q, int G, int take, int init,
                     int local, int bs, int dt, int32_t* out) {
  hipLaunchKernelGGL((ls_topk_kernel<KPL, KEY32>), grid, dim3(256), 0, s, P, ps, cu_q, cu_a,
                     batch, total_q, G, take, init, local, bs, prefill_rule(dt),
                     dt == LS_BF16 ? 1 : 0, out);
}

template <bool KEY32>
int launch_topk(int max_pages, dim3 grid, hipStream_t s, const void* P, int64_t ps,
                const int32_t* cu_q, const int32_t* cu_a, int batch, int64_t total_q, int G,
                int take, int init, int local, int bs, int dt, int32_t* out) {
#define LS_TOPK_ARGS grid, s, P, ps, cu_q, cu_a, batch, total_q, G, take, init, local, bs, dt, out
  if (max_pages <= 256)
    launch_topk_kpl<4, KEY32>(LS_TOPK_ARGS);
  else if (max_pages <= 1024)
    launch_topk_kpl<16, KEY32>(LS_TOPK_ARGS);
  else if (max_pages <= 2048)
    launch_topk_kpl<32, KEY32>(LS_TOPK_ARGS);
  else if (max_pages <= 4096)
    launch_topk_kpl<64, KEY32>(LS_TOPK_ARGS);
  else if (max_pages <= 8192)
    launch_topk_kpl<128, KEY32>(LS_TOPK_ARGS);
#undef LS_TOPK_ARGS
  else
    return ls_fail(LS_ERR_UNSUPPORTED, "select: at most 8192 pages per sequence (got %d)", max_pages);
  return ls_check_launch("ls_topk_kernel");
}

}  // namespace

// ---------------------------------------------------------------------------
// C ABI
// ---------------------------------------------------------------------------
extern "C" size_t ls_select_workspace_size(int64_t total_q, int64_t total_atoms, int32_t batch,
                                           int32_t num_heads, int32_t num_kv_heads,
                                           int32_t head_dim, int32_t router_heads,
                                           int32_t router_dim, int32_t max_pages,
                                           int32_t dtype) {
  return ws_layout(total_q, total_atoms, batch, num_heads, num_kv_heads, head_dim,
                   router_heads * router_dim, max_pages, (int)ls_dtype_bytes(dtype))
      .total;
}

extern "C" int ls_fused_weights(const float* head_mix, const float* kv_head_mix,
                                const float* q_proj, const float* k_proj, int32_t num_heads,
                                int32_t num_kv_heads, int32_t head_dim, int32_t router_heads,
                                int32_t router_dim, int32_t dtype, void* q_fused,
                                void* kv_fused, void* stream) {
  LS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && head_dim > 0 && router_heads > 0 &&
                 router_dim > 0,
             LS_ERR_INVALID, "ls_fused_weights: bad sizes");
  LS_REQUIRE(dtype == LS_F32 || dtype == LS_BF16 || dtype == LS_F16, LS_ERR_INVALID,
             "ls_fused_weights: unknown dtype %d", dtype);
  LS_REQUIRE(head_mix && kv_head_mix && q_proj && k_proj && q_fused && kv_fused, LS_ERR_INVALID,
             "ls_fused_weights: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int64_t F = (int64_t)router_heads * router_dim;
  const int64_t nq = (int64_t)num_heads * head_dim * F, nk = (int64_t)num_kv_heads * head_dim * F;
#define LS_FUSE(DT, TT)                                                                         \
  hipLaunchKernelGGL(ls_fuse_ref_kernel<DT>, dim3((unsigned)((nq + 255) / 256)), dim3(256), 0, s, \
                     head_mix, q_proj, num_heads, router_heads, head_dim, router_dim, (TT*)q_fused); \
  hipLaunchKernelGGL(ls_fuse_ref_kernel<DT>, dim3((unsigned)((nk + 255) / 256)), dim3(256), 0, s, \
                     kv_head_mix, k_proj, num_kv_heads, router_heads, head_dim, router_dim,        \
                     (TT*)kv_fused);
  if (dtype == LS_BF16) { LS_FUSE(LS_BF16, uint16_t) }
  else if (dtype == LS_F16) { LS_FUSE(LS_F16, uint16_t) }
  else { LS_FUSE(LS_F32, float) }
#undef LS_FUSE
  return ls_check_launch("ls_fuse_ref_kernel");
}

extern "C" int ls_project_queries(const void* query, int64_t q_row_stride, int64_t total_q,
                                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                  const float* head_mix, const float* q_proj,
                                  int32_t router_heads, int32_t router_dim, int32_t dtype,
                                  void* out, void* workspace, size_t workspace_bytes,
                                  void* stream) {
  int rc = check_dims("ls_project_queries", num_heads, num_kv_heads, head_dim, router_heads,
                      router_dim, dtype);
  if (rc) return rc;
  LS_REQUIRE(total_q >= 0 && (total_q == 0 || (query && out)), LS_ERR_INVALID,
             "ls_project_queries: null tensor");
  const int eb = (int)ls_dtype_bytes(dtype);
  const int F = router_heads * router_dim, G = num_kv_heads, gs = num_heads / num_kv_heads;
  const WsLayout L = ws_layout(0, 0, 0, num_heads, G, head_dim, F, 0, eb);
  LS_REQUIRE(workspace && workspace_bytes >= L.total, LS_ERR_WORKSPACE,
             "ls_project_queries: workspace needs %zu bytes", L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  rc = fuse_t(dtype, head_mix, q_proj, G, gs, router_heads, head_dim, router_dim, ws + L.wq, s);
  if (rc) return rc;
  return project(dtype, query, q_row_stride, (int64_t)gs * head_dim, total_q, gs * head_dim, F,
                 G, ws + L.wq, out, s);
}

extern "C" int ls_rope_project_queries(void* query, int64_t q_row_stride,
                                       const int32_t* positions, int64_t total_q,
                                       int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                       const float* cos_table, const float* sin_table,
                                       int64_t table_rows, const float* head_mix,
                                       const float* q_proj, int32_t router_heads,
                                       int32_t router_dim, int32_t dtype, void* out,
                                       void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_dims("ls_rope_project_queries", num_heads, num_kv_heads, head_dim, router_heads,
                      router_dim, dtype);
  if (rc) return rc;
  const int F = router_heads * router_dim, G = num_kv_heads, gs = num_heads / num_kv_heads;
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "ls_rope_project_queries: bf16 or fp16 queries");
  LS_REQUIRE(head_dim == 128 && (F == 64 || F == 128), LS_ERR_UNSUPPORTED,
             "ls_rope_project_queries: head_dim 128 and router width 64 or 128 (got %d, %d)",
             head_dim, F);
  LS_REQUIRE(total_q >= 0 && table_rows > 0 && q_row_stride % 8 == 0 &&
                 q_row_stride >= (int64_t)num_heads * head_dim,
             LS_ERR_INVALID, "ls_rope_project_queries: bad sizes or row stride");
  if (total_q == 0) return LS_OK;
  LS_REQUIRE(query && positions && cos_table && sin_table && out, LS_ERR_INVALID,
             "ls_rope_project_queries: null tensor");
  LS_REQUIRE(ls_aligned16(query) && ls_aligned16(cos_table) && ls_aligned16(sin_table),
             LS_ERR_UNSUPPORTED, "ls_rope_project_queries: tensors must be 16-byte aligned");
  const int eb = (int)ls_dtype_bytes(dtype);
  const WsLayout L = ws_layout(0, 0, 0, num_heads, G, head_dim, F, 0, eb);
  LS_REQUIRE(workspace && workspace_bytes >= L.total, LS_ERR_WORKSPACE,
             "ls_rope_project_queries: workspace needs %zu bytes", L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  rc = fuse_t(dtype, head_mix, q_proj, G, gs, router_heads, head_dim, router_dim, ws + L.wq, s);
  if (rc) return rc;
  const dim3 grid((unsigned)((total_q + 16 * LS_RP_WAVES - 1) / (16 * LS_RP_WAVES)), G);
  const dim3 block(64 * LS_RP_WAVES);
  uint16_t* x = (uint16_t*)query;
  const uint16_t* w = (const uint16_t*)(ws + L.wq);
  uint16_t* o = (uint16_t*)out;
  if (dtype == LS_BF16) {
    if (F == 64)
      hipLaunchKernelGGL((ls_rope_proj_kernel<LS_BF16, 4>), grid, block, 0, s, x, q_row_stride,
                         gs, total_q, positions, cos_table, sin_table, table_rows, w, o);
    else
      hipLaunchKernelGGL((ls_rope_proj_kernel<LS_BF16, 8>), grid, block, 0, s, x, q_row_stride,
                         gs, total_q, positions, cos_table, sin_table, table_rows, w, o);
  } else {
    if (F == 64)
      hipLaunchKernelGGL((ls_rope_proj_kernel<LS_F16, 4>), grid, block, 0, s, x, q_row_stride,
                         gs, total_q, positions, cos_table, sin_table, table_rows, w, o);
    else
      hipLaunchKernelGGL((ls_rope_proj_kernel<LS_F16, 8>), grid, block, 0, s, x, q_row_stride,
                         gs, total_q, positions, cos_table, sin_table, table_rows, w, o);
  }
  return ls_check_launch("ls_rope_proj_kernel");
}

extern "C" int ls_project_atom_keys(const void* kc, int64_t kc_row_stride, int64_t n_atoms,
                                    int32_t num_kv_heads, int32_t head_dim,
                                    const float* kv_head_mix, const float* k_proj,
                                    int32_t router_heads, int32_t router_dim, int32_t dtype,
                                    void* out, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  int rc = check_dims("ls_project_atom_keys", num_kv_heads, num_kv_heads, head_dim,
                      router_heads > num_kv_heads ? 1 : router_heads, router_dim, dtype);
  if (rc) return rc;
  LS_REQUIRE(router_heads > 0, LS_ERR_INVALID, "ls_project_atom_keys: bad router_heads");
  LS_REQUIRE(n_atoms >= 0 && (n_atoms == 0 || (kc && out)), LS_ERR_INVALID,
             "ls_project_atom_keys: null tensor");
  const int eb = (int)ls_dtype_bytes(dtype);
  const int F = router_heads * router_dim, G = num_kv_heads;
  LS_REQUIRE(dtype == LS_F32 || (F % 32 == 0 && F <= 256), LS_ERR_UNSUPPORTED,
             "ls_project_atom_keys: router width %d unsupported on the 16-bit path", F);
  const WsLayout L = ws_layout(0, 0, 0, G, G, head_dim, F, 0, eb);
  LS_REQUIRE(workspace && workspace_bytes >= L.total, LS_ERR_WORKSPACE,
             "ls_project_atom_keys: workspace needs %zu bytes", L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  rc = fuse_t(dtype, kv_head_mix, k_proj, G, 1, router_heads, head_dim, router_dim, ws + L.wk, s);
  if (rc) return rc;
  return project(dtype, kc, kc_row_stride, head_dim, n_atoms, head_dim, F, G, ws + L.wk, out, s);
}

extern "C" int ls_score_pages(const void* query, int64_t q_row_stride, int64_t n_queries,
                              const void* kc, int64_t kc_row_stride, int64_t n_atoms,
                              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                              const float* head_mix, const float* kv_head_mix,
                              const float* q_proj, const float* k_proj, int32_t router_heads,
                              int32_t router_dim, int32_t dtype, int64_t seq_len,
                              int32_t block_size, int32_t kernel_stride, void* out,
                              void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_dims("ls_score_pages", num_heads, num_kv_heads, head_dim, router_heads,
                      router_dim, dtype);
  if (rc) return rc;
  LS_REQUIRE(seq_len > 0 && block_size > 0 && kernel_stride > 0, LS_ERR_INVALID,
             "ls_score_pages: page geometry must be positive");
  LS_REQUIRE(block_size % kernel_stride == 0, LS_ERR_INVALID,
             "ls_score_pages: block_size must be divisible by kernel_stride");
  LS_REQUIRE(n_atoms > 0, LS_ERR_INVALID, "ls_score_pages: need at least one atom");
  const int eb = (int)ls_dtype_bytes(dtype);
  const int F = router_heads * router_dim, G = num_kv_heads, gs = num_heads / num_kv_heads;
  const WsLayout L = ws_layout(n_queries, n_atoms, 0, num_heads, G, head_dim, F, 0, eb);
  LS_REQUIRE(workspace && workspace_bytes >= L.total, LS_ERR_WORKSPACE,
             "ls_score_pages: workspace needs %zu bytes", L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  if ((rc = fuse_t(dtype, head_mix, q_proj, G, gs, router_heads, head_dim, router_dim,
                   ws + L.wq, s)))
    return rc;
  if ((rc = fuse_t(dtype, kv_head_mix, k_proj, G, 1, router_heads, head_dim, router_dim,
                   ws + L.wk, s)))
    return rc;
  if ((rc = project(dtype, query, q_row_stride, (int64_t)gs * head_dim, n_queries,
                    gs * head_dim, F, G, ws + L.wq, ws + L.qt, s)))
    return rc;
  if ((rc = project(dtype, kc, kc_row_stride, head_dim, n_atoms, head_dim, F, G, ws + L.wk,
                    ws + L.kt, s)))
    return rc;
  const int64_t n_pages = (seq_len + block_size - 1) / block_size;
  return score<LS_SCORE_FULL>(dtype, F, ws + L.qt, n_queries, ws + L.kt, n_atoms, nullptr, nullptr,
                      nullptr, 0, 0, 0, 0, block_size, kernel_stride, seq_len, n_pages, out,
                      n_pages, G, s);
}

static int select_prefill_impl(const char* who, const void* q, int64_t q_row_stride,
                               const void* q_tilde, int64_t total_q,
                                 const void* kc, int64_t kc_row_stride, int64_t total_atoms,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kc,
                                 int32_t batch, int32_t max_seqlen_q, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, const float* head_mix,
                                 const float* kv_head_mix, const float* q_proj,
                                 const float* k_proj, int32_t router_heads, int32_t router_dim,
                                 int32_t dtype, int32_t topk, int32_t block_size,
                                 int32_t kernel_stride, int32_t init_blocks,
                                 int32_t local_blocks, int32_t* topk_idx, int32_t take,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  int rc = check_dims(who, num_heads, num_kv_heads, head_dim, router_heads,
                      router_dim, dtype);
  if (rc) return rc;
  LS_REQUIRE(batch >= 0 && total_q >= 0 && total_atoms >= 0 && max_seqlen_q >= 0, LS_ERR_INVALID,
             "%s: bad sizes", who);
  LS_REQUIRE(block_size > 0 && kernel_stride > 0 && block_size % kernel_stride == 0,
             LS_ERR_INVALID, "%s: bad page geometry", who);
  LS_REQUIRE(init_blocks >= 0 && local_blocks >= 0 && topk >= 0, LS_ERR_INVALID,
             "%s: init_blocks, local_blocks and topk must be >= 0", who);
  const int max_pages = (max_seqlen_q + block_size - 1) / block_size;
  LS_REQUIRE(take == (topk < max_pages ? topk : max_pages), LS_ERR_INVALID,
             "%s: take must be min(topk, ceil(max_seqlen_q / block_size)) = %d", who,
             topk < max_pages ? topk : max_pages);
  if (total_q == 0 || batch == 0 || take == 0) return LS_OK;
  // kc may be null only when there is no compressed key at all (every sequence
  // shorter than one window: its rows get no pages, as the reference skips it).
  LS_REQUIRE((q || q_tilde) && (kc || total_atoms == 0) && cu_seqlens_q && cu_seqlens_kc &&
                 topk_idx,
             LS_ERR_INVALID, "%s: null pointer", who);
  const int eb = (int)ls_dtype_bytes(dtype);
  const int F = router_heads * router_dim, G = num_kv_heads, gs = num_heads / num_kv_heads;
  const WsLayout L = ws_layout(total_q, total_atoms, batch, num_heads, G, head_dim, F,
                               max_pages, eb);
  LS_REQUIRE(workspace && workspace_bytes >= L.total, LS_ERR_WORKSPACE,
             "%s: workspace needs %zu bytes", who, L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int32_t* blk = (int32_t*)(ws + L.blk);
  // q~ is either given (projected where the queries were produced) or formed here.
  if (!q_tilde && (rc = fuse_t(dtype, head_mix, q_proj, G, gs, router_heads, head_dim,
                               router_dim, ws + L.wq, s)))
    return rc;
  if ((rc = fuse_t(dtype, kv_head_mix, k_proj, G, 1, router_heads, head_dim, router_dim,
                   ws + L.wk, s)))
    return rc;
  const void* qt = q_tilde ? q_tilde : (const void*)(ws + L.qt);
  if (!q_tilde &&
      (rc = project(dtype, q, q_row_stride, (int64_t)gs * head_dim, total_q, gs * head_dim, F,
                    G, ws + L.wq, ws + L.qt, s)))
    return rc;
  if (total_atoms > 0 &&
      (rc = project(dtype, kc, kc_row_stride, head_dim, total_atoms, head_dim, F, G, ws + L.wk,
                    ws + L.kt, s)))
    return rc;
  hipLaunchKernelGGL(ls_select_plan_kernel, dim3(1), dim3(64), 0, s, cu_seqlens_q, batch,
                     block_size, blk);
  if ((rc = ls_check_launch("ls_select_plan_kernel"))) return rc;
  const int64_t n_blk_launch = (total_q + block_size - 1) / block_size + batch;
  if (total_atoms > 0 &&
      (rc = score<LS_SCORE_SELECT>(dtype, F, qt, total_q, ws + L.kt, total_atoms, cu_seqlens_q,
                        cu_seqlens_kc, blk, batch, n_blk_launch, init_blocks, local_blocks,
                        block_size, kernel_stride, 0, max_pages, ws + L.p, L.p_stride, G, s)))
    return rc;
  const dim3 grid((unsigned)((total_q + 3) / 4), G);
  if (dtype == LS_F32)
    return launch_topk<true>(max_pages, grid, s, ws + L.p, L.p_stride, cu_seqlens_q,
                             cu_seqlens_kc, batch, total_q, G, take, init_blocks, local_blocks,
                             block_size, dtype, topk_idx);
  return launch_topk<false>(max_pages, grid, s, ws + L.p, L.p_stride, cu_seqlens_q,
                            cu_seqlens_kc, batch, total_q, G, take, init_blocks, local_blocks,
                            block_size, dtype, topk_idx);
}

extern "C" int ls_select_prefill(const void* q, int64_t q_row_stride, int64_t total_q,
                                 const void* kc, int64_t kc_row_stride, int64_t total_atoms,
                                 const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kc,
                                 int32_t batch, int32_t max_seqlen_q, int32_t num_heads,
                                 int32_t num_kv_heads, int32_t head_dim, const float* head_mix,
                                 const float* kv_head_mix, const float* q_proj,
                                 const float* k_proj, int32_t router_heads, int32_t router_dim,
                                 int32_t dtype, int32_t topk, int32_t block_size,
                                 int32_t kernel_stride, int32_t init_blocks,
                                 int32_t local_blocks, int32_t* topk_idx, int32_t take,
                                 void* workspace, size_t workspace_bytes, void* stream) {
  return select_prefill_impl("ls_select_prefill", q, q_row_stride, nullptr, total_q, kc,
                             kc_row_stride, total_atoms, cu_seqlens_q, cu_seqlens_kc, batch,
                             max_seqlen_q, num_heads, num_kv_heads, head_dim, head_mix,
                             kv_head_mix, q_proj, k_proj, router_heads, router_dim, dtype, topk,
                             block_size, kernel_stride, init_blocks, local_blocks, topk_idx, take,
                             workspace, workspace_bytes, stream);
}

extern "C" int ls_select_prefill_qt(const void* q_tilde, int64_t total_q, const void* kc,
                                    int64_t kc_row_stride, int64_t total_atoms,
                                    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kc,
                                    int32_t batch, int32_t max_seqlen_q, int32_t num_heads,
                                    int32_t num_kv_heads, int32_t head_dim,
                                    const float* kv_head_mix, const float* k_proj,
                                    int32_t router_heads, int32_t router_dim, int32_t dtype,
                                    int32_t topk, int32_t block_size, int32_t kernel_stride,
                                    int32_t init_blocks, int32_t local_blocks, int32_t* topk_idx,
                                    int32_t take, void* workspace, size_t workspace_bytes,
                                    void* stream) {
  return select_prefill_impl("ls_select_prefill_qt", nullptr, 0, q_tilde, total_q, kc,
                             kc_row_stride, total_atoms, cu_seqlens_q, cu_seqlens_kc, batch,
                             max_seqlen_q, num_heads, num_kv_heads, head_dim, nullptr,
                             kv_head_mix, nullptr, k_proj, router_heads, router_dim, dtype, topk,
                             block_size, kernel_stride, init_blocks, local_blocks, topk_idx, take,
                             workspace, workspace_bytes, stream);
}

extern "C" size_t ls_nosa_select_workspace_size(int64_t total_q, int64_t total_atoms,
                                                int32_t batch, int32_t num_heads,
                                                int32_t num_kv_heads, int32_t head_dim,
                                                int32_t router_heads, int32_t router_dim,
                                                int32_t max_pages, int32_t dtype) {
  return nosa_ws_layout(total_q, total_atoms, batch, num_heads, num_kv_heads, head_dim,
                        router_heads * router_dim, max_pages, (int)ls_dtype_bytes(dtype))
      .total;
}

// NOSA page plans (prefill): qk page scores of every page with atoms, the
// qk shortlist, CIS page scores and the CIS top-k with the reference's masks
// (leanselect/models/nosa.py:1144-1307 on the LeanSelect branch, whose atom
// scores come from the folded router, nosa.py:1822-1853).
extern "C" int ls_nosa_select_prefill(
    const void* q, int64_t q_row_stride, int64_t total_q, const void* kc, int64_t kc_row_stride,
    int64_t total_atoms, const void* cis, int64_t cis_row_stride, int32_t cis_dtype,
    const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_kc, const int32_t* cu_seqlens_k,
    int32_t batch, int32_t max_seqlen_q, int32_t num_heads, int32_t num_kv_heads,
    int32_t head_dim, const float* head_mix, const float* kv_head_mix, const float* q_proj,
    const float* k_proj, int32_t router_heads, int32_t router_dim, int32_t dtype, int32_t topk,
    int32_t block_size, int32_t kernel_stride, int32_t init_blocks, int32_t local_blocks,
    int32_t select_blocks, int32_t pool_clip, int32_t* topk_idx, int32_t take, void* workspace,
    size_t workspace_bytes, void* stream) {
  int rc = check_dims("ls_nosa_select_prefill", num_heads, num_kv_heads, head_dim, router_heads,
                      router_dim, dtype);
  if (rc) return rc;
  LS_REQUIRE(batch >= 0 && total_q >= 0 && total_atoms >= 0 && max_seqlen_q >= 0, LS_ERR_INVALID,
             "ls_nosa_select_prefill: bad sizes");
  LS_REQUIRE(block_size == 64 && kernel_stride == 16, LS_ERR_UNSUPPORTED,
             "ls_nosa_select_prefill: block_size 64 with kernel_stride 16 only (got %d/%d)",
             block_size, kernel_stride);
  LS_REQUIRE(cis_dtype == LS_F32 || cis_dtype == LS_BF16 || cis_dtype == LS_F16, LS_ERR_INVALID,
             "ls_nosa_select_prefill: unknown CIS dtype %d", cis_dtype);
  LS_REQUIRE(init_blocks >= 0 && local_blocks >= 0 && select_blocks >= 0 && topk >= 0,
             LS_ERR_INVALID, "ls_nosa_select_prefill: block counts and topk must be >= 0");
  LS_REQUIRE(pool_clip == LS_POOL_CLIP_SEQUENCE || pool_clip == LS_POOL_CLIP_ROW, LS_ERR_INVALID,
             "ls_nosa_select_prefill: unknown pool_clip %d", pool_clip);
  const int out_len = (max_seqlen_q + block_size - 1) / block_size;
  const int want = topk < out_len ? topk : out_len;
  LS_REQUIRE(take == want, LS_ERR_INVALID,
             "ls_nosa_select_prefill: take must be min(topk, ceil(max_seqlen_q / 64)) = %d", want);
  if (total_q == 0 || batch == 0 || take == 0) return LS_OK;
  LS_REQUIRE(q && (kc || total_atoms == 0) && cis && cu_seqlens_q && cu_seqlens_kc &&
                 cu_seqlens_k && topk_idx,
             LS_ERR_INVALID, "ls_nosa_select_prefill: null pointer");
  const int qk_sel_raw = init_blocks + local_blocks + select_blocks;
  const int qk_select = qk_sel_raw < out_len ? qk_sel_raw : out_len;
  const int eb = (int)ls_dtype_bytes(dtype);
  const int F = router_heads * router_dim, G = num_kv_heads, gs = num_heads / num_kv_heads;
  const NosaWsLayout N = nosa_ws_layout(total_q, total_atoms, batch, num_heads, G, head_dim, F,
                                        out_len, eb);
  const WsLayout& L = N.L;
  LS_REQUIRE(workspace && workspace_bytes >= N.total, LS_ERR_WORKSPACE,
             "ls_nosa_select_prefill: workspace needs %zu bytes", N.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  int32_t* blk = (int32_t*)(ws + L.blk);
  if ((rc = fuse_t(dtype, head_mix, q_proj, G, gs, router_heads, head_dim, router_dim,
                   ws + L.wq, s)))
    return rc;
  if ((rc = fuse_t(dtype, kv_head_mix, k_proj, G, 1, router_heads, head_dim, router_dim,
                   ws + L.wk, s)))
    return rc;
  if ((rc = project(dtype, q, q_row_stride, (int64_t)gs * head_dim, total_q, gs * head_dim, F,
                    G, ws + L.wq, ws + L.qt, s)))
    return rc;
  if (total_atoms > 0 &&
      (rc = project(dtype, kc, kc_row_stride, head_dim, total_atoms, head_dim, F, G, ws + L.wk,
                    ws + L.kt, s)))
    return rc;
  hipLaunchKernelGGL(ls_select_plan_kernel, dim3(1), dim3(64), 0, s, cu_seqlens_q, batch,
                     block_size, blk);
  if ((rc = ls_check_launch("ls_select_plan_kernel"))) return rc;
  const int64_t n_blk_launch = (total_q + block_size - 1) / block_size + batch;
  if (total_atoms > 0 &&
      (rc = score<LS_SCORE_ALL>(dtype, F, ws + L.qt, total_q, ws + L.kt, total_atoms,
                                cu_seqlens_q, cu_seqlens_kc, blk, batch, n_blk_launch,
                                init_blocks, local_blocks, block_size, kernel_stride, out_len,
                                out_len, ws + L.p, L.p_stride, G, s)))
    return rc;
  int32_t* pg_off = (int32_t*)(ws + N.pg);
  float* cpg = (float*)(ws + N.cpg);
  if ((rc = ls_nosa_cis_pages_launch(cis, cis_row_stride, cis_dtype, cu_seqlens_k, cu_seqlens_kc,
                                     batch, total_atoms, G, pool_clip, pg_off, cpg,
                                     N.cpg_stride, s)))
    return rc;
  return ls_nosa_topk_launch(dtype, out_len, ws + L.p, L.p_stride, cpg, N.cpg_stride, pg_off,
                             cu_seqlens_q, cu_seqlens_kc, blk, N.n_blk, batch, total_q, G,
                             max_seqlen_q, init_blocks, local_blocks, qk_select, take, block_size,
                             pool_clip, (int32_t*)(ws + N.order), topk_idx, s);
}
