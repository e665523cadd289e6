// Launchers shared between the NOSA kernels (ls_nosa.hip) and the fused NOSA
// selection entry point (ls_select.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

// CIS page scores of every sequence: pg_off[b] (batch + 1 entries, then the
// largest atom count A_max in pg_off[batch + 1]) and cpg[g * cpg_g_stride +
// pg_off[b] + p] for p <= A_b / 4.  clip_row selects LS_POOL_CLIP_ROW.
int ls_nosa_cis_pages_launch(const void* cis, int64_t cis_rs, int cis_dtype, const int32_t* cu_k,
                             const int32_t* cu_a, int batch, int64_t total_atoms, int G,
                             int clip_row, int32_t* pg_off, float* cpg, int64_t cpg_g_stride,
                             hipStream_t s);

// Two-stage NOSA top-k over the page-score scratch P ([G][total_q][p_stride]
// of p_dtype, LS_F32 / LS_BF16 / LS_F16) and the CIS page scores (float32).
// blk_off (batch + 1) holds the 64-row query blocks before each sequence and
// n_blk bounds their total; `order` is scratch of ls_nosa_order_bytes(n_blk,
// G, LS_NOSA_ORDER_STRIDE) bytes for the blocks' stage-2 orders.
#define LS_NOSA_ORDER_STRIDE 320
size_t ls_nosa_order_bytes(int64_t n_blk, int G, int n_order);
int ls_nosa_topk_launch(int p_dtype, int out_len, const void* P, int64_t p_stride, const float* cpg,
                        int64_t cpg_g_stride, const int32_t* pg_off, const int32_t* cu_q,
                        const int32_t* cu_a, const int32_t* blk_off, int64_t n_blk, int batch,
                        int64_t total_q, int G, int max_seqlen_q, int init_blocks,
                        int local_blocks, int qk_select, int take, int block_size,
                        int clip_row, int32_t* order, int32_t* topk_idx, hipStream_t s);
