// Launchers shared between the NOSA kernels (ls_nosa.hip) and the fused NOSA
// selection entry point (ls_select.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

// CIS page scores of every sequence: pg_off[b] (batch + 1 entries) and
// cpg[g * cpg_g_stride + pg_off[b] + p] for p <= A_b / 4.
int ls_nosa_cis_pages_launch(const void* cis, int64_t cis_rs, int cis_dtype, const int32_t* cu_k,
                             const int32_t* cu_a, int batch, int64_t total_atoms, int G,
                             int32_t* pg_off, float* cpg, int64_t cpg_g_stride, hipStream_t s);

// Two-stage NOSA top-k over the page-score scratch P ([G][total_q][p_stride]
// of p_dtype, LS_F32 / LS_BF16 / LS_F16) and the CIS page scores (float32
// holding values of cis_dtype).
int ls_nosa_topk_launch(int p_dtype, int cis_dtype, int out_len, const void* P, int64_t p_stride, const float* cpg,
                        int64_t cpg_g_stride, const int32_t* pg_off, const int32_t* cu_q,
                        const int32_t* cu_a, int batch, int64_t total_q, int G, int max_seqlen_q,
                        int init_blocks, int local_blocks, int qk_select, int take,
                        int block_size, int32_t* topk_idx, hipStream_t s);
