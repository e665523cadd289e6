// Block-sparse causal attention over per-token page plans.
//
// Contract: infllmv2_attn_varlen_func(..., topk_idx=)
// (third_party/infllmv2/paper1.patch:1993-2100; called from
// leanselect/models/minicpm.py:3216-3244): for query row t and KV group g the
// keys are those of the valid ids in topk_idx[g, t, :] (each page once) with
// j <= t + len_k - len_q when causal; all H/G heads of the group share the plan.
//
// Design (one workgroup per 24 query rows of one KV group and 16-head tile):
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

#include <mutex>

// Work-item and workgroup ids straight from the hardware: this file is built
// without IEEE NaN quieting, and the device library's id helpers (built with
// it) would then stay out-of-line calls.
#define LS_TID ((int)__builtin_amdgcn_workitem_id_x())
#define LS_BID_X ((int)__builtin_amdgcn_workgroup_id_x())
#define LS_BID_Y ((int)__builtin_amdgcn_workgroup_id_y())
#define LS_BID_Z ((int)__builtin_amdgcn_workgroup_id_z())

#define LS_ATTN_MAX_PAGES 8192
#define LS_ATTN_MAX_TAKE 128
#define LS_ATTN_RING_TIMEOUT 1  // status bit: a ring wait expired (outputs invalid)

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
// sequence in the transposed V copy (in pages); tile_off[b] = sum_{b' < b}
// ceil(len_q(b') / tile): first row tile of each sequence; tok[i] = i for
// i < n_tok (the ready tokens the tile kernel's copies deliver); *status = 0
// (the tile kernel ORs in LS_ATTN_RING_TIMEOUT when a ring wait expires).
__global__ void ls_attn_plan_kernel(const int32_t* __restrict__ cu_q,
                                    const int32_t* __restrict__ cu_k, int batch, int tile,
                                    int32_t* __restrict__ pg_off, int32_t* __restrict__ tile_off,
                                    int32_t* __restrict__ tok, int n_tok,
                                    int32_t* __restrict__ status) {
  if (LS_BID_X != 0) return;
  for (int i = LS_TID; i < n_tok; i += 64) tok[i] = i;
  if (LS_TID != 0) return;
  *status = 0;
  int32_t acc = 0, acc_t = 0;
  pg_off[0] = 0;
  tile_off[0] = 0;
  for (int b = 0; b < batch; ++b) {
    const int len = cu_k[b + 1] - cu_k[b];
    acc += len > 0 ? (len + 63) / 64 : 0;
    pg_off[b + 1] = acc;
    const int lq = cu_q[b + 1] - cu_q[b];
    acc_t += lq > 0 ? (lq + tile - 1) / tile : 0;
    tile_off[b + 1] = acc_t;
  }
}

// Writes 0 to a caller's status word (a kernel rather than a memset, so that
// the call stays safe to capture in a graph).
__global__ void ls_attn_status_clear_kernel(int32_t* __restrict__ status) {
  if (LS_BID_X == 0 && LS_TID == 0) *status = 0;
}

// ---------------------------------------------------------------------------
// Tile kernel: one workgroup = 8 x TPW consecutive query rows of one sequence
// and one KV group for 16 of its query heads (8 waves x TPW rows, two waves per
// SIMD; the launcher uses TPW = 3, 24-row tiles, for every plan of up to
// LS_ATTN_MAX_TAKE ids).  The rows' page plans are OR-ed into a union page list;
// each union page of staged K and V^T is streamed once into a 4-stage LDS ring
// with direct global->LDS loads, and every row that selected the page runs its
// MFMAs on it.  Rows that did not select a page skip it (no masked-out work).
// A wave keeps its rows' O^T accumulators (TPW x 8 x 4 floats per lane) and
// Q^T fragments in registers.  Larger tiles share each page copy among more
// rows; three rows of O and Q are what the register file holds at two waves per
// SIMD (with each row reading the chunk's V^T fragments where it uses them).
// ---------------------------------------------------------------------------
#ifndef LS_ATT_WAVES
#define LS_ATT_WAVES 8                       // waves per workgroup
#endif
#define LS_ATT_THREADS (64 * LS_ATT_WAVES)
#define LS_ATT_STAGES 4
#define LS_ATT_KBYTES (64 * 256)             // K page: 64 rows x 256 B
#define LS_ATT_STAGE_BYTES (2 * LS_ATT_KBYTES)  // + V^T page: 128 rows x 128 B
#define LS_ATT_WORDS (LS_ATTN_MAX_PAGES / 32)
#ifndef LS_ATT_XCD_CHUNK
#define LS_ATT_XCD_CHUNK 16                  // consecutive tiles per XCD run
#endif
#ifndef LS_ATT_SHARE_STRIDED
#define LS_ATT_SHARE_STRIDED 25              // plan ids per union page (x10) for the strided order
#endif
#ifndef LS_ATT_SPIN_SLEEP
#define LS_ATT_SPIN_SLEEP 1                  // s_sleep units between a waiting wave's polls
#endif
#define LS_ATT_UNION_CAP (64 * 64)           // union pages of a tile: one 64-bit need word per lane

// Tile geometry for TPW rows per wave: rows per tile, the most ids per row it
// accepts (so that its union fits LS_ATT_UNION_CAP) and the union bound.
template <int TPW>
struct LsAttTile {
  static constexpr int kTile = LS_ATT_WAVES * TPW;
  static constexpr int kMaxTake =
      LS_ATTN_MAX_TAKE < LS_ATT_UNION_CAP / kTile ? LS_ATTN_MAX_TAKE : LS_ATT_UNION_CAP / kTile;
  static constexpr int kMaxUnion = kTile * kMaxTake;
  static_assert(kTile <= 32, "row masks are 32-bit");
  static_assert(kMaxUnion <= LS_ATT_UNION_CAP, "one need word per lane");
};

typedef _Float16 ls_half2 __attribute__((ext_vector_type(2)));
typedef float ls_float2 __attribute__((ext_vector_type(2)));

// LDS row of key j (0..63) of a page: inside each 32-key chunk, MFMA row r of
// key block nb holds key 8*(r/4) + 4*nb + r%4, so storing that key at row
// 16*nb + r makes the 16 rows an MFMA reads consecutive, while lane group q
// still ends up with the keys 8q..8q+7 of the chunk.
__device__ __forceinline__ int ls_att_key_of_row(int row) {
  const int c = row >> 5, rr = row & 31, nb = rr >> 4, r = rr & 15;
  return 32 * c + 8 * (r >> 2) + 4 * nb + (r & 3);
}

// Page-major staging of K and V in the ring's own byte order: block
// kv[g][pg_off[b] + p] (LS_ATT_STAGE_BYTES) holds page p of sequence b, group
// g, exactly as a ring stage holds it, so a page copy is one contiguous
// 32 KB transfer:
//  - bytes [0, 16K): K, 64 rows of 256 B; row R holds key ls_att_key_of_row(R)
//    of the page, its 16-byte chunk C (dims 8C..8C+7) at position C ^ (R & 15);
//  - bytes [16K, 32K): V^T, 128 rows of 128 B; row d holds fp16(v[key][d] * 2^-e)
//    of the page's 64 keys, chunk C (keys 8C..8C+7) at position C ^ ((d >> 1) & 7).
// Keys past the sequence end are zero (their scores are always masked).
// vexp[g * n_pages + pg_off[b] + p] = e: the smallest e >= 0 (at most 15) that
// keeps the page's scaled V within +-32768, so it is finite in fp16 (e = 0 for
// ordinary activations; bf16 values are then exact in fp16 down to 2^-14).
// One workgroup stages one page of one group (V^T goes through LDS).
template <int DT>
__global__ __launch_bounds__(256) void ls_kv_stage_kernel(
    const uint16_t* __restrict__ k, int64_t k_rs, const uint16_t* __restrict__ v, int64_t v_rs,
    const int32_t* __restrict__ cu_k, const int32_t* __restrict__ pg_off, int batch,
    int64_t n_pages, uint8_t* __restrict__ kv, int32_t* __restrict__ vexp) {
  constexpr int D = 128, PITCH = D + 2, CH = D / 8;
  __shared__ uint16_t tile[64 * PITCH];
  __shared__ float wave_max[4];
  const int64_t tile_id = LS_BID_X;
  if (tile_id >= pg_off[batch]) return;
  const int g = LS_BID_Y;
  const int b = ls_find_segment(pg_off, batch, tile_id);
  const int p = (int)(tile_id - pg_off[b]);
  const int lk = cu_k[b + 1] - cu_k[b];
  const int64_t krow0 = (int64_t)cu_k[b] + 64LL * p;
  uint8_t* blk = kv + ((int64_t)g * n_pages + pg_off[b] + p) * LS_ATT_STAGE_BYTES;
  // K: output chunk o = 16 R + position.
  for (int o = LS_TID; o < 64 * CH; o += 256) {
    const int R = o >> 4, C = (o & 15) ^ (R & 15);
    const int key = ls_att_key_of_row(R);
    ls_u32x4 val = {0u, 0u, 0u, 0u};
    if (64 * p + key < lk) val = ls_load16(k + (krow0 + key) * k_rs + (int64_t)g * D + 8 * C);
    *reinterpret_cast<ls_u32x4*>(blk + 16 * o) = val;
  }
  // V through LDS, then V^T rows.
  float mx = 0.f;
  for (int c = LS_TID; c < 64 * CH; c += 256) {
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
  if ((LS_TID & 63) == 0) wave_max[LS_TID >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
  int e = 0;
  while (e < 15 && mx * __builtin_ldexpf(1.f, -e) > 32768.f) ++e;
  const float scale = __builtin_ldexpf(1.f, -e);
  if (LS_TID == 0) vexp[(int64_t)g * n_pages + pg_off[b] + p] = e;
  uint8_t* vblk = blk + LS_ATT_KBYTES;
  for (int c = LS_TID; c < D * 8; c += 256) {
    const int d = c / 8, k0 = (c % 8) * 8;
    ls_u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      o[i] = ls_pack2(ls_f32_to_f16(LsElem<DT>::to_f(tile[(k0 + 2 * i) * PITCH + d]) * scale),
                      ls_f32_to_f16(LsElem<DT>::to_f(tile[(k0 + 2 * i + 1) * PITCH + d]) * scale));
    *reinterpret_cast<ls_u32x4*>(vblk + d * 128 + 16 * ((c % 8) ^ ((d >> 1) & 7))) = o;
  }
}




// Two float32 -> one packed fp16 pair (round to nearest even).
__device__ __forceinline__ uint32_t ls_pack_f16x2(float a, float b) {
  const ls_half2 h = __builtin_convertvector((ls_float2){a, b}, ls_half2);
  return __builtin_bit_cast(uint32_t, h);
}

// acc + lo(x) + hi(x) for a packed fp16 pair, in float32.
__device__ __forceinline__ float ls_sum_f16x2(uint32_t x, float acc) {
  const ls_half2 one = {(_Float16)1.0f, (_Float16)1.0f};
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(ls_half2, x), one, acc, false);
}


// BIAS adds a per-key score bias (the NOSA eviction score, pre-scaled to base
// 2): weight_j = 2^(scale_log2 * q.k_j + cb_j).  cb[g][64 pg_off[b] + j] is
// staged like V^T and copied with each page (256 B per stage).
template <int DT, bool BIAS, int TPW>
__global__ __launch_bounds__(LS_ATT_THREADS, LS_ATT_THREADS / 256) void ls_attn_tile_kernel(
    const uint16_t* __restrict__ qg, int64_t q_rs, const uint8_t* __restrict__ kv, int64_t lpad,
    const int32_t* __restrict__ vexp, const float* __restrict__ cb,
    const int32_t* __restrict__ tok, int64_t n_pages_ws,
    const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
    const int32_t* __restrict__ pg_off, const int32_t* __restrict__ tile_off, int batch,
    int64_t total_q, int G, int gs, const int32_t* __restrict__ topk_idx, int take,
    float scale_log2, int causal, uint16_t* __restrict__ out, float* __restrict__ lse,
    int per_xcd, int32_t* __restrict__ status, int spin_limit) {
  constexpr int D = 128;
  constexpr int TILE = LsAttTile<TPW>::kTile;
  constexpr int MAX_UNION = LsAttTile<TPW>::kMaxUnion;
  constexpr int NEED_LANES = (MAX_UNION + 63) / 64;  // lanes holding a 64-bit need word
  constexpr int NEED_WORDS = 2 * NEED_LANES;         // 32-bit need-mask words per wave
  constexpr uint32_t ROWS_MASK = (1u << TPW) - 1u;
  // The per-row page bitmaps are only needed before streaming starts and
  // share their LDS with the ring.
  __shared__ __align__(16) uint8_t s_ring[LS_ATT_STAGES * LS_ATT_STAGE_BYTES];
  // Union entry: the mask of the tile rows that selected the page, and the page.
  __shared__ uint32_t s_umeta[MAX_UNION];
  __shared__ uint16_t s_upage[MAX_UNION];
  __shared__ uint8_t s_uneed[MAX_UNION];  // waves with a row on the page
  // Bit u of s_wneed[w] is set when a row of wave w selected union page u.
  __shared__ uint32_t s_wneed[LS_ATT_WAVES][NEED_WORDS];
  __shared__ int s_wsum[LS_ATT_WAVES];
  // Ring protocol: s_next = next union page to be claimed for copying;
  // s_rdy[st][0] = union index + 1 of the page whose copy into stage st has
  // landed, s_rdy[st][1] = that page's V exponent (read together); s_done[st] = (union index << 8) | number of its waves done with
  // it, for the page in stage st (tagged, so a stale count never matches).
  __shared__ uint32_t s_next, s_done[LS_ATT_STAGES];
  __shared__ __align__(8) uint32_t s_rdy[LS_ATT_STAGES][2];
  __shared__ __align__(16) float s_bias[BIAS ? LS_ATT_STAGES * 64 : 4];
  static_assert(TILE * LS_ATT_WORDS * 4 <= LS_ATT_STAGES * LS_ATT_STAGE_BYTES,
                "page bitmaps must fit in the ring");
  static_assert(TILE <= 32, "row masks are 32-bit");
  static_assert(LS_ATT_WORDS <= LS_ATT_THREADS, "one bitmap word per thread");
#ifdef LS_ATT_NO_ALIAS
  __shared__ uint32_t s_bits[TILE][LS_ATT_WORDS];
#else
  uint32_t(*s_bits)[LS_ATT_WORDS] = reinterpret_cast<uint32_t(*)[LS_ATT_WORDS]>(s_ring);
#endif

  const int tid = LS_TID;
  const int lane = tid & 63, w = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = lane & 15, q = lane >> 4;

  // XCD-aware tile order.  Consecutive workgroups land on different XCDs
  // (workgroup x runs on XCD x % 8).  Each XCD takes runs of LS_ATT_XCD_CHUNK
  // consecutive tiles, so the tiles in flight on one XCD are neighbours that
  // share pages in its L2, and the runs go round-robin over the XCDs, so every
  // XCD gets an even share of early (small-union) and late (large-union) rows.
  // Runs are taken from the end of the sequence first: the largest tiles
  // start first and small ones fill the tail.  The grid is a multiple of
  // 8 * LS_ATT_XCD_CHUNK, so this is a permutation of the workgroup indices.
  const int64_t xi = LS_BID_X / 8;
  const int64_t tile = 8LL * per_xcd - 1 -
                       ((xi / LS_ATT_XCD_CHUNK) * (8 * LS_ATT_XCD_CHUNK) +
                        (int64_t)(LS_BID_X % 8) * LS_ATT_XCD_CHUNK + xi % LS_ATT_XCD_CHUNK);
  if (tile >= tile_off[batch]) return;
  const int g = LS_BID_Y;
  const int head = LS_BID_Z * 16 + r;
  const bool head_ok = head < gs;

  const int b = ls_find_segment(tile_off, batch, tile);
  const int64_t t0 = (int64_t)cu_q[b] + TILE * (tile - tile_off[b]);
  const int n_rows = (int)min((int64_t)TILE, (int64_t)cu_q[b + 1] - t0);
  const int lq = cu_q[b + 1] - cu_q[b];
  const int lk = cu_k[b + 1] - cu_k[b];
  const int64_t vbase = 64LL * pg_off[b];
  const int64_t tr0 = t0 - cu_q[b];
  // Keys visible to row i of the tile: j <= jmax(i) (the last row sees the most).
  auto row_jmax = [&](int i) -> int64_t {
    int64_t jm = lk - 1;
    if (causal) jm = min(jm, tr0 + i + (int64_t)(lk - lq));
    return jm;
  };
  const int64_t tile_jmax = row_jmax(n_rows - 1);
  const int last_page =
      tile_jmax >= 0 ? (int)min(tile_jmax / 64, (int64_t)LS_ATTN_MAX_PAGES - 1) : -1;
  const int nwords = last_page / 32 + 1;

  // ---- per-row state: Q^T fragments (B operand), softmax stats, O^T ----
  // (the Q loads are issued first; they land while the page list is built)
  ls_u32x4 qf[TPW][4];
  // m_run: running max in scaled base-2 units (score * scale_log2); thr: the
  // raw score above which a key would exceed m_run by more than 2^8.
  float m_run[TPW], l_run[TPW], thr[TPW];
  int jmax_r[TPW];
  ls_f32x4 o[TPW][8];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int row = w * TPW + j;
    const int64_t t = t0 + min(row, n_rows - 1);
    const uint16_t* qrow = qg + t * q_rs + ((int64_t)g * gs + (head_ok ? head : 0)) * D + 8 * q;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      qf[j][ks] = ls_load16(qrow + 32 * ks);
      if (!head_ok) qf[j][ks] = ls_u32x4{0u, 0u, 0u, 0u};
    }
    m_run[j] = -INFINITY;
    l_run[j] = 0.f;
    thr[j] = -INFINITY;
    // Wave-uniform, so each chunk's row mask below is scalar work.
    jmax_r[j] = __builtin_amdgcn_readfirstlane(row < n_rows ? (int)row_jmax(row) : -1);
#pragma unroll
    for (int db = 0; db < 8; ++db) o[j][db] = ls_f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // ---- per-row page bitmaps and their sorted union ----
  for (int i = tid; i < TILE * nwords; i += LS_ATT_THREADS) s_bits[i / nwords][i % nwords] = 0u;
  for (int i = tid; i < LS_ATT_WAVES * NEED_WORDS; i += LS_ATT_THREADS)
    s_wneed[i / NEED_WORDS][i % NEED_WORDS] = 0u;
  if (tid < LS_ATT_STAGES) {
    s_rdy[tid][0] = 0u;
    s_done[tid] = 0u;
  }
  if (tid == 0) s_next = LS_ATT_STAGES;  // pages 0..3 are copied at the start
  __syncthreads();
  if (last_page >= 0) {
    const int32_t* ids = topk_idx + ((int64_t)g * total_q + t0) * take;
    for (int i = tid; i < n_rows * take; i += LS_ATT_THREADS) {
      const int row = i / take;
      const int p = ids[i];
      const int64_t jm = row_jmax(row);
      if (p >= 0 && jm >= 0 && p <= jm / 64 && p <= last_page)
        atomicOr(&s_bits[row][p >> 5], 1u << (p & 31));
    }
  }
  __syncthreads();
  uint32_t word = 0u, row_word[TILE];
#pragma unroll
  for (int i = 0; i < TILE; ++i) {
    row_word[i] = tid < nwords ? s_bits[i][tid] : 0u;
    word |= row_word[i];
  }
  int wtot;
  const int wpos = ls_wave_excl_scan(__popc(word), lane, &wtot);
  if (lane == 0) s_wsum[w] = wtot;
  __syncthreads();
  int pos = wpos;
  for (int i = 0; i < w; ++i) pos += s_wsum[i];
  int n_union = 0;
#pragma unroll
  for (int i = 0; i < LS_ATT_WAVES; ++i) n_union += s_wsum[i];
  const int32_t* vexp_seq = vexp + (int64_t)g * n_pages_ws + pg_off[b];
  const float inv_scale_log2 = 1.f / scale_log2;
  // Page order.  Where the rows share many pages (at least
  // LS_ATT_SHARE_STRIDED / 10 plan ids per union page) the pages are visited in
  // a strided order (ascending page i goes to slot i * stride mod n_union, a
  // bijection for stride coprime to n_union): neighbouring pages tend to be
  // selected by the same rows, and spreading them out evens the work of the
  // waves over any window of pages.  Where they share few, ascending order:
  // the tiles running side by side on an XCD then reach a shared page at
  // nearly the same time, while it is still in that XCD's L2, and the waves'
  // work is even anyway.  (Empty or one-page lists keep stride 1; a coprime
  // odd stride below 64 + 7 exists for any list this kernel accepts, the loop
  // bound only caps it.)
  int stride = 1;
  if (n_union > 1 && 10 * n_rows * take >= LS_ATT_SHARE_STRIDED * n_union) {
    for (int cand = 7; cand < 71; cand += 2) {
      int a = cand, b = n_union;
      while (b) {
        const int t = a % b;
        a = b;
        b = t;
      }
      if (a == 1) {
        stride = cand;
        break;
      }
    }
  }
  while (word) {
    const int bit = __ffs(word) - 1;
    word &= word - 1;
    const int page = tid * 32 + bit;
    uint32_t rows = 0u;
#pragma unroll
    for (int i = 0; i < TILE; ++i) rows |= ((row_word[i] >> bit) & 1u) << i;
    const int dst = (int)(((uint32_t)pos * (uint32_t)stride) % (uint32_t)n_union);
    int n_waves = 0;
#pragma unroll
    for (int i = 0; i < LS_ATT_WAVES; ++i) {
      if (((rows >> (TPW * i)) & ROWS_MASK) != 0u) {
        ++n_waves;
        atomicOr(&s_wneed[i][dst >> 5], 1u << (dst & 31));
      }
    }
    s_umeta[dst] = rows;
    s_upage[dst] = (uint16_t)page;
    s_uneed[dst] = (uint8_t)n_waves;
    ++pos;
  }

  __syncthreads();  // the union list is complete and the bitmaps are dead, so
                    // the ring may be written
  LS_WAIT_VMCNT(0);
  // This wave's pages: bit b of lane l is set when one of its rows selected
  // union page 64 l + b (the union holds at most 64 x 64 pages).
  static_assert(NEED_LANES <= 64, "one need word per lane");
  const uint64_t wneed =
      lane < NEED_LANES
          ? ((uint64_t)s_wneed[w][2 * lane + 1] << 32) | (uint64_t)s_wneed[w][2 * lane]
          : 0ull;

  // ---- staging ----
  // One wave copies a whole union page into its stage: the page's staged
  // block (K rows with chunk C of row R at position C ^ (R & 15), V^T rows
  // with chunk C of row d at C ^ ((d >> 1) & 7), so the sixteen lanes of an
  // MFMA operand read hit sixteen distinct bank groups) is copied byte for
  // byte, 1 KB per load (lane l -> byte 16 l).
  //
  // Waves are not kept in lockstep, and a wave visits only the pages its rows
  // selected, waiting only for the page it is about to read.  Union page u
  // goes to stage u % 4.  The copies of pages 0..3 are issued at the start.
  // A waiting wave claims the next unclaimed page (at most three ahead of the
  // page it waits for) once every wave with rows on the stage's previous page
  // is done with it, issues its copy and goes back to waiting without
  // waiting for the copy: the copy's final load brings the page's token
  // (union index + 1) from global memory into s_rdy[stage][0], and a wave's
  // loads land in issue order, so the token lands after the page's K, V^T and
  // bias.  Computing waves never copy (the last wave on a page is often the
  // slowest one).  A page's copy depends only on earlier pages being
  // finished, so every wait ends.
  const uint8_t* kvgrp = kv + ((int64_t)g * n_pages_ws + pg_off[b]) * LS_ATT_STAGE_BYTES;
  const float* cgrp = BIAS ? cb + (int64_t)g * lpad + vbase : nullptr;
  const uint32_t ring_off = __builtin_amdgcn_readfirstlane(
      (uint32_t)(uintptr_t)(ls_lds_void*)s_ring);
  auto issue_page = [&](int ui_copy) {
    const int page = __builtin_amdgcn_readfirstlane((int)s_upage[ui_copy]);
    const uint32_t kb = ring_off + (ui_copy % LS_ATT_STAGES) * LS_ATT_STAGE_BYTES;
    // The staged page is the stage's byte image: 32 contiguous 1 KB copies.
    const uint8_t* src = kvgrp + (int64_t)page * LS_ATT_STAGE_BYTES;
#pragma unroll
    for (int i = 0; i < LS_ATT_STAGE_BYTES / 1024; ++i)
      ls_dma16(src + 1024 * i, 16u * (uint32_t)lane, kb + i * 1024);
    // The page's 64 biases (lanes 0..15, 16 bytes each).
    if constexpr (BIAS)
      if (lane < 16)
        ls_dma16(cgrp + 64LL * page, 16u * (uint32_t)lane,
                 (uint32_t)(uintptr_t)(ls_lds_void*)s_bias + (ui_copy % LS_ATT_STAGES) * 256u);
    // The page's V exponent, then last the ready token ui_copy + 1 (lane 0 only).
    if (lane == 0) {
      ls_dma4(vexp_seq + page, 0u,
              (uint32_t)(uintptr_t)(ls_lds_void*)&s_rdy[ui_copy % LS_ATT_STAGES][1]);
      ls_dma4(tok + ui_copy + 1, 0u,
              (uint32_t)(uintptr_t)(ls_lds_void*)&s_rdy[ui_copy % LS_ATT_STAGES][0]);
    }
  };
  // Hands stage u % 4 to page u (its waves count from zero) and copies it.
  auto issue_copy = [&](int u) {
    if (lane == 0)
      __hip_atomic_store(&s_done[u % LS_ATT_STAGES], (uint32_t)u << 8, __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_WORKGROUP);
    LS_WAIT_LGKMCNT0();  // the count is reset before the token can land
    issue_page(u);
  };
  // A waiting wave at page ui claims and copies page s_next when its stage is free.
  auto try_claim = [&](int ui) {
    const int nx = __builtin_amdgcn_readfirstlane(
        (int)__hip_atomic_load(&s_next, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP));
    if (nx >= n_union || nx > ui + LS_ATT_STAGES - 1) return false;
    const int prev = nx - LS_ATT_STAGES;  // >= 0: pages 0..3 are copied at the start
    const uint32_t want = ((uint32_t)prev << 8) | (uint32_t)s_uneed[prev];
    if ((uint32_t)__builtin_amdgcn_readfirstlane((int)__hip_atomic_load(
            &s_done[nx % LS_ATT_STAGES], __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP)) != want)
      return false;  // a wave may still read the stage's previous page
    int won = 0;
    if (lane == 0) {
      uint32_t expect = (uint32_t)nx;
      won = __hip_atomic_compare_exchange_strong(&s_next, &expect, (uint32_t)nx + 1u,
                                                 __ATOMIC_ACQ_REL, __ATOMIC_RELAXED,
                                                 __HIP_MEMORY_SCOPE_WORKGROUP);
    }
    if (!__builtin_amdgcn_readfirstlane(won)) return false;
    issue_copy(nx);
    return true;
  };
  if (w < LS_ATT_STAGES && w < n_union) issue_copy(w);
  // The ready token (low word) and V exponent (high word) of union page ui's
  // stage, read in one access: the exponent lands before the token, so a
  // read that sees the token sees the page's exponent.
  auto stage_word = [&](int ui) -> uint64_t {
    return __hip_atomic_load(reinterpret_cast<uint64_t*>(&s_rdy[ui % LS_ATT_STAGES][0]),
                             __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  auto is_ready = [&](int ui, uint64_t word) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)word) == (uint32_t)ui + 1u;
  };

  auto compute_page = [&](int ui, int page, uint32_t sel, int v_e) {
    const float p_unscale = __builtin_ldexpf(1.f, -v_e);
    const uint8_t* kb = s_ring + (ui % LS_ATT_STAGES) * LS_ATT_STAGE_BYTES;
    const uint8_t* vb = kb + LS_ATT_KBYTES;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const int base = 64 * page + 32 * c;
      uint32_t need = 0;
#pragma unroll
      for (int j = 0; j < TPW; ++j) need |= (uint32_t)(((sel >> j) & 1u) && base <= jmax_r[j]) << j;
      if (!need) continue;
      // The chunk's K and V^T fragments are read once and shared by the rows.
      const int R0 = 32 * c + r, R1 = 32 * c + 16 + r;
      ls_u32x4 kf0[4], kf1[4], vf[8];
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const int C = 4 * ks + q;
        kf0[ks] = *reinterpret_cast<const ls_u32x4*>(kb + R0 * 256 + ((C ^ (R0 & 15)) << 4));
        kf1[ks] = *reinterpret_cast<const ls_u32x4*>(kb + R1 * 256 + ((C ^ (R1 & 15)) << 4));
      }
      // V^T row 16 db + r (so (row >> 1) & 7 == (r >> 1) & 7), logical chunk 4c + q.
      const uint8_t* vrow = vb + r * 128 + (((4 * c + q) ^ ((r >> 1) & 7)) << 4);
      ls_f32x4 cbv0, cbv1;  // this lane's eight key biases (BIAS only)
      if constexpr (BIAS) {
        const float* bp = s_bias + (ui % LS_ATT_STAGES) * 64 + 32 * c + 8 * q;
        cbv0 = *reinterpret_cast<const ls_f32x4*>(bp);
        cbv1 = *reinterpret_cast<const ls_f32x4*>(bp + 4);
      }
      // S^T of one row: lane (r, q) gets head r's raw scores of keys base + 8q + 0..7.
      auto qk = [&](int j, ls_f32x4& s0, ls_f32x4& s1) {
        s0 = ls_f32x4{0.f, 0.f, 0.f, 0.f};
        s1 = ls_f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < 4; ++ks) {
          s0 = LsElem<DT>::mfma(kf0[ks], qf[j][ks], s0);
          s1 = LsElem<DT>::mfma(kf1[ks], qf[j][ks], s1);
        }
      };
      // Online softmax update of row j with its chunk scores, then O^T += V^T P^T.
      auto soft_pv = [&](int j, const ls_f32x4& s0, const ls_f32x4& s1) {
        float sv[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
        if (base + 31 > jmax_r[j]) {  // the chunk crosses this row's causal frontier
          // This lane's last visible key offset, formed here so that the eight
          // key indices are not kept for every chunk (the empty asm keeps the
          // compiler from rewriting the compares back into them).
          int lim = jmax_r[j] - base - 8 * q;
          asm("" : "+v"(lim));
#pragma unroll
          for (int i = 0; i < 8; ++i)
            if (i > lim) sv[i] = -INFINITY;
        }
        // With a bias the scores are taken to base-2 units here (thr, m_run
        // and the maxima below are then all in those units).
        if constexpr (BIAS) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            sv[i] = fmaf(sv[i], scale_log2, cbv0[i]);
            sv[4 + i] = fmaf(sv[4 + i], scale_log2, cbv1[i]);
          }
        }
        // Plain maxima: the compiler inserts the wait states an MFMA result
        // needs before a VALU read (it cannot for inline asm), and this file is
        // built without IEEE NaN quieting, so they fuse into v_max3 (grouped
        // here as three v_max3 and one v_max).
        const float lmax = fmaxf(fmaxf(fmaxf(sv[6], sv[7]), fmaxf(fmaxf(sv[0], sv[1]), sv[2])),
                                 fmaxf(fmaxf(sv[3], sv[4]), sv[5]));
        // Rescale only when some head's max grows by more than 2^8 (or when the
        // page's V scale leaves too little fp16 headroom for P up to 2^8).
        if (__ballot(lmax > thr[j]) != 0ull || v_e > 7) {
          float cm = lmax;
          cm = fmaxf(cm, ls_shfl_xor(cm, 16));
          cm = fmaxf(cm, ls_shfl_xor(cm, 32));
          const float m_new = fmaxf(m_run[j], BIAS ? cm : cm * scale_log2);
          const float alpha = __builtin_amdgcn_exp2f(m_run[j] - m_new);
          m_run[j] = m_new;
          thr[j] = BIAS ? m_new + 8.f : (m_new + 8.f) * inv_scale_log2;
          l_run[j] *= alpha;
#pragma unroll
          for (int db = 0; db < 8; ++db) o[j][db] *= alpha;
        }
        // P' = P * 2^e (the page's V scale moved onto P, exact): one exp each;
        // the row sum adds the fp16 P' that the MFMA uses, scaled back by 2^-e.
        const float bias = (float)v_e - m_run[j];
        ls_u32x4 pf;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          if constexpr (BIAS)
            pf[i] = ls_pack_f16x2(__builtin_amdgcn_exp2f(sv[2 * i] + bias),
                                  __builtin_amdgcn_exp2f(sv[2 * i + 1] + bias));
          else
            pf[i] = ls_pack_f16x2(__builtin_amdgcn_exp2f(fmaf(sv[2 * i], scale_log2, bias)),
                                  __builtin_amdgcn_exp2f(fmaf(sv[2 * i + 1], scale_log2, bias)));
        }
        const float lsum = ls_sum_f16x2(pf[3], ls_sum_f16x2(pf[2], ls_sum_f16x2(pf[1], ls_sum_f16x2(pf[0], 0.f))));
        l_run[j] = fmaf(lsum, p_unscale, l_run[j]);
        // The row's V^T fragments, read where they are used.
#pragma unroll
        for (int db = 0; db < 8; ++db) vf[db] = *reinterpret_cast<const ls_u32x4*>(vrow + db * 2048);
#pragma unroll
        for (int db = 0; db < 8; ++db) o[j][db] = LsElem<LS_F16>::mfma(vf[db], pf, o[j][db]);
      };
#pragma unroll
      for (int j = 0; j < TPW; ++j) {
        if (!((need >> j) & 1u)) continue;
        ls_f32x4 s0, s1;
        qk(j, s0, s1);
        soft_pv(j, s0, s1);
      }
    }
  };

  // Next page of this wave: the lowest set need bit above `after` (n_union if none).
  auto next_page = [&](int after) -> int {
    const int from = after + 1, fl = from >> 6;
    const uint64_t word = lane < fl ? 0ull : (lane == fl ? wneed & (~0ull << (from & 63)) : wneed);
    const uint64_t lanes = __ballot(word != 0ull);
    if (lanes == 0ull) return n_union;
    const int L = (int)__builtin_ctzll(lanes);
    const uint64_t wl = ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(word >> 32), L) << 32) |
                        (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)word, L);
    return 64 * L + (int)__builtin_ctzll(wl);
  };
  // The next page's union entry is read before the current page is computed.
  int ui = next_page(-1);
  uint32_t meta = ui < n_union ? s_umeta[ui] : 0u;
  int page_cur = ui < n_union ? (int)s_upage[ui] : 0;
  int spins = spin_limit;  // bound of this wave's next wait (in polls)
  while (ui < n_union) {
    uint64_t sw = stage_word(ui);
    if (!is_ready(ui, sw)) {
      // Bounded wait (the protocol cannot deadlock; the bound only guarantees
      // that a wave always finishes).  A wave whose wait expires reports it
      // in the status word and goes on without waiting again (its outputs are
      // void), so a broken ring costs one bound per wave, not one per page;
      // the host turns the status into an error, and the epilogue below
      // writes NaN rows once it is set.
      bool landed = false;
      for (int spin = 0; spin < spins; ++spin) {
        if (!try_claim(ui)) __builtin_amdgcn_s_sleep(LS_ATT_SPIN_SLEEP);
        sw = stage_word(ui);
        if (is_ready(ui, sw)) {
          landed = true;
          break;
        }
      }
      if (!landed) {
        spins = 0;
        if (lane == 0)
          __hip_atomic_fetch_or(status, LS_ATTN_RING_TIMEOUT, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
      }
    }

    const int nxt = next_page(ui);
    const uint32_t meta_next = nxt < n_union ? s_umeta[nxt] : 0u;
    const int page_next = nxt < n_union ? (int)s_upage[nxt] : 0;
    const uint32_t m = (uint32_t)__builtin_amdgcn_readfirstlane((int)meta);
    compute_page(ui, __builtin_amdgcn_readfirstlane(page_cur), (m >> (TPW * w)) & ROWS_MASK,
                 __builtin_amdgcn_readfirstlane((int)(uint32_t)(sw >> 32)));
    // Done with the stage (the release orders this wave's reads of it first).
    if (lane == 0)
      __hip_atomic_fetch_add(&s_done[ui % LS_ATT_STAGES], 1u, __ATOMIC_RELEASE,
                             __HIP_MEMORY_SCOPE_WORKGROUP);
    ui = nxt;
    meta = meta_next;
    page_cur = page_next;
  }
  LS_WAIT_VMCNT(0);  // no copy of this wave may land after the workgroup ends

  // ---- epilogue ----
  // A wait that expired (this wave's, or any earlier one seen here) makes the
  // rows NaN, so the failure also shows where the host cannot read the status
  // word (a replayed graph).  Read once per wave, after the loop.
  const bool expired = (__builtin_amdgcn_readfirstlane((int)__hip_atomic_load(
                            status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) &
                        LS_ATTN_RING_TIMEOUT) != 0;
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int row = w * TPW + j;
    float l_tot = l_run[j] + ls_shfl_xor(l_run[j], 16);
    l_tot += ls_shfl_xor(l_tot, 32);
    if (row >= n_rows || !head_ok) continue;
    const int64_t t = t0 + row;
    const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
    uint16_t* orow = out + (t * G * gs + (int64_t)g * gs + head) * D + 4 * q;
    if (expired) {  // quiet-NaN bit patterns (this file assumes no NaN arithmetic)
      const uint32_t nan2 = DT == LS_BF16 ? 0x7fc07fc0u : 0x7e007e00u;
#pragma unroll
      for (int db = 0; db < 8; ++db) *reinterpret_cast<uint2*>(orow + 16 * db) = make_uint2(nan2, nan2);
      if (lse && q == 0) lse[((int64_t)g * gs + head) * total_q + t] = __uint_as_float(0x7fc00000u);
      continue;
    }
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const uint32_t lo = ls_pack2(LsElem<DT>::from_f(o[j][db][0] * inv), LsElem<DT>::from_f(o[j][db][1] * inv));
      const uint32_t hi = ls_pack2(LsElem<DT>::from_f(o[j][db][2] * inv), LsElem<DT>::from_f(o[j][db][3] * inv));
      *reinterpret_cast<uint2*>(orow + 16 * db) = make_uint2(lo, hi);
    }
    if (lse && q == 0)
      lse[((int64_t)g * gs + head) * total_q + t] =
          l_tot > 0.f ? m_run[j] * 0.69314718055994531f + __logf(l_tot) : INFINITY;
  }
}

// NOSA key biases: cb[g][64 pg_off[b] + j] = log2(e) * cis[cu_k[b] + j][g] for
// j < len_k(b), 0 past each sequence end (those keys are never visible).  One
// workgroup per 64-key page of one group.
template <int CT>
__global__ __launch_bounds__(64) void ls_bias_kernel(const typename LsElem<CT>::T* __restrict__ cis,
                                                     int64_t cis_rs, const int32_t* __restrict__ cu_k,
                                                     const int32_t* __restrict__ pg_off, int batch,
                                                     int64_t lpad, float* __restrict__ cb) {
  const int64_t tile_id = LS_BID_X;
  if (tile_id >= pg_off[batch]) return;
  const int g = LS_BID_Y;
  const int b = ls_find_segment(pg_off, batch, tile_id);
  const int p = (int)(tile_id - pg_off[b]);
  const int lk = cu_k[b + 1] - cu_k[b];
  const int j = 64 * p + LS_TID;
  float v = 0.f;
  if (j < lk) v = LsElem<CT>::to_f(cis[((int64_t)cu_k[b] + j) * cis_rs + g]) * 1.4426950408889634f;
  cb[(int64_t)g * lpad + 64LL * (pg_off[b] + p) + LS_TID] = v;
}

// ---------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------
namespace {
constexpr int kDefaultSpinLimit = 1 << 22;
int g_spin_limit = kDefaultSpinLimit;  // bound of one ring wait (in polls)

struct AttnWs {
  size_t status, kv, pg, tiles, vexp, cb, tok, total;
  int64_t lpad, n_pages;
};
AttnWs attn_ws(int64_t total_k, int batch, int G, bool bias) {
  AttnWs L;
  L.n_pages = (total_k + 63) / 64 + batch;
  L.lpad = L.n_pages * 64;
  size_t off = 0;
  L.status = off; off += 256;  // the call's status word comes first
  L.kv = off; off += ls_align256((size_t)G * L.n_pages * LS_ATT_STAGE_BYTES);
  L.pg = off; off += ls_align256((size_t)(batch + 1) * 4);
  L.tiles = off; off += ls_align256((size_t)(batch + 1) * 4);
  L.vexp = off; off += ls_align256((size_t)G * L.n_pages * 4);
  L.cb = off; off += bias ? ls_align256((size_t)G * L.lpad * 4) : 0;
  L.tok = off; off += ls_align256((size_t)(LS_ATT_UNION_CAP + 1) * 4);
  L.total = off;
  return L;
}

template <int DT, bool BIAS, int TPW>
void launch_tile(dim3 grid, hipStream_t s, const void* q, int64_t q_rs, const uint8_t* kv,
                 const AttnWs& L, const int32_t* vexp, const float* cb,
                 const int32_t* tok,
                 const int32_t* cu_q, const int32_t* cu_k, const int32_t* pg,
                 const int32_t* tiles, int batch, int64_t total_q, int G, int gs,
                 const int32_t* topk_idx, int take, float scale_log2, int causal, void* out,
                 float* lse, int32_t* status) {
  hipLaunchKernelGGL((ls_attn_tile_kernel<DT, BIAS, TPW>), grid, dim3(LS_ATT_THREADS), 0, s,
                     (const uint16_t*)q, q_rs, kv, L.lpad, vexp, cb, tok,
                     L.n_pages, cu_q, cu_k, pg, tiles, batch, total_q, G, gs, topk_idx, take,
                     scale_log2, causal, (uint16_t*)out, lse, (int)(grid.x / 8), status,
                     g_spin_limit);
}

// Shared body of the plain and the NOSA (cis != nullptr) entry points.
int attn_run(const char* who, const void* q, int64_t q_row_stride, const void* k,
             int64_t k_row_stride, const void* v, int64_t v_row_stride, const void* cis,
             int64_t cis_row_stride, int32_t cis_dtype, const int32_t* cu_seqlens_q,
             const int32_t* cu_seqlens_k, int32_t batch, int64_t total_q, int64_t total_k,
             int32_t max_seqlen_k, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
             int32_t dtype, const int32_t* topk_idx, int32_t take, int32_t block_size,
             float softmax_scale, int32_t causal, void* out, float* lse, void* workspace,
             size_t workspace_bytes, void* stream, int32_t* status_out = nullptr) {
  const bool bias = cis != nullptr;
  LS_REQUIRE(dtype == LS_BF16 || dtype == LS_F16, LS_ERR_UNSUPPORTED,
             "%s: only bf16 and fp16 are supported (dtype %d)", who, dtype);
  LS_REQUIRE(head_dim == 128, LS_ERR_UNSUPPORTED, "%s: head_dim must be 128 (got %d)", who,
             head_dim);
  LS_REQUIRE(block_size == 64, LS_ERR_UNSUPPORTED, "%s: block_size must be 64 (got %d)", who,
             block_size);
  LS_REQUIRE(num_heads > 0 && num_kv_heads > 0 && num_heads % num_kv_heads == 0, LS_ERR_INVALID,
             "%s: num_heads must be a positive multiple of num_kv_heads", who);
  LS_REQUIRE(batch >= 0 && total_q >= 0 && total_k >= 0 && take >= 0, LS_ERR_INVALID,
             "%s: bad sizes", who);
  LS_REQUIRE(take <= LS_ATTN_MAX_TAKE, LS_ERR_UNSUPPORTED, "%s: at most %d ids per row (got %d)",
             who, LS_ATTN_MAX_TAKE, take);
  LS_REQUIRE((int64_t)max_seqlen_k <= 64LL * LS_ATTN_MAX_PAGES, LS_ERR_UNSUPPORTED,
             "%s: max_seqlen_k above %d", who, 64 * LS_ATTN_MAX_PAGES);
  LS_REQUIRE(!bias || cis_dtype == LS_F32 || cis_dtype == LS_BF16 || cis_dtype == LS_F16,
             LS_ERR_INVALID, "%s: unknown CIS dtype %d", who, cis_dtype);
  if (total_q == 0 || batch == 0) return LS_OK;
  LS_REQUIRE(q && k && v && out && cu_seqlens_q && cu_seqlens_k && (take == 0 || topk_idx),
             LS_ERR_INVALID, "%s: null pointer", who);
  LS_REQUIRE(ls_aligned16(q) && ls_aligned16(k) && ls_aligned16(v) && ls_aligned16(out) &&
                 q_row_stride % 8 == 0 && k_row_stride % 8 == 0 && v_row_stride % 8 == 0,
             LS_ERR_UNSUPPORTED,
             "%s: tensors must be 16-byte aligned with row strides %% 8 == 0", who);
  const AttnWs L = attn_ws(total_k, batch, num_kv_heads, bias);
  LS_REQUIRE(workspace && workspace_bytes >= L.total, LS_ERR_WORKSPACE,
             "%s: workspace needs %zu bytes", who, L.total);
  hipStream_t s = (hipStream_t)stream;
  char* ws = (char*)workspace;
  uint8_t* kv = (uint8_t*)(ws + L.kv);
  int32_t* pg = (int32_t*)(ws + L.pg);
  int32_t* vexp = (int32_t*)(ws + L.vexp);
  int32_t* tiles = (int32_t*)(ws + L.tiles);
  float* cb = bias ? (float*)(ws + L.cb) : nullptr;
  int32_t* tok = (int32_t*)(ws + L.tok);
  int32_t* status = status_out ? status_out : (int32_t*)(ws + L.status);
  // 24-row tiles (three rows a wave): their union bound holds every plan accepted.
  constexpr int kTpw = 3;
  static_assert(LsAttTile<kTpw>::kMaxTake >= LS_ATTN_MAX_TAKE, "every accepted plan fits a tile");
  const int tile_rows = LsAttTile<kTpw>::kTile;
  hipLaunchKernelGGL(ls_attn_plan_kernel, dim3(1), dim3(64), 0, s, cu_seqlens_q, cu_seqlens_k,
                     batch, tile_rows, pg, tiles, tok, LS_ATT_UNION_CAP + 1, status);
  int rc = ls_check_launch("ls_attn_plan_kernel");
  if (rc) return rc;
  if (total_k > 0) {
    const dim3 vgrid((unsigned)((total_k + 63) / 64 + batch), num_kv_heads);
    if (dtype == LS_BF16)
      hipLaunchKernelGGL(ls_kv_stage_kernel<LS_BF16>, vgrid, dim3(256), 0, s, (const uint16_t*)k,
                         k_row_stride, (const uint16_t*)v, v_row_stride, cu_seqlens_k, pg, batch,
                         L.n_pages, kv, vexp);
    else
      hipLaunchKernelGGL(ls_kv_stage_kernel<LS_F16>, vgrid, dim3(256), 0, s, (const uint16_t*)k,
                         k_row_stride, (const uint16_t*)v, v_row_stride, cu_seqlens_k, pg, batch,
                         L.n_pages, kv, vexp);
    if ((rc = ls_check_launch("ls_kv_stage_kernel"))) return rc;
    if (bias) {
      if (cis_dtype == LS_BF16)
        hipLaunchKernelGGL(ls_bias_kernel<LS_BF16>, vgrid, dim3(64), 0, s, (const uint16_t*)cis,
                           cis_row_stride, cu_seqlens_k, pg, batch, L.lpad, cb);
      else if (cis_dtype == LS_F16)
        hipLaunchKernelGGL(ls_bias_kernel<LS_F16>, vgrid, dim3(64), 0, s, (const uint16_t*)cis,
                           cis_row_stride, cu_seqlens_k, pg, batch, L.lpad, cb);
      else
        hipLaunchKernelGGL(ls_bias_kernel<LS_F32>, vgrid, dim3(64), 0, s, (const float*)cis,
                           cis_row_stride, cu_seqlens_k, pg, batch, L.lpad, cb);
      if ((rc = ls_check_launch("ls_bias_kernel"))) return rc;
    }
  }
  const int gs = num_heads / num_kv_heads;
  const float scale = softmax_scale > 0.f ? softmax_scale : 1.0f / sqrtf((float)head_dim);
  const float scale_log2 = scale * 1.4426950408889634f;
  const int64_t tile_bound = (total_q + tile_rows - 1) / tile_rows + batch;
  constexpr int64_t kRound = 8 * LS_ATT_XCD_CHUNK;  // whole runs on every XCD
  const dim3 grid((unsigned)(kRound * ((tile_bound + kRound - 1) / kRound)), num_kv_heads,
                  (gs + 15) / 16);
#define LS_TILE_ARGS                                                                              \
  grid, s, q, q_row_stride, kv, L, vexp, cb, tok, cu_seqlens_q, cu_seqlens_k, pg,              \
      tiles, batch, total_q, num_kv_heads, gs, topk_idx, take, scale_log2, causal, out, lse, \
      status
  if (dtype == LS_BF16) {
    if (bias) launch_tile<LS_BF16, true, kTpw>(LS_TILE_ARGS);
    else launch_tile<LS_BF16, false, kTpw>(LS_TILE_ARGS);
  } else {
    if (bias) launch_tile<LS_F16, true, kTpw>(LS_TILE_ARGS);
    else launch_tile<LS_F16, false, kTpw>(LS_TILE_ARGS);
  }
#undef LS_TILE_ARGS
  return ls_check_launch("ls_attn_tile_kernel");
}
}  // namespace

extern "C" int32_t ls_attn_set_spin_limit(int32_t spins) {
  const int32_t prev = g_spin_limit;
  g_spin_limit = spins < 0 ? kDefaultSpinLimit : spins;
  return prev;
}

extern "C" size_t ls_sparse_attn_workspace_size(int64_t total_k, int32_t batch,
                                                int32_t num_kv_heads, int32_t head_dim,
                                                int32_t max_seqlen_k, int32_t dtype) {
  (void)max_seqlen_k;
  (void)head_dim;
  (void)dtype;
  return attn_ws(total_k, batch, num_kv_heads, false).total;
}

extern "C" size_t ls_nosa_attn_workspace_size(int64_t total_k, int32_t batch,
                                              int32_t num_kv_heads, int32_t head_dim,
                                              int32_t max_seqlen_k, int32_t dtype) {
  (void)max_seqlen_k;
  (void)head_dim;
  (void)dtype;
  return attn_ws(total_k, batch, num_kv_heads, true).total;
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
  (void)max_seqlen_q;
  return attn_run("ls_sparse_attn_varlen", q, q_row_stride, k, k_row_stride, v, v_row_stride,
                  nullptr, 0, 0, cu_seqlens_q, cu_seqlens_k, batch, total_q, total_k,
                  max_seqlen_k, num_heads, num_kv_heads, head_dim, dtype, topk_idx, take,
                  block_size, softmax_scale, causal, out, lse, workspace, workspace_bytes,
                  stream);
}

extern "C" int ls_nosa_attn_varlen(const void* q, int64_t q_row_stride, const void* k,
                                   int64_t k_row_stride, const void* v, int64_t v_row_stride,
                                   const void* cis, int64_t cis_row_stride, int32_t cis_dtype,
                                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                                   int32_t batch, int64_t total_q, int64_t total_k,
                                   int32_t max_seqlen_q, int32_t max_seqlen_k, int32_t num_heads,
                                   int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
                                   const int32_t* topk_idx, int32_t take, int32_t block_size,
                                   float softmax_scale, void* out, float* lse, void* workspace,
                                   size_t workspace_bytes, void* stream) {
  (void)max_seqlen_q;
  LS_REQUIRE(total_k == 0 || cis, LS_ERR_INVALID, "ls_nosa_attn_varlen: null CIS scores");
  static const uint16_t kNoKeys = 0;  // any non-null pointer: no key reads it
  return attn_run("ls_nosa_attn_varlen", q, q_row_stride, k, k_row_stride, v, v_row_stride,
                  cis ? cis : &kNoKeys, cis_row_stride, cis_dtype, cu_seqlens_q, cu_seqlens_k,
                  batch, total_q, total_k, max_seqlen_k, num_heads, num_kv_heads, head_dim,
                  dtype, topk_idx, take, block_size, softmax_scale, 1, out, lse, workspace,
                  workspace_bytes, stream);
}

// ---------------------------------------------------------------------------
// Allocation-free variant of ls_sparse_attn_varlen: the workspace is a static
// device array of the library instead of a caller buffer.  In host code
// `scratch` only names the symbol; its device address (one per GPU) comes
// from hipGetSymbolAddress, taken once per device with that device current.
// ---------------------------------------------------------------------------
#define LS_MAX_DEVICES 64  // LS_NOALLOC_SCRATCH_BYTES comes from the public header

static __device__ __align__(256) uint8_t scratch[LS_NOALLOC_SCRATCH_BYTES];

namespace {
std::mutex g_scratch_mu;
void* g_scratch_ptr[LS_MAX_DEVICES] = {};

// Device address of `scratch` on the device that owns `stream`.
int scratch_for_stream(hipStream_t stream, void** ptr) {
  int dev = -1;
  hipError_t e = stream ? hipStreamGetDevice(stream, &dev) : hipGetDevice(&dev);
  if (e != hipSuccess)
    return ls_fail(LS_ERR_HIP, "ls_sparse_attn_varlen_noalloc: no device for the stream: %s",
                   hipGetErrorString(e));
  LS_REQUIRE(dev >= 0 && dev < LS_MAX_DEVICES, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen_noalloc: device %d out of range", dev);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    int cur = -1;
    if ((e = hipGetDevice(&cur)) != hipSuccess)
      return ls_fail(LS_ERR_HIP, "ls_sparse_attn_varlen_noalloc: %s", hipGetErrorString(e));
    if (cur != dev && (e = hipSetDevice(dev)) != hipSuccess)
      return ls_fail(LS_ERR_HIP, "ls_sparse_attn_varlen_noalloc: %s", hipGetErrorString(e));
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (e != hipSuccess || !p)
      return ls_fail(LS_ERR_HIP, "ls_sparse_attn_varlen_noalloc: scratch address on device %d: %s",
                     dev, hipGetErrorString(e));
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return LS_OK;
}
}  // namespace

extern "C" int ls_sparse_attn_varlen_noalloc(
    const void* q, int64_t q_row_stride, const void* k, int64_t k_row_stride, const void* v,
    int64_t v_row_stride, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int32_t batch,
    int64_t total_q, int64_t total_k, int32_t max_seqlen_q, int32_t max_seqlen_k,
    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, int32_t dtype,
    const int32_t* topk_idx, int32_t take, int32_t block_size, float softmax_scale,
    int32_t causal, void* out, float* lse, int32_t* status, void* stream) {
  (void)max_seqlen_q;
  // The size check comes first and touches no device.
  LS_REQUIRE(batch >= 0 && total_k >= 0 && num_kv_heads > 0, LS_ERR_INVALID,
             "ls_sparse_attn_varlen_noalloc: bad sizes");
  const size_t need = attn_ws(total_k, batch, num_kv_heads, false).total;
  LS_REQUIRE(need <= LS_NOALLOC_SCRATCH_BYTES, LS_ERR_UNSUPPORTED,
             "ls_sparse_attn_varlen_noalloc: %lld keys in %d sequences of %d KV heads need "
             "%zu bytes of scratch, above the static %u (use ls_sparse_attn_varlen with a "
             "workspace)",
             (long long)total_k, batch, num_kv_heads, need, LS_NOALLOC_SCRATCH_BYTES);
  if (total_q == 0 || batch == 0) {
    // Nothing to attend; the caller's status word still gets this call's value.
    if (!status) return LS_OK;
    hipLaunchKernelGGL(ls_attn_status_clear_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream,
                       status);
    return ls_check_launch("ls_attn_status_clear_kernel");
  }
  void* ws = nullptr;
  const int rc = scratch_for_stream((hipStream_t)stream, &ws);
  if (rc) return rc;
  return attn_run("ls_sparse_attn_varlen_noalloc", q, q_row_stride, k, k_row_stride, v,
                  v_row_stride, nullptr, 0, 0, cu_seqlens_q, cu_seqlens_k, batch, total_q,
                  total_k, max_seqlen_k, num_heads, num_kv_heads, head_dim, dtype, topk_idx,
                  take, block_size, softmax_scale, causal, out, lse, ws,
                  LS_NOALLOC_SCRATCH_BYTES, stream, status);
}
