// Wave-level top-k of one score row (shared by the prefill and decode
// selections).
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

#include "ls_common.h"

// Order keys whose pages are chosen but emitted as -1: keys above `hi` (NaN
// scores, whose keys lie above +inf's once NaN is canonical) and the key
// `ninf` (-inf).  The default rule marks none (no key exceeds 0xffffffff and
// the empty key 0 is never emitted).
struct LsInvalidKeys {
  uint32_t hi = 0xffffffffu;
  uint32_t ninf = 0u;
};

// An emitted page id: -1 above id_max (rows whose kept ids end at a bound)
// and for keys the rule marks invalid.
__device__ __forceinline__ int32_t ls_topk_id(int id, int id_max, uint32_t key,
                                              const LsInvalidKeys& rule) {
  return (id > id_max || key > rule.hi || key == rule.ninf) ? -1 : id;
}

// ---------------------------------------------------------------------------
// Top-k page selection.  One wave per row.  The k'-th largest
// order-preserving key T is found by bisection over the key bits, counting
// with ballots over keys held in registers; pages above T and the first
// (lowest-index) pages equal to T are emitted in ascending order between the
// sink pages and the local pages.
// ---------------------------------------------------------------------------
// Top-kk of one row's cn candidate scores (columns base .. base + cn - 1 of
// P), held as order-preserving keys in NS register slots of 64 lanes.  Loads
// are issued together (addresses clamped into the row), then converted; keys
// of lanes past cn are 0, which no threshold candidate (>= 1) counts.  The
// kk-th largest key T is found by bisection over the key bits with ballot
// counts; the winners (key > T, then the first kk - #{key > T} keys equal to
// T in page order) are written in page order after the lo_end sink pages.
// Returns T (uniform).
template <int NS, bool KEY32>
__device__ __forceinline__ uint32_t ls_topk_row(const void* __restrict__ P, int64_t base, int cn,
                                                int kk, int lo_end, int lane,
                                                int32_t* __restrict__ orow,
                                                uint32_t* __restrict__ scr, int id_max,
                                                const LsInvalidKeys& rule = LsInvalidKeys()) {
  uint32_t key[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int c = min(s * 64 + lane, cn - 1);
    if constexpr (KEY32) key[s] = ((const uint32_t*)P)[base + c];
    else key[s] = ((const uint16_t*)P)[base + c];
  }
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    uint32_t k;
    if constexpr (KEY32) k = ls_order_key32(key[s]);
    else k = ls_order_key16((uint16_t)key[s]);
    key[s] = s * 64 + lane < cn ? k : 0u;
  }
  const uint32_t T = ls_kth_key_row<NS, KEY32 ? 32 : 16>(key, kk, scr, lane);
  int gt = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) gt += __popcll(__ballot(key[s] > T));
  const int m = kk - gt;

  int out_pos = lo_end, eq_before = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const int c = s * 64 + lane;
    const bool valid = c < cn;
    const bool eq = valid && key[s] == T;
    const uint64_t eq_mask = __ballot(eq);
    const int eq_rank = eq_before + ls_lanes_below(eq_mask);
    const bool sel = valid && (key[s] > T || (eq && eq_rank < m));
    const uint64_t sel_mask = __ballot(sel);
    const int pos = out_pos + ls_lanes_below(sel_mask);
    if (sel && pos < lo_end + kk) orow[pos] = ls_topk_id(lo_end + c, id_max, key[s], rule);  // exactly kk
    out_pos += __popcll(sel_mask);
    eq_before += __popcll(eq_mask);
  }
  return T;
}

// The end of ls_topk_row16 for n gathered candidates (key << 16 | column,
// in column order) held in NP slots of the wave's scratch: the kk-th key T
// bisected from the common bit prefix of lo and the row maximum m1 (per-lane
// maxima, reduced here), then the chosen columns written in column order.
// Returns T (uniform).
// (or_mask is OR-ed into every gathered entry as it is read back: the bf16
// fast path below gathers raw score bits, which become order keys that way;
// with m1_reduced, m1 is already the row maximum and is not reduced again.)
template <int NP>
__device__ __forceinline__ uint32_t ls_topk_emit_packed(const uint32_t* __restrict__ scr, int n,
                                                        uint32_t lo, uint32_t m1, int kk,
                                                        int lo_end, int lane,
                                                        int32_t* __restrict__ orow, int id_max,
                                                        const LsInvalidKeys& rule = LsInvalidKeys(),
                                                        uint32_t or_mask = 0u,
                                                        bool m1_reduced = false) {
  uint32_t pk[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i) pk[i] = i * 64 + lane < n ? (scr[i * 64 + lane] | or_mask) : 0u;
  const uint32_t hi = m1_reduced ? m1 : ls_wave_max_u32(m1);
  // T: the largest 16-bit key with #{key >= T} >= kk, sharing lo's and hi's
  // common bit prefix.
  uint32_t T = lo;
  const uint32_t d = lo ^ hi;
  if (d != 0u) {
    const int tb = 31 - __builtin_clz(d);
    T = lo & ~((2u << tb) - 1u);
#pragma unroll 1
    for (int bit = tb; bit >= 0; --bit) {
      const uint32_t cand = (T | (1u << bit)) << 16;
      int cnt = 0;
#pragma unroll
      for (int i = 0; i < NP; ++i) cnt += __popcll(__ballot(pk[i] >= cand));
      if (cnt >= kk) T |= 1u << bit;
    }
  }
  const uint32_t above = (T << 16) | 0xffffu;  // packed keys above T
  int gt = 0;
#pragma unroll
  for (int i = 0; i < NP; ++i) gt += __popcll(__ballot(pk[i] > above));
  const int m = kk - gt;
  int out_pos = lo_end, eq_before = 0;
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const bool valid = i * 64 + lane < n;
    const bool eq = valid && (pk[i] >> 16) == T;
    const uint64_t eq_mask = __ballot(eq);
    const int eq_rank = eq_before + ls_lanes_below(eq_mask);
    const bool sel = valid && (pk[i] > above || (eq && eq_rank < m));
    const uint64_t sel_mask = __ballot(sel);
    const int pos = out_pos + ls_lanes_below(sel_mask);
    if (sel && pos < lo_end + kk)
      orow[pos] = ls_topk_id(lo_end + (int)(pk[i] & 0xffffu), id_max, pk[i] >> 16, rule);
    out_pos += __popcll(sel_mask);
    eq_before += __popcll(eq_mask);
  }
  return T;
}

// The same for 16-bit scores of rows of more than four slots, emitting from
// the gathered candidates: the keys >= lo (lo = the kk-th largest of the
// lanes' two largest keys, a lower bound of the kk-th key) are packed as
// key << 16 | column into at most four slots in column order, the kk-th key T
// is bisected on them from the common bit prefix of lo and the row maximum,
// and the chosen columns (keys > T, then the lowest-column ties) are written
// from those four slots instead of from all NS.  When more than 256 keys pass
// (or no bound exists) the row is searched and emitted over all NS slots.
template <int NS>
__device__ __forceinline__ uint32_t ls_topk_row16(const void* __restrict__ P, int64_t base, int cn,
                                                  int kk, int lo_end, int lane,
                                                  int32_t* __restrict__ orow,
                                                  uint32_t* __restrict__ scr, int id_max,
                                                  const LsInvalidKeys& rule = LsInvalidKeys()) {
  if (NS <= 4 || kk < 1 || kk > 128)
    return ls_topk_row<NS, false>(P, base, cn, kk, lo_end, lane, orow, scr, id_max, rule);
  // Keys are held shifted up by 16 (order key << 16), so a gathered entry is
  // key | column; 0 marks a column past the row.  Only the slots that reach
  // the row's end (a uniform test) pay for the per-lane column check.
  cn = __builtin_amdgcn_readfirstlane(cn);
  uint32_t key[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) key[s] = ((const uint16_t*)P)[base + min(s * 64 + lane, cn - 1)];
  const int n_full = cn >> 6;  // slots lying wholly inside the row (uniform)
  uint32_t m1 = 0u, m2 = 0u;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const uint32_t b = key[s];
    uint32_t k = (b ^ ((b >> 15) * 0x7fffu) ^ 0x8000u) << 16;  // ls_order_key16(b) << 16
    if (s >= n_full) k = s * 64 + lane < cn ? k : 0u;
    key[s] = k;
    m2 = max(m2, min(m1, k));
    m1 = max(m1, k);
  }
  m1 >>= 16;
  m2 >>= 16;
  const uint32_t mm[2] = {m1, m2};
  const uint32_t lo = ls_kth_bisect<2>(mm, kk, 0u, 15);
  // Gather the keys >= lo with their columns, in column order; stop once more
  // than 256 have been found (the scratch holds 256 + 63).
  int n = 0;
  if (lo != 0u) {
    const uint32_t lo_sh = lo << 16;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      if (n <= 256) {
        const bool sv = key[s] >= lo_sh;
        const uint64_t mk = __ballot(sv);
        const int pos = (int)__builtin_amdgcn_mbcnt_hi(
            (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, (uint32_t)n));
        if (sv) scr[pos] = key[s] | (uint32_t)(s * 64 + lane);
        n += __popcll(mk);
      }
    }
  }
  if (lo == 0u || n > 256) {  // no usable bound: every slot is searched and emitted
#pragma unroll
    for (int s = 0; s < NS; ++s) key[s] >>= 16;
    // (The row length is re-read through an empty asm so that the column
    // checks below are formed here, not kept alive from the loop above.)
    asm volatile("" : "+s"(cn));
    const uint32_t T = ls_kth_bisect<NS>(key, kk, 0u, 15);
    int gt = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) gt += __popcll(__ballot(key[s] > T));
    const int m = kk - gt;
    int out_pos = lo_end, eq_before = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const int c = s * 64 + lane;
      const bool valid = c < cn;
      const bool eq = valid && key[s] == T;
      const uint64_t eq_mask = __ballot(eq);
      const int eq_rank = eq_before + ls_lanes_below(eq_mask);
      const bool sel = valid && (key[s] > T || (eq && eq_rank < m));
      const uint64_t sel_mask = __ballot(sel);
      const int pos = out_pos + ls_lanes_below(sel_mask);
      if (sel && pos < lo_end + kk) orow[pos] = ls_topk_id(lo_end + c, id_max, key[s], rule);
      out_pos += __popcll(sel_mask);
      eq_before += __popcll(eq_mask);
    }
    return T;
  }
  if (n <= 64) return ls_topk_emit_packed<1>(scr, n, lo, m1, kk, lo_end, lane, orow, id_max, rule);
  if (n <= 128) return ls_topk_emit_packed<2>(scr, n, lo, m1, kk, lo_end, lane, orow, id_max, rule);
  return ls_topk_emit_packed<4>(scr, n, lo, m1, kk, lo_end, lane, orow, id_max, rule);
}


// The top kk of cn 16-bit scores at P[base ..], written in column order to
// orow[lo_end ..] as lo_end + column (ids above id_max as -1), by one wave of
// which every lane calls this.  The slot count (uniform) picks one
// straight-line body, in steps of about an eighth so that a row runs few empty
// slots; rows of up to four slots are searched over all their keys.
// Returns the kk-th key T (uniform, the 16-bit order key).
template <int KPL>
__device__ __forceinline__ uint32_t ls_topk_select16(const void* __restrict__ P, int64_t base,
                                                     int cn, int kk, int lo_end, int lane,
                                                     int32_t* __restrict__ orow,
                                                     uint32_t* __restrict__ scr, int id_max,
                                                     const LsInvalidKeys& rule = LsInvalidKeys()) {
  const int n_slots = (cn + 63) >> 6;
  if (n_slots <= 1)
    return ls_topk_row<1, false>(P, base, cn, kk, lo_end, lane, orow, scr, id_max, rule);
  if (n_slots <= 2)
    return ls_topk_row<2, false>(P, base, cn, kk, lo_end, lane, orow, scr, id_max, rule);
  if (n_slots <= 4 || KPL <= 4)
    return ls_topk_row<(KPL < 4 ? KPL : 4), false>(P, base, cn, kk, lo_end, lane, orow, scr,
                                                   id_max, rule);
#define LS_TOPK16_CASE(N)                                                                  \
  if (n_slots <= (N) || KPL <= (N))                                                        \
    return ls_topk_row16<(KPL < (N) ? KPL : (N))>(P, base, cn, kk, lo_end, lane, orow, scr, \
                                                  id_max, rule);
  LS_TOPK16_CASE(6)
  LS_TOPK16_CASE(8)
  LS_TOPK16_CASE(10)
  LS_TOPK16_CASE(12)
  LS_TOPK16_CASE(14)
  LS_TOPK16_CASE(16)
  LS_TOPK16_CASE(20)
  LS_TOPK16_CASE(24)
  LS_TOPK16_CASE(28)
  LS_TOPK16_CASE(32)
  LS_TOPK16_CASE(40)
  LS_TOPK16_CASE(48)
  LS_TOPK16_CASE(56)
  LS_TOPK16_CASE(64)
  LS_TOPK16_CASE(96)
#undef LS_TOPK16_CASE
  return ls_topk_row16<KPL>(P, base, cn, kk, lo_end, lane, orow, scr, id_max, rule);
}

// Fast path of ls_topk_row16 for a row of bf16 scores whose kk-th largest
// score is positive and which holds no NaN.  The row is read through a buffer
// resource bounded at cn columns, so the slots need no address clamping and no
// per-lane column masks: reads past the row return 0, i.e. +0.0, which only the
// bound check below has to keep out.  The scores are compared as float32 (the
// bf16 bits shifted up by 16), which orders them as their order keys do apart
// from -0 / +0, and that difference cannot matter here:
//  * the lanes' two largest values (v_maximum / v_med3; a NaN anywhere makes
//    the lane maximum NaN) are values of distinct row entries or of the +0 read
//    past the row, and their order keys are at most those entries' keys, so the
//    kk-th largest of those keys, lo, is a lower bound of the row's kk-th key
//    when it lies above +0's key (then no +0 read past the row is among the kk);
//  * every score >= lo (as floats) is gathered with its column (at most 256 of
//    them), which includes every key >= lo, and none of the +0 past the row;
//  * all gathered scores are positive, so bf16 | 0x8000 is their order key and
//    the gathered entries become ls_topk_emit_packed's key << 16 | column with
//    one OR.
// Returns false, having written nothing to orow, when a condition fails (kk
// outside 1..128, a NaN, lo at or below +0, more than 256 gathered); the caller
// then runs the general path.  Otherwise T is the kk-th largest order key.
template <int NS>
__device__ __forceinline__ bool ls_topk_row16_bf16(const uint16_t* __restrict__ row, int cn,
                                                   int kk, int lo_end, int lane,
                                                   int32_t* __restrict__ orow,
                                                   uint32_t* __restrict__ scr, int id_max,
                                                   const LsInvalidKeys& rule, uint32_t& T) {
  if (kk < 1 || kk > 128) return false;
  // One resource bounded at the row's end; each slot's whole byte offset is
  // a lane register (hidden from the compiler, so that no part of it moves
  // into the scalar offset, which the hardware range check leaves out).
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc((void*)row, (short)0, cn * 2, 0x00020000);
  uint32_t f[NS];
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    uint32_t off = (uint32_t)(lane * 2 + 128 * s);
    asm("" : "+v"(off));
    f[s] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b16(rs, (int)off, 0, 0) << 16;
  }
  float m1 = -INFINITY, m2 = -INFINITY;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const float x = __uint_as_float(f[s]);
    m2 = __builtin_amdgcn_fmed3f(m1, m2, x);
    m1 = __builtin_elementwise_maximum(m1, x);
  }
  if (__ballot(__builtin_isnan(m1)) != 0ull) return false;
  const uint32_t k1 = ls_order_key16((uint16_t)(__float_as_uint(m1) >> 16));
  const uint32_t k2 = ls_order_key16((uint16_t)(__float_as_uint(m2) >> 16));
  // lo: the kk-th largest of the 128 keys, bisected below the bit prefix that
  // all of them share (that of the smallest second and the largest first key),
  // with the loop unrolled.
  const uint32_t kmin = ls_wave_min_u32(k2), kmax = ls_wave_max_u32(k1);
  const uint32_t dk = kmin ^ kmax;
  const int top = dk ? 31 - __builtin_clz(dk) : -1;  // highest differing bit
  uint32_t lo = top >= 0 ? kmin & ~((2u << top) - 1u) : kmin;
#pragma unroll
  for (int bit = 15; bit >= 0; --bit) {
    if (bit <= top) {
      const uint32_t cand = lo | (1u << bit);
      const int cnt = __popcll(__ballot(k1 >= cand)) + __popcll(__ballot(k2 >= cand));
      lo = cnt >= kk ? cand : lo;
    }
  }
  if (lo <= 0x8000u) return false;  // the bound must be a positive score
  const float lo_f = __uint_as_float((lo & 0x7fffu) << 16);
  // Gather without branches: a lane whose score is below lo writes a word of
  // its own past the 256 entries (words 256 + lane), and entries beyond 256
  // (the row then takes the general path) all land on word 255.
  int n = 0;
#pragma unroll
  for (int s = 0; s < NS; ++s) {
    const bool sv = __uint_as_float(f[s]) >= lo_f;
    const uint64_t mk = __ballot(sv);
    int pos = (int)__builtin_amdgcn_mbcnt_hi(
        (uint32_t)(mk >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)mk, (uint32_t)n));
    asm("" : "+v"(pos));  // formed in every lane: the store below needs no branch
    scr[sv ? min(pos, 255) : 256 + lane] = f[s] | (uint32_t)(s * 64 + lane);
    n += __popcll(mk);
  }
  if (n > 256) return false;
  if (n <= 64)
    T = ls_topk_emit_packed<1>(scr, n, lo, kmax, kk, lo_end, lane, orow, id_max, rule, 0x80000000u,
                                   true);
  else if (n <= 128)
    T = ls_topk_emit_packed<2>(scr, n, lo, kmax, kk, lo_end, lane, orow, id_max, rule, 0x80000000u,
                                   true);
  else
    T = ls_topk_emit_packed<4>(scr, n, lo, kmax, kk, lo_end, lane, orow, id_max, rule, 0x80000000u,
                                   true);
  return true;
}

// ls_topk_select16 for bf16 rows of more than four slots through the fast path
// above (same slot-count steps); false when the row needs the general path
// (rows of up to four slots always do).
template <int KPL>
__device__ __forceinline__ bool ls_topk_select16_bf16(const uint16_t* __restrict__ row, int cn,
                                                      int kk, int lo_end, int lane,
                                                      int32_t* __restrict__ orow,
                                                      uint32_t* __restrict__ scr, int id_max,
                                                      const LsInvalidKeys& rule, uint32_t& T) {
  const int n_slots = (cn + 63) >> 6;
  if (n_slots <= 4 || KPL <= 4) return false;
#define LS_TOPK16F_CASE(N)                                                                   \
  if (n_slots <= (N) || KPL <= (N))                                                          \
    return ls_topk_row16_bf16<(KPL < (N) ? KPL : (N))>(row, cn, kk, lo_end, lane, orow, scr, \
                                                       id_max, rule, T);
  LS_TOPK16F_CASE(6)
  LS_TOPK16F_CASE(8)
  LS_TOPK16F_CASE(10)
  LS_TOPK16F_CASE(12)
  LS_TOPK16F_CASE(14)
  LS_TOPK16F_CASE(16)
  LS_TOPK16F_CASE(20)
  LS_TOPK16F_CASE(24)
  LS_TOPK16F_CASE(28)
  LS_TOPK16F_CASE(32)
  LS_TOPK16F_CASE(40)
  LS_TOPK16F_CASE(48)
  LS_TOPK16F_CASE(56)
  LS_TOPK16F_CASE(64)
  LS_TOPK16F_CASE(96)
#undef LS_TOPK16F_CASE
  return ls_topk_row16_bf16<KPL>(row, cn, kk, lo_end, lane, orow, scr, id_max, rule, T);
}
