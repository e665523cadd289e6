// Shared device/host helpers for the gfx950 LeanSelect kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stddef.h>

#include "../../include/leanselect_hip.h"

#define LS_WAVE 64

typedef __bf16 ls_bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 ls_f16x8 __attribute__((ext_vector_type(8)));
typedef float ls_f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t ls_u32x4 __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------------------
// Host-side error plumbing (definitions in ls_runtime.hip).
// ---------------------------------------------------------------------------
int ls_fail(int code, const char* fmt, ...);
int ls_check_launch(const char* what);

#define LS_REQUIRE(cond, code, ...)          \
  do {                                       \
    if (!(cond)) return ls_fail((code), __VA_ARGS__); \
  } while (0)

static inline size_t ls_align256(size_t x) { return (x + 255) & ~(size_t)255; }
static inline size_t ls_dtype_bytes(int dt) { return dt == LS_F32 ? 4 : 2; }
static inline bool ls_aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

// ---------------------------------------------------------------------------
// Scalar conversions.  bf16 rounding is round-to-nearest-even of the float32
// bit pattern (NaN -> canonical quiet NaN), which is what torch's float->bf16
// cast does, so a kernel output rounds exactly like the reference's tensors.
// ---------------------------------------------------------------------------
__device__ __forceinline__ float ls_bf16_to_f32(uint16_t b) {
  return __uint_as_float(((uint32_t)b) << 16);
}

// Round to nearest even (v_cvt_pk_bf16_f32 on gfx950; NaN stays NaN).
__device__ __forceinline__ uint16_t ls_f32_to_bf16(float f) {
  return __builtin_bit_cast(uint16_t, (__bf16)f);
}

__device__ __forceinline__ float ls_f16_to_f32(uint16_t b) {
  return (float)__builtin_bit_cast(_Float16, b);
}

__device__ __forceinline__ uint16_t ls_f32_to_f16(float f) {
  // Materialise the float32 value first: otherwise the compiler may fuse the
  // producing multiply into a mixed-precision op that rounds once to fp16,
  // which differs from torch's float32-then-fp16 double rounding on ties.
  asm volatile("" : "+v"(f));
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// Element traits: storage type, float conversions and the 16x16x32 MFMA.
template <int DT> struct LsElem;

template <> struct LsElem<LS_BF16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float to_f(T v) { return ls_bf16_to_f32(v); }
  static __device__ __forceinline__ T from_f(float v) { return ls_f32_to_bf16(v); }
  static __device__ __forceinline__ ls_f32x4 mfma(ls_u32x4 a, ls_u32x4 b, ls_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(ls_bf16x8, a),
                                                   __builtin_bit_cast(ls_bf16x8, b), c, 0, 0, 0);
  }
};

template <> struct LsElem<LS_F16> {
  typedef uint16_t T;
  static __device__ __forceinline__ float to_f(T v) { return ls_f16_to_f32(v); }
  static __device__ __forceinline__ T from_f(float v) { return ls_f32_to_f16(v); }
  static __device__ __forceinline__ ls_f32x4 mfma(ls_u32x4 a, ls_u32x4 b, ls_f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(ls_f16x8, a),
                                                  __builtin_bit_cast(ls_f16x8, b), c, 0, 0, 0);
  }
};

template <> struct LsElem<LS_F32> {
  typedef float T;
  static __device__ __forceinline__ float to_f(T v) { return v; }
  static __device__ __forceinline__ T from_f(float v) { return v; }
};

// Two 16-bit values packed into one 32-bit lane register.
__device__ __forceinline__ uint32_t ls_pack2(uint16_t lo, uint16_t hi) {
  return (uint32_t)lo | ((uint32_t)hi << 16);
}

// 16-byte global load (8 half-width elements or 4 floats).
__device__ __forceinline__ ls_u32x4 ls_load16(const void* p) {
  return *reinterpret_cast<const ls_u32x4*>(p);
}

// Lane helpers.
__device__ __forceinline__ int ls_lane() { return (int)__lane_id(); }

__device__ __forceinline__ float ls_shfl(float v, int src_lane) {
  return __shfl(v, src_lane, LS_WAVE);
}

__device__ __forceinline__ float ls_shfl_xor(float v, int mask) {
  return __shfl_xor(v, mask, LS_WAVE);
}

// Wave-wide maximum / minimum of a 32-bit value, with all 64 lanes active.
// DPP steps inside each row of 16 lanes (swaps within quads, then the
// half-row and row mirrors) leave every lane with its row's result; the four
// row results are then read into scalar registers.  No LDS round trip, unlike
// a shuffle reduction.  The result is uniform.  (No source lane of these
// patterns lies outside its row, so bound_ctrl changes nothing here; it lets
// each move fold into the min/max as one DPP instruction.)
template <bool MAX>
__device__ __forceinline__ uint32_t ls_wave_extreme_u32(uint32_t x) {
  auto pick = [](uint32_t a, uint32_t b) { return MAX ? max(a, b) : min(a, b); };
  x = pick(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0xB1, 0xF, 0xF, true));
  x = pick(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x4E, 0xF, 0xF, true));
  x = pick(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x141, 0xF, 0xF, true));
  x = pick(x, (uint32_t)__builtin_amdgcn_mov_dpp((int)x, 0x140, 0xF, 0xF, true));
  const uint32_t a = (uint32_t)__builtin_amdgcn_readlane((int)x, 0);
  const uint32_t b = (uint32_t)__builtin_amdgcn_readlane((int)x, 16);
  const uint32_t c = (uint32_t)__builtin_amdgcn_readlane((int)x, 32);
  const uint32_t d = (uint32_t)__builtin_amdgcn_readlane((int)x, 48);
  return pick(pick(a, b), pick(c, d));
}
__device__ __forceinline__ uint32_t ls_wave_max_u32(uint32_t x) { return ls_wave_extreme_u32<true>(x); }
__device__ __forceinline__ uint32_t ls_wave_min_u32(uint32_t x) { return ls_wave_extreme_u32<false>(x); }

// NaN-propagating maximum (v_maximum3_f32 on gfx950), as torch's amax and
// max_pool1d propagate NaN.  Only meaningful where NaN is honoured (files
// built without -fno-honor-nans).
__device__ __forceinline__ float ls_fmax_nan(float a, float b) {
  return __builtin_elementwise_maximum(a, b);
}

// NaN of either sign becomes the positive canonical quiet NaN, whose order key
// lies above +inf's (torch.topk ranks every NaN above +inf).
__device__ __forceinline__ float ls_canon_nan(float x) {
  return __builtin_isnan(x) ? __builtin_nanf("") : x;
}

// Order-preserving unsigned keys of 16-bit (bf16 / fp16) and float32 scores:
// a > b as floats  <=>  key(a) > key(b) as integers (NaN aside).
__host__ __device__ __forceinline__ uint32_t ls_order_key16(uint16_t b) {
  return (b & 0x8000u) ? (~(uint32_t)b & 0xffffu) : ((uint32_t)b | 0x8000u);
}
__host__ __device__ __forceinline__ uint32_t ls_order_key32(uint32_t u) {
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Number of set bits of `mask` in the lanes below this one.
__device__ __forceinline__ int ls_lanes_below(uint64_t mask) {
  return (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(mask >> 32),
                                        __builtin_amdgcn_mbcnt_lo((uint32_t)mask, 0u));
}

// k-th largest key of one wave-wide row: keys live in NS register slots of
// 64 lanes, 0 marks an empty slot and is never counted.  The result is the
// largest T with #{key >= T} >= kk (0 when fewer than kk keys are nonzero).
// Plain bisection over the bits below top_bit, starting from prefix T.
template <int NS>
__device__ __forceinline__ uint32_t ls_kth_bisect(const uint32_t (&key)[NS], int kk, uint32_t T,
                                                  int top_bit) {
#pragma unroll 1
  for (int bit = top_bit; bit >= 0; --bit) {
    const uint32_t cand = T | (1u << bit);
    int cnt = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) cnt += __popcll(__ballot(key[s] >= cand));
    if (cnt >= kk) T = cand;
  }
  return T;
}

// The same for long rows (kk <= 128), with a wave-private LDS scratch of 256
// words.  lo = the kk-th largest of the lanes' two largest keys is a lower
// bound of the answer (those keys are a subset of the row), so every key the
// answer counts is >= lo; the keys >= lo are gathered into four slots (when
// at most 256 of them) and bisected from the common bit prefix of lo and the
// row maximum, which the answer shares.  Otherwise plain bisection.
template <int NS, int BITS>
__device__ __forceinline__ uint32_t ls_kth_key_row(const uint32_t (&key)[NS], int kk,
                                                   uint32_t* __restrict__ scr, int lane) {
  if constexpr (NS <= 4) {
    return ls_kth_bisect<NS>(key, kk, 0u, BITS - 1);
  } else {
    if (kk < 1 || kk > 128) return ls_kth_bisect<NS>(key, kk, 0u, BITS - 1);
    uint32_t m1 = 0u, m2 = 0u;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      m2 = max(m2, min(m1, key[s]));
      m1 = max(m1, key[s]);
    }
    const uint32_t mm[2] = {m1, m2};
    const uint32_t lo = ls_kth_bisect<2>(mm, kk, 0u, BITS - 1);
    if (lo == 0u) return ls_kth_bisect<NS>(key, kk, 0u, BITS - 1);
    int n = 0;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const bool sv = key[s] >= lo;
      const uint64_t mk = __ballot(sv);
      const int pos = n + ls_lanes_below(mk);
      if (sv && pos < 256) scr[pos] = key[s];
      n += __popcll(mk);
    }
    if (n > 256) return ls_kth_bisect<NS>(key, kk, 0u, BITS - 1);
    uint32_t sk[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) sk[i] = i * 64 + lane < n ? scr[i * 64 + lane] : 0u;
    const uint32_t hi = ls_wave_max_u32(m1);
    const uint32_t d = lo ^ hi;
    if (d == 0u) return lo;
    const int tb = 31 - __builtin_clz(d);
    const uint32_t T0 = tb >= 31 ? 0u : (lo & ~((2u << tb) - 1u));
    return ls_kth_bisect<4>(sk, kk, T0, tb);
  }
}

// ---------------------------------------------------------------------------
// Direct global->LDS copies and counter waits (gfx9 encodings).
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void ls_lds_void;

// One 16-byte global->LDS load per lane from sbase + voff bytes (lane l lands
// at lds_off + 16 l; sbase and lds_off are wave-uniform, voff a 32-bit lane
// offset).  Issued as inline asm so the compiler's wait insertion does not
// treat every later LDS read as aliasing the in-flight copy (which would
// drain the whole prefetch queue); callers order the copies themselves with
// vmcnt waits and barriers or ready tokens.  An SALU write of M0 followed by a
// global load with LDS destination needs one wait state, which the compiler
// cannot insert inside the asm block.  M0 is listed as clobbered, which the
// compiler notes it may not honour for a reserved register: every copy sets
// M0 itself, and no code of these kernels keeps a value in M0 across one (no
// indexed register moves, GWS, append/consume or messages).
__device__ __forceinline__ void ls_dma16(const void* sbase, uint32_t voff, uint32_t lds_off) {
  const uint64_t a = (uint64_t)(uintptr_t)sbase;
  // (readfirstlane returns int: widen each half as unsigned, or the low half
  // would be sign-extended into the high one.)
  const uint64_t sa = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sa), "s"((uint32_t)__builtin_amdgcn_readfirstlane(lds_off))
               : "memory", "m0");
}

// One 4-byte global->LDS load per active lane (lane l lands at lds_off + 4 l).
__device__ __forceinline__ void ls_dma4(const void* sbase, uint32_t voff, uint32_t lds_off) {
  const uint64_t a = (uint64_t)(uintptr_t)sbase;
  const uint64_t sa = ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)(a >> 32)) << 32) |
                      (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)a);
  asm volatile("s_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dword %0, %1"
               :
               : "v"(voff), "s"(sa), "s"((uint32_t)__builtin_amdgcn_readfirstlane(lds_off))
               : "memory", "m0");
}

// lgkmcnt(0) with the other counters left alone (gfx9 encoding).
#define LS_WAIT_LGKMCNT0() __builtin_amdgcn_s_waitcnt(0xf | (0x7 << 4) | (0x3 << 14))

// vmcnt(n) with the other counters left alone (gfx9 encoding).
#define LS_WAIT_VMCNT(n) \
  __builtin_amdgcn_s_waitcnt(((n) & 0xf) | (((n) >> 4) << 14) | (0x7 << 4) | (0xf << 8))

// Index of the segment containing `x` in a nondecreasing prefix array
// `off[0..n]` (off[0] == 0): largest b < n with off[b] <= x.
__device__ __forceinline__ int ls_find_segment(const int32_t* off, int n, int64_t x) {
  int lo = 0, hi = n - 1;
  while (lo < hi) {
    int mid = (lo + hi + 1) >> 1;
    if ((int64_t)off[mid] <= x) lo = mid; else hi = mid - 1;
  }
  return lo;
}
