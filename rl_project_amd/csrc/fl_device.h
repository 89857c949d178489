// Device-side helpers shared by the sampling kernels (gfx950, wave64).
//
// Rounding helpers reproduce how PyTorch evaluates a reduced-precision tensor
// op with a Python scalar operand: the element is widened to float32, combined
// with the scalar rounded to float32, and the float32 result is rounded to the
// tensor dtype with round-to-nearest-even.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <rocprim/warp/warp_reduce.hpp>
#include <rocprim/warp/warp_scan.hpp>

#include "../../include/fl_sampler.h"

// Phase timestamps for kernel tuning builds (-DFL_PHASE_TIMES): thread 0 of
// each of the first 1024 work-groups records the constant-rate wall clock at
// each FL_MARK(n), n < 32, in slot 32 * blockIdx.x + n.
#ifdef FL_PHASE_TIMES
#define FL_PHASE_SLOTS (32 * 1024)
static __device__ uint64_t fl_phase_ts[FL_PHASE_SLOTS];
#ifndef FL_MARK_MASK
#define FL_MARK_MASK 0xFFFFFFFFu  // marks recorded (bit n: FL_MARK(n)); fewer marks, fewer spills
#endif
#define FL_MARK(n)                                                              \
  do {                                                                          \
    if (((FL_MARK_MASK >> (n)) & 1) && threadIdx.x == 0 && blockIdx.x < 1024)   \
      fl_phase_ts[blockIdx.x * 32 + (n)] = wall_clock64();                      \
  } while (0)
#else
#define FL_MARK(n) \
  do {             \
  } while (0)
#endif

namespace fl {

constexpr int NT = 1024;          // threads per work-group
constexpr int WAVE = 64;
constexpr int NWAVE = NT / WAVE;

// ---------------------------------------------------------------- dtypes

struct BF16 {
  static constexpr int id = FL_DTYPE_BF16;
  static constexpr uint32_t INF_BITS = 0x7F80u;
  __device__ static __forceinline__ float to_f32(uint32_t b) { return __uint_as_float(b << 16); }
  __device__ static __forceinline__ uint32_t from_f32(float x) {
    const uint32_t u = __float_as_uint(x);
    const uint32_t rne = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    return ((u & 0x7fffffffu) > 0x7f800000u) ? ((u >> 16) | 0x40u) : rne;  // a NaN stays a quiet NaN
  }
  __device__ static __forceinline__ float rn(float x) { return to_f32(from_f32(x)); }
};

struct F16 {
  static constexpr int id = FL_DTYPE_F16;
  static constexpr uint32_t INF_BITS = 0x7C00u;
  __device__ static __forceinline__ float to_f32(uint32_t b) {
    return __half2float(__ushort_as_half(static_cast<unsigned short>(b)));
  }
  // (the empty asm keeps x a rounded float32: without it the compiler fuses
  // a product into this conversion (v_fma_mixlo_f16) and rounds the exact
  // product once, where the reference rounds it to float32 first)
  __device__ static __forceinline__ uint32_t from_f32(float x) {
    asm("" : "+v"(x));
    return __half_as_ushort(__float2half_rn(x));
  }
  __device__ static __forceinline__ float rn(float x) { return to_f32(from_f32(x)); }
};

struct F32 {
  static constexpr int id = FL_DTYPE_F32;
  __device__ static __forceinline__ float rn(float x) { return x; }
};

// Raw buffer access to one row: the hardware range check returns zeros for
// bytes at or beyond `bytes`, so loads need neither clamped addresses nor
// branches, and an address is one 32-bit offset (plus an SGPR offset).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t row_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), static_cast<short>(0), static_cast<int>(bytes),
                                           0x00020000);
}
__device__ __forceinline__ uint4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
// The same with the non-temporal cache policy (aux bit 1: nt), for data read
// exactly once: the headline kernel's row tile loads 0.75 us faster per
// launch with it (34.25 -> 33.5 us), the row statistics 3 % faster (A/B on one
// box); the lm_head gemm's weight stream through LDS 4 % faster (376 -> 362 us
// per step).
__device__ __forceinline__ uint4 buf_load16_once(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(r, static_cast<int>(voff), static_cast<int>(soff), 2);
  return make_uint4(v[0], v[1], v[2], v[3]);
}

// Order index of a 16-bit float pattern: 0 for the largest value (+NaN
// patterns first), increasing towards the most negative value.
__device__ __forceinline__ uint32_t order16(uint32_t bits) { return (bits & 0x8000u) ? bits : (0x7FFFu - bits); }
__device__ __forceinline__ uint32_t bits_of_order16(uint32_t o) { return (o & 0x8000u) ? o : (0x7FFFu - o); }

// Monotone uint32 key of a float32: larger float -> larger key.
__device__ __forceinline__ uint32_t f32_key(float x) {
  const uint32_t u = __float_as_uint(x);
  return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}
__device__ __forceinline__ float f32_of_key(uint32_t k) {
  return __uint_as_float((k & 0x80000000u) ? (k & 0x7fffffffu) : ~k);
}

// ------------------------------------------------- per-value transforms
// Each mirrors one tensor op of the reference, evaluated in dtype D.

// tanh.  For |z| < 0.625 the odd polynomial z + z^3 P(z^2), P of degree 5
// with the coefficients below (a weighted least-squares fit of
// (tanh(z) - z) / z^3 driven toward minimax; relative error 1.6e-10 before
// rounding), evaluated by Horner's rule in FMAs: over every float32 in
// [0, 0.625) it lies within 0.75 ulp of tanh, equals the correctly rounded
// value for all but 0.04 % of them, and is monotone (an exhaustive check
// against double-precision tanh runs in the CPU tests).  The odd form makes
// it exactly antisymmetric.  Larger |z| take tanhf, floored in magnitude at
// the polynomial's value at the largest float below 0.625 (which is the
// correctly rounded tanh(0.625); the CPU test checks the constant), so that
// a tanhf an ulp low at the switch cannot make the function decrease there.
// A logit row's values, divided by a soft-cap such as 30, fall in the
// polynomial's range, where a wave then runs this branch alone.
constexpr float TANH_P[6] = {-0.33333330807135236f, 0.13333206186821212f, -0.05394678612676864f,
                             0.021700831796483553f, -0.008177720758405421f, 0.00214326075575256f};
constexpr uint32_t TANH_AT_SWITCH_BITS = 0x3f0dfa3fu;  // poly(nextafter(0.625, 0)) = 0.5545997
__device__ __forceinline__ float fl_tanh(float z) {
  if (fabsf(z) < 0.625f) {
    const float t = z * z;
    float p = __builtin_fmaf(t, TANH_P[5], TANH_P[4]);
    p = __builtin_fmaf(t, p, TANH_P[3]);
    p = __builtin_fmaf(t, p, TANH_P[2]);
    p = __builtin_fmaf(t, p, TANH_P[1]);
    p = __builtin_fmaf(t, p, TANH_P[0]);
    return __builtin_fmaf(z * t, p, z);
  }
  // (a compare and select, not fmaxf: a NaN stays NaN)
  const float a = fabsf(tanhf(z));
  const float lo = __uint_as_float(TANH_AT_SWITCH_BITS);
  return copysignf(a < lo ? lo : a, z);
}

// fl_tanh of four values with one range test: the polynomial for all four
// when every |z| is below the switch (a row's logits over a soft-cap nearly
// always are), else fl_tanh one by one.  Equal to fl_tanh element by element.
__device__ __forceinline__ void fl_tanh4(float (&z)[4]) {
  const float m = fmaxf(fmaxf(fabsf(z[0]), fabsf(z[1])), fmaxf(fabsf(z[2]), fabsf(z[3])));
  if (m < 0.625f) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float t = z[e] * z[e];
      float p = __builtin_fmaf(t, TANH_P[5], TANH_P[4]);
      p = __builtin_fmaf(t, p, TANH_P[3]);
      p = __builtin_fmaf(t, p, TANH_P[2]);
      p = __builtin_fmaf(t, p, TANH_P[1]);
      p = __builtin_fmaf(t, p, TANH_P[0]);
      z[e] = __builtin_fmaf(z[e] * t, p, z[e]);
    }
  } else {
    // (the empty volatile asm keeps this a branch: speculated, the tanhf
    // sequence would run for every chunk)
    asm volatile("" : "+v"(z[0]));
#pragma unroll
    for (int e = 0; e < 4; ++e) z[e] = fl_tanh(z[e]);
  }
}

// soft-cap tanh(x / c) * c  (models/attention/causal.py:109-110): three ops.
template <class D>
__device__ __forceinline__ float softcap_val(float x, float cap) {
  if constexpr (D::id == FL_DTYPE_F32) {
    // float32 rows: x / cap as x * (1 / cap) (1 / cap is loop-invariant and
    // hoisted), at most an ulp from the quotient -- as far as a tanh
    // implementation's own last-place error; the soft-cap is an extension
    // of the reference sampler.  Every kernel applies this same function,
    // so their values agree bit for bit.
    return fl_tanh(x * (1.0f / cap)) * cap;
  } else {
    const float a = D::rn(x / cap);
    const float t = D::rn(fl_tanh(a));
    return D::rn(t * cap);
  }
}

// The float32 soft-cap of four values, rcap = RN(1 / cap): softcap_val<F32>
// element by element.
__device__ __forceinline__ void softcap4_f32(float (&x)[4], float cap, float rcap) {
  float z[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) z[e] = x[e] * rcap;
  fl_tanh4(z);
#pragma unroll
  for (int e = 0; e < 4; ++e) x[e] = z[e] * cap;
}

// repetition penalty on one value (sampling.py:30): x>0 ? x/rp : x*rp.
template <class D>
__device__ __forceinline__ float penalty_val(float x, float rp) {
  return x > 0.0f ? D::rn(x / rp) : D::rn(x * rp);
}

// x / t correctly rounded, for a t fixed per row and rt = recip_rt(t) below.
// q0 = x * rt lies within one ulp of x / t; the remainder x - t * q0 is then
// exact in one FMA, and q0 + remainder * rt rounded once is
// RN(x / t): Markstein's correction (P. Markstein, "Computation of elementary
// functions on the IBM RISC System/6000 processor", IBM J. Res. Dev. 34(1),
// 1990; Theorem 8.10 of Muller et al., Handbook of Floating-Point
// Arithmetic).  It needs the remainder and the quotient in the normal range:
// zeros, operands or quotients below 2^-100 or above 2^100, infinities and
// NaNs take the division itself.  Checked against IEEE division over every
// finite float32 x for 8 divisors and every bfloat16 x for 200000 divisors
// (tests/test_division.py).  Three instructions instead of the ~10 of the
// division sequence.
__device__ __forceinline__ float div_rt(float x, float t, float rt) {
  const float q0 = x * rt;
  const float aq = fabsf(q0);
  if (!(fabsf(x) >= 0x1p-100f && aq >= 0x1p-100f && aq <= 0x1p100f)) {
    // (the empty volatile asm keeps this a branch: speculated into a select,
    // the division sequence would run for every value)
    asm volatile("" : "+v"(x));
    return x / t;
  }
  const float r = __builtin_fmaf(-t, q0, x);
  return __builtin_fmaf(r, rt, q0);
}

// The reciprocal div_rt needs for a divisor t fixed per row: RN(1 / t) for t
// in [2^-100, 2^100], else 0, which sends every quotient to the division
// itself (a t near 2^127 has a subnormal reciprocal, too short for the
// correction).  One IEEE division per row.
__device__ __forceinline__ float recip_rt(float t) {
  return (t >= 0x1p-100f && t <= 0x1p100f) ? 1.0f / t : 0.0f;
}

// repetition penalty with the row's rpr = recip_rt(rp): equal to penalty_val
// bit for bit, the division as div_rt.
template <class D>
__device__ __forceinline__ float penalty_val(float x, float rp, float rpr) {
  return x > 0.0f ? D::rn(div_rt(x, rp, rpr)) : D::rn(x * rp);
}

// temperature (sampling.py:33-34).
template <class D>
__device__ __forceinline__ float temperature_val(float x, float t) {
  return t > 0.0f ? D::rn(x / t) : x;
}
// the same with the row's rt = recip_rt(t) (equal bit for bit)
template <class D>
__device__ __forceinline__ float temperature_val(float x, float t, float rt) {
  return t > 0.0f ? D::rn(div_rt(x, t, rt)) : x;
}

// ------------------------------------------------- fixed-point masses
// Masses e in [0, 1] as unsigned 2^-45 fixed point: sums are exact and
// associative (deterministic scans), and a row of up to 2^18 values sums to
// below 2^63 even when every e is 1 (probabilities, which sum to 1, stay
// below 2^53, so converting their sums back to double is exact).
constexpr int FX_BITS = 45;
constexpr double FX_ONE = 35184372088832.0;  // 2^45
// round(p * 2^45) for p in [0, 1] from the float's fields (ties round up);
// integer arithmetic only
// (with m = the 24-bit significand, p * 2^45 = m * 2^(ex - 105)
// = (m << 24) >> (129 - ex); a right shift of 49 or more leaves 0, as do
// zero and denormals)
__device__ __forceinline__ uint64_t to_fx(float p) {
  const uint32_t u = __float_as_uint(p);
  const uint32_t ex = u >> 23;
  const uint64_t m24 = static_cast<uint64_t>((u & 0x7FFFFFu) | 0x800000u) << 24;
  const uint32_t sh = min(129u - ex, 63u);  // ex <= 127 for p <= 1 (p > 1 handled below)
  const uint64_t r = (m24 + (1ull << (sh - 1))) >> sh;
  return ex > 128u ? (m24 >> 24) << min(ex - 105u, 63u) : r;
}
__device__ __forceinline__ double from_fx(uint64_t v) { return static_cast<double>(v) * (1.0 / FX_ONE); }

// Work-group barrier that orders LDS only: waits for this wave's LDS
// operations (lgkmcnt) but not for its outstanding global loads (vmcnt), so
// loads issued before it stay in flight.  __syncthreads() would drain them.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// ------------------------------------------------------ reductions

template <typename T>
__device__ __forceinline__ T shfl_xor(T v, int m) { return __shfl_xor(v, m, WAVE); }
template <typename T>
__device__ __forceinline__ T shfl_up(T v, int d) { return __shfl_up(v, d, WAVE); }

struct OpAdd { template <typename T> __device__ T operator()(T a, T b) const { return a + b; } };
struct OpMin { template <typename T> __device__ T operator()(T a, T b) const { return b < a ? b : a; } };
struct OpMax { template <typename T> __device__ T operator()(T a, T b) const { return a < b ? b : a; } };

// Wave-level reduction / scan through rocPRIM's cross-lane (DPP) primitives;
// the combination order is fixed, so floating-point results are deterministic.
template <typename T, class Op>
__device__ __forceinline__ T wave_reduce(T v, Op op) {
  using WR = rocprim::warp_reduce<T, WAVE, true>;
  typename WR::storage_type st;
  T out;
  WR().reduce(v, out, st, op);
  return out;
}

template <typename T>
__device__ __forceinline__ T wave_incl_scan(T v) {
  using WS = rocprim::warp_scan<T, WAVE>;
  typename WS::storage_type st;
  T out;
  WS().inclusive_scan(v, out, st, OpAdd());
  return out;
}

// Integer inclusive scans on DPP alone (few temporaries): within each row of
// 16 lanes, adds of the value 1, 2, 4 and 8 lanes down (row_shr); then
// row_bcast:15 carries each row's total into the next row and row_bcast:31
// the first two rows' total into the last two.  A lane whose source is out of
// its row, or whose row is masked off, adds 0.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint32_t dpp_or_zero(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), CTRL, ROW_MASK, 0xF, false));
}
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ uint64_t dpp_or_zero64(uint64_t v) {
  const uint32_t lo = dpp_or_zero<CTRL, ROW_MASK>(static_cast<uint32_t>(v));
  const uint32_t hi = dpp_or_zero<CTRL, ROW_MASK>(static_cast<uint32_t>(v >> 32));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}
__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v) {
  v += dpp_or_zero<0x111, 0xF>(v);  // row_shr:1
  v += dpp_or_zero<0x112, 0xF>(v);  // row_shr:2
  v += dpp_or_zero<0x114, 0xF>(v);  // row_shr:4
  v += dpp_or_zero<0x118, 0xF>(v);  // row_shr:8
  v += dpp_or_zero<0x142, 0xA>(v);  // row_bcast:15 into rows 1, 3
  v += dpp_or_zero<0x143, 0xC>(v);  // row_bcast:31 into rows 2, 3
  return v;
}
__device__ __forceinline__ uint64_t wave_incl_scan(uint64_t v) {
  v += dpp_or_zero64<0x111, 0xF>(v);
  v += dpp_or_zero64<0x112, 0xF>(v);
  v += dpp_or_zero64<0x114, 0xF>(v);
  v += dpp_or_zero64<0x118, 0xF>(v);
  v += dpp_or_zero64<0x142, 0xA>(v);
  v += dpp_or_zero64<0x143, 0xC>(v);
  return v;
}

// Block-wide reduction in a fixed order (deterministic for floating point).
// `red` holds NW elements of T (NW = waves per work-group).  Two barriers.
template <typename T, class Op, int NW = NWAVE>
__device__ __forceinline__ T block_reduce(T v, Op op, T* red) {
  v = wave_reduce(v, op);
  if ((threadIdx.x & (WAVE - 1)) == 0) red[threadIdx.x / WAVE] = v;
  __syncthreads();
  T r = red[0];
#pragma unroll
  for (int i = 1; i < NW; ++i) r = op(r, red[i]);
  __syncthreads();
  return r;
}

// Block-wide exclusive prefix sum in thread order; *total receives the sum.
template <typename T, int NW = NWAVE>
__device__ __forceinline__ T block_excl_scan(T v, T* red, T* total) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int w = threadIdx.x / WAVE;
  const T inc = wave_incl_scan(v);
  T exc;
  if constexpr (__is_integral(T)) {
    exc = inc - v;
  } else {
    exc = shfl_up(inc, 1);
    if (lane == 0) exc = T(0);
  }
  if (lane == WAVE - 1) red[w] = inc;
  __syncthreads();
  T base = T(0), tot = T(0);
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const T x = red[i];
    if (i < w) base = base + x;
    tot = tot + x;
  }
  __syncthreads();
  *total = tot;
  return base + exc;
}

// Exclusive prefix sums of two quantities in thread order with one pair of
// barriers; ta / tb receive the totals.  TRAIL false leaves out the second
// barrier, for callers that pass a barrier of their own before ra / rb are
// written again.
template <int NW = NWAVE, bool TRAIL = true>
__device__ __forceinline__ void block_excl_scan2(uint32_t a, uint64_t b, uint32_t* ra, uint64_t* rb, uint32_t& ea,
                                                 uint64_t& eb, uint32_t& ta, uint64_t& tb) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int w = threadIdx.x / WAVE;
  const uint32_t ia = wave_incl_scan(a);
  const uint64_t ib = wave_incl_scan(b);
  const uint32_t xa = ia - a;
  const uint64_t xb = ib - b;
  if (lane == WAVE - 1) {
    ra[w] = ia;
    rb[w] = ib;
  }
  __syncthreads();
  uint32_t ba = 0, sa = 0;
  uint64_t bb = 0, sb = 0;
#pragma unroll
  for (int i = 0; i < NW; ++i) {
    const uint32_t x = ra[i];
    const uint64_t y = rb[i];
    if (i < w) {
      ba += x;
      bb += y;
    }
    sa += x;
    sb += y;
  }
  if constexpr (TRAIL) __syncthreads();
  ea = ba + xa;
  eb = bb + xb;
  ta = sa;
  tb = sb;
}

// Lane l's value of a 64-bit quantity (l wave-uniform).
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
  const uint32_t lo = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v)), l));
  const uint32_t hi = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(static_cast<uint32_t>(v >> 32)), l));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

// First index i in [a, b) with pred(i) true, for a predicate that is false
// then true along the range (b if it never holds).  The 64 lanes of a wave
// probe 64 evenly spaced indices per step, so a range of n needs about
// log64(n) + 1 steps; every wave computes the same result, without barriers.
template <class P>
__device__ __forceinline__ int wave_first(int a, int b, P&& pred) {
  const int lane = threadIdx.x & (WAVE - 1);
  for (;;) {
    const int s = max(1, (b - a + WAVE - 1) / WAVE);
    const int p = a + lane * s;
    const uint64_t m = __ballot(p < b && pred(p));
    if (s == 1) return m ? a + __ffsll(static_cast<unsigned long long>(m)) - 1 : b;
    if (m == 0) {
      a += min(WAVE - 1, (b - a - 1) / s) * s + 1;  // past the last probe inside [a, b)
    } else {
      const int f = __ffsll(static_cast<unsigned long long>(m)) - 1;
      if (f == 0) return a;
      b = a + f * s;
      a = a + (f - 1) * s + 1;
    }
  }
}

// Indices held by this thread for a slice partition of n items.
__device__ __forceinline__ void thread_slice(int n, int& lo, int& hi) {
  const int per = (n + NT - 1) / NT;
  lo = min(n, static_cast<int>(threadIdx.x) * per);
  hi = min(n, lo + per);
}

// Membership of `tok` in row b's stop set.
__device__ __forceinline__ bool is_stop(const int32_t* stop_ids, int64_t stop_ld, int64_t n_stop, int64_t b,
                                        int64_t tok) {
  if (stop_ids == nullptr || tok < 0) return false;
  const int32_t* s = stop_ids + b * stop_ld;
  for (int64_t i = 0; i < n_stop; ++i)
    if (s[i] >= 0 && s[i] == tok) return true;
  return false;
}

}  // namespace fl
