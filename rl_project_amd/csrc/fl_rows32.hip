// Fused per-row sampler for float32 logits on gfx950.
//
// One work-group of 1024 threads owns one row.  Float32 rows have too many
// distinct values to histogram exactly, so each decision of the reference
// sampler (src/forgeline/models/generation/sampling.py:26-61) is located in
// value bins and settled element by element among the members of the bins
// that hold a decision point.
//
// Two-read path (taken whenever it applies):
//   read 1   anchors 4095 bins of width 1/64 on A = the largest value among
//            the first 16384 elements (bin b holds values in about
//            (A + 24 - (b+1)/64, A + 24 - b/64]; the last bin takes everything
//            lower).  Each element adds one packed 64-bit word to its bin:
//            count << 45 | round(exp(y - ub_b) * 2^26), a term relative to the
//            bin's upper bound, so the row maximum is not needed yet.  After
//            the read, M = max y is known and every bin's mass becomes
//            exp(ub_b - M) * (its term sum) in 2^-45 fixed point.
//   plan     the bin of each decision point is bounded from the bin prefix
//            counts and masses alone (top-k by rank, min-p by the value where
//            exp(y - M) >= min_p starts, top-p and the inverse CDF by mass,
//            widened by the uncertainty of the cuts before them).
//   read 2   gathers the members of those bins into LDS, sorts them by
//            descending value then ascending index and settles each decision
//            exactly; mass prefixes inside a bin use the same terms as the bin
//            sums, so they meet the bin totals exactly.
// Rows outside this envelope (a value more than 24 above A, a decision in the
// last bin, more than CAP members to gather) take the multi-pass path below.
//
// Multi-pass path, by radix narrowing on an order-preserving 32-bit key of the
// filtered value y:
//
//   max      a pass over the row finds M = max y (the softmax shift) and
//            checks for NaN / +inf
//   bins     a pass builds 2048 bins on key bits 31..21; each bin holds its
//            element count and its mass sum(exp(y - M)) in 2^-45 fixed point,
//            so every partial sum is exact and order-independent
//   narrow   the decision point (the k-th value, the min-p boundary, the top-p
//            crossing, the inverse-CDF target) is located in one bin by a block
//            scan over the bins; a bin with more than CAP elements is split on
//            the next 11, then 10, key bits by another pass
//   exact    the elements of the final bin are gathered into LDS as
//            (key, index) pairs, sorted by descending value then ascending
//            index, and the decision is made element by element.
//
// Float32 decisions use exact arithmetic on the fixed-point masses:
//   top-k  keeps y >= the k-th largest value (ties kept)          (:36-38)
//   min-p  keeps exp(y - M) >= min_p, the reference's p < min_p * max p with
//          the common 1/S factor cancelled                          (:40-43)
//   top-p  removes sorted position j when the mass before it reaches
//          top_p times the mass of the survivors                    (:45-51)
//   select inverse CDF: the first member, in descending value / ascending
//          index order, whose inclusive mass exceeds u times the kept mass
//          (replaces torch.multinomial, :61); T <= 0 takes the first index of
//          the maximal value (argmax, :59-60).
// The reference evaluates the same predicates through float32 softmax and
// cumsum roundings; the two can differ only where a quantity lies within a few
// ulp of its threshold.
//
// Every pass reads the row again: the first from HBM, later ones mostly from
// L2 for rows of up to a few hundred KB.
#include <cfloat>
#include <climits>
#include <type_traits>

#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {

namespace {

constexpr int NB = 2048;                   // bins of the first two narrowing levels
constexpr int NB3 = 1024;                  // bins of the last level (one key each)
constexpr int CAP = 4096;                  // elements gathered and sorted in LDS
constexpr uint32_t KEY_POS_INF = 0xFF800000u;
constexpr uint32_t KEY_NEG_INF = 0x007FFFFFu;
constexpr uint32_t KEY_MIN_FINITE = 0x00800000u;  // smallest key of a value above -inf
constexpr int FXB = 45;                    // 2^-45 fixed point: 2^18 unit terms fit in 64 bits

// Two-read path
constexpr int NBF = 4096;                  // value bins; bin NBF-1 takes every lower value
constexpr float BPU = 64.0f;               // bins per unit of filtered value
constexpr float ANCHOR_UP = 24.0f;         // bin 0 starts this far above the anchor
constexpr int CNT_SH = 45;                 // bin word: count << 45 | sum of 2^-26 terms
constexpr uint64_t TERM_MASK = (1ull << CNT_SH) - 1u;
constexpr int NRANGE = 4;                  // bin ranges gathered by the second read
constexpr int RANK_SORT_MAX = 384;         // candidates sorted by rank counting; more by the bitonic network

// e in [0, 1] as fixed point round(e * 2^45) (halves rounded up).
__device__ __forceinline__ uint64_t fx45(float e) {
  const uint32_t u = __float_as_uint(e);
  const int ex = static_cast<int>(u >> 23);
  if (ex == 0) return 0;  // zero or denormal: below the resolution
  const uint64_t m = (u & 0x7FFFFFu) | 0x800000u;  // e = m * 2^(ex - 150)
  const int s = ex - 150 + FXB;
  if (s >= 0) return m << s;
  if (s < -24) return 0;
  return (m + (1ull << (-s - 1))) >> (-s);
}
__device__ __forceinline__ double from_fx45(uint64_t v) { return static_cast<double>(v) * (1.0 / 35184372088832.0); }

struct Shared32 {
  union {
    struct {
      uint32_t cnt1[NB];   // level-1 bins, kept for every decision
      uint64_t mass1[NB];
      uint32_t cnt[NB];    // deeper levels
      uint64_t mass[NB];
    };
    struct {
      uint64_t acc[NBF + 1];  // two-read bins: packed sums, then exclusive mass prefixes; [NBF]: discard slot
      uint32_t pc[NBF];    // exclusive count prefixes
    };
    alignas(16) uint32_t tkc[1 << 13];  // top-k path bins (key >> 19)
  };
  uint64_t cand[CAP];  // (key << 32) | ~index, sorted descending
  uint64_t cscan[CAP]; // two-read path: inclusive mass prefix at each candidate
  int32_t rlo[NRANGE], rhi[NRANGE], rbase[NRANGE];
  int32_t fplan[8];
  float xlo[2][NRANGE], xhi[2][NRANGE];
  uint32_t fkey[2];
  uint64_t fmass_out;
  uint64_t fck;
  int64_t ftok;
  uint64_t redq[NWAVE];
  uint32_t redu[NWAVE];
  int32_t redi[NWAVE];
  int32_t status;
  uint32_t ncand;
  int32_t pick_bin;
  uint32_t pick_n;
  uint64_t pick_m;
  int32_t result;
  uint32_t bcast_u;
  uint64_t bcast_q;
  uint32_t grp[4];  // next chunk group (wave_groups): two-read path reads 1, 2; top-k path reads 1, 2
};

// Element source: raw buffer loads of one row (range-checked, so loads past
// the row return zeros and need no clamping).
struct Src {
  __amdgpu_buffer_rsrc_t rs;
  int V;
  int nfull;  // chunks of 4 elements that lie wholly inside the row
  bool aligned;
  __device__ __forceinline__ float4 chunk(int c) const {
    if (aligned && c < nfull) {
      const uint4 u = buf_load16(rs, 16u * c, 0u);
      return make_float4(__uint_as_float(u.x), __uint_as_float(u.y), __uint_as_float(u.z), __uint_as_float(u.w));
    }
    float4 f;
    f.x = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 16 * c + 0, 0, 0));
    f.y = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 16 * c + 4, 0, 0));
    f.z = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 16 * c + 8, 0, 0));
    f.w = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, 16 * c + 12, 0, 0));
    return f;
  }
  // chunks c0 + u * NT + tid, u < U.  When all of them are whole chunks of an
  // aligned row (every iteration of a streaming loop but the last), one
  // uniform test covers them and each is one 16-byte load; a test per chunk
  // would put a branch around every load and make the wave wait for all U
  // loads before it uses the first.  A row of whole chunks (V a multiple of
  // 4) takes 16-byte loads throughout: a chunk past its end lies wholly
  // outside the buffer's range and reads zeros.
  template <int U>
  __device__ __forceinline__ void chunks(int c0, float4 (&q)[U]) const {
    const int tid = threadIdx.x;
    if (aligned && (c0 + U * NT <= nfull || 4 * nfull == V)) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint4 v = buf_load16(rs, 16u * static_cast<uint32_t>(c0 + u * NT + tid), 0u);
        q[u] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) q[u] = chunk(c0 + u * NT + tid);
    }
  }
  // The same for one wave: chunks base + u * WAVE + lane, u < U.
  template <int U>
  __device__ __forceinline__ void wchunks(int base, float4 (&q)[U]) const {
    const int lane = threadIdx.x & (WAVE - 1);
    if (aligned && (base + U * WAVE <= nfull || 4 * nfull == V)) {
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const uint4 v = buf_load16(rs, 16u * static_cast<uint32_t>(base + u * WAVE + lane), 0u);
        q[u] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
      }
    } else {
#pragma unroll
      for (int u = 0; u < U; ++u) q[u] = chunk(base + u * WAVE + lane);
    }
  }
};

// Chunk groups claimed wave by wave.  Group k holds chunks c_first +
// 4 WAVE g + u WAVE + lane (u < 4) of the calling wave's lanes, with g = k,
// or g = ng - 1 - k when last_first; a wave takes the next k from the LDS
// counter `next` (zero before the first claim) until none is left, and calls
// f(c, q) for each of its chunks (q: the chunk's 4 values, zeros past the
// row).  The SIMDs favour older waves, so with a fixed share per wave the
// youngest waves finish a read well after the oldest (16 us after them on
// rows of 262144 values); claimed groups let the favoured waves take more,
// and every wave ends within a group of the others.  For passes whose result
// does not depend on which wave takes which chunk (bin sums, candidate lists
// that are sorted afterwards).
template <class F>
__device__ __forceinline__ void wave_groups(const Src& S, uint32_t* next, int c_first, int ng, bool last_first,
                                            F&& f) {
  if (ng <= 0) return;  // (no claim: its LDS round trip would be the pass's only cost)
  const int lane = threadIdx.x & (WAVE - 1);
  auto claim = [&]() -> int {
    uint32_t k = 0;
    if (lane == 0) k = atomicAdd(next, 1u);
    return __builtin_amdgcn_readfirstlane(static_cast<int>(k));
  };
  int k = claim();
  while (k < ng) {
    const int base = c_first + 4 * WAVE * (last_first ? ng - 1 - k : k);
    float4 q[4];
    S.wchunks(base, q);
    const int kn = claim();  // (the next claim in flight with the loads)
#pragma unroll
    for (int u = 0; u < 4; ++u) f(base + u * WAVE + lane, q[u]);
    k = kn;
  }
}

// Logit -> filtered value: soft-cap, repetition penalty (history elements),
// temperature, each rounded to float32 as the reference's tensor ops round.
struct Xform {
  float cap, rp, t, rt;  // rt = recip_rt(t) when t > 0
  float rpr;             // recip_rt(rp)
  float rcap;            // RN(1 / cap) when cap > 0
  bool pen;
  const uint32_t* hbits;
  int nch;
  __device__ __forceinline__ float y(float x, bool hist) const {
    float z = x;
    if (cap > 0.0f) z = softcap_val<F32>(z, cap);
    if (hist) z = penalty_val<F32>(z, rp, rpr);
    // + 0.0f turns -0 into +0: the filters compare -0 == +0, so both get one key
    return temperature_val<F32>(z, t, rt) + 0.0f;
  }
  // y with the row's uniform choices fixed at compile time: TDIV = t > 0
  // (a division by the temperature), PEN = pen.  Equal to y() bit for bit.
  template <bool TDIV, bool PEN>
  __device__ __forceinline__ float yt(float x, bool hist) const {
    float z = x;
    if (cap > 0.0f) z = softcap_val<F32>(z, cap);
    if (PEN && hist) z = penalty_val<F32>(z, rp, rpr);
    if (TDIV) z = div_rt(z, t, rt);
    return z + 0.0f;
  }
  // yt of the four elements of a chunk (history bits hb), SC = cap > 0 fixed
  // at compile time (the soft-cap's tanh range test taken once for the
  // chunk).  With TDIV the range guard of div_rt is taken once for the
  // chunk: when every element passes it (the usual case) each quotient is
  // Markstein's two FMAs, else each element takes div_rt.  Equal to yt() bit
  // for bit.
  template <bool TDIV, bool PEN, bool SC>
  __device__ __forceinline__ void yt4(const float (&xs)[4], uint32_t hb, float (&y)[4]) const {
    float z[4] = {xs[0], xs[1], xs[2], xs[3]};
    if constexpr (SC) softcap4_f32(z, cap, rcap);
    if constexpr (!TDIV) {
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (PEN && ((hb >> e) & 1u)) z[e] = penalty_val<F32>(z[e], rp, rpr);
        y[e] = z[e] + 0.0f;
      }
      return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (PEN && ((hb >> e) & 1u)) z[e] = penalty_val<F32>(z[e], rp, rpr);
    if constexpr (TDIV) {
      float q0[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) q0[e] = z[e] * rt;
      // (NaN: fminf / fmaxf skip it and the FMAs return NaN, as the division does)
      const float zmin = fminf(fminf(fabsf(z[0]), fabsf(z[1])), fminf(fabsf(z[2]), fabsf(z[3])));
      const float qmin = fminf(fminf(fabsf(q0[0]), fabsf(q0[1])), fminf(fabsf(q0[2]), fabsf(q0[3])));
      const float qmax = fmaxf(fmaxf(fabsf(q0[0]), fabsf(q0[1])), fmaxf(fabsf(q0[2]), fabsf(q0[3])));
      if (zmin >= 0x1p-100f && qmin >= 0x1p-100f && qmax <= 0x1p100f) {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = __builtin_fmaf(__builtin_fmaf(-t, q0[e], z[e]), rt, q0[e]) + 0.0f;
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = div_rt(z[e], t, rt) + 0.0f;
      }
    }
  }
  // history bits of elements 4c .. 4c+3
  __device__ __forceinline__ uint32_t nibble(int c) const {
    return (pen && c < nch) ? (hbits[c >> 3] >> ((c & 7) * 4)) & 0xFu : 0u;
  }
};

// f(idx, y, valid) for every element of the row, read from memory: the first
// pass streams the row from HBM, later passes of a row of up to a few hundred
// KB mostly hit L2.  Called by all threads (block-uniform control flow).
template <class F>
__device__ __forceinline__ void row_pass(const Src& S, const Xform& X, F&& f, int from = 0) {
  const int tid = threadIdx.x;
  const int nch = X.nch;
  for (int c0 = from; c0 < nch; c0 += 4 * NT) {
    float4 q[4];
    S.chunks(c0, q);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int c = c0 + u * NT + tid;
      const uint32_t hb = X.nibble(c);
      const float xs[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int idx = 4 * c + e;
        f(idx, X.y(xs[e], (hb >> e) & 1u), idx < S.V);
      }
      // one chunk's elements at a time (interleaving all 16 costs VGPRs)
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// First key k in [a, b) with pred(k) true, for a predicate that is false then
// true along the range (b if it never holds); 64 probes per step, as
// wave_first, over the 32-bit key range.
template <class P>
__device__ __forceinline__ uint32_t wave_first_key(uint32_t a, uint32_t b, P&& pred) {
  const uint64_t lane = threadIdx.x & (WAVE - 1);
  uint64_t lo = a, hi = b;
  for (;;) {
    if (hi <= lo) return static_cast<uint32_t>(hi);
    const uint64_t n = hi - lo;
    const uint64_t s = n >= WAVE ? (n + WAVE - 1) / WAVE : 1u;
    const uint64_t p = lo + lane * s;
    const uint64_t m = __ballot(p < hi && pred(static_cast<uint32_t>(p)));
    if (s == 1) return m ? static_cast<uint32_t>(lo + __ffsll(static_cast<unsigned long long>(m)) - 1) : static_cast<uint32_t>(hi);
    if (m == 0) {
      lo += min<uint64_t>(WAVE - 1, (n - 1) / s) * s + 1;
    } else {
      const uint64_t f = __ffsll(static_cast<unsigned long long>(m)) - 1;
      if (f == 0) return static_cast<uint32_t>(lo);
      hi = lo + f * s;
      lo = lo + (f - 1) * s + 1;
    }
  }
}

// Wave-aggregated append of v to buf (one LDS atomic per wave).
__device__ __forceinline__ void wave_append(bool p, uint64_t v, uint32_t* counter, uint64_t* buf) {
  const uint64_t m = __ballot(p);
  if (m == 0) return;
  const uint32_t below =
      __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m >> 32), __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m), 0));
  const int leader = __ffsll(static_cast<unsigned long long>(m)) - 1;
  uint32_t base = 0;
  if ((threadIdx.x & (WAVE - 1)) == leader) base = atomicAdd(counter, static_cast<uint32_t>(__popcll(m)));
  base = __shfl(base, leader, WAVE);
  if (p && base + below < static_cast<uint32_t>(CAP)) buf[base + below] = v;
}

// Compare-exchange of one entry v (index idx) with the entry j positions
// away, held by lane ^ j (j <= 32), in the bitonic step (k, j): the lower
// index keeps the larger value where the k-block runs descending.
__device__ __forceinline__ uint64_t bitonic_lane_step(uint64_t v, int idx, int k, int j) {
  const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), j, WAVE);
  const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), j, WAVE);
  const uint64_t pv = (static_cast<uint64_t>(hi) << 32) | lo;
  const bool keep_max = ((idx & j) == 0) == ((idx & k) == 0);
  return keep_max ? (v > pv ? v : pv) : (v < pv ? v : pv);
}

// Steps (k, j) for j = jtop .. 1 (jtop <= 64) on one 128-entry block held in
// registers: lane l holds entries base + l (v0) and base + 64 + l (v1).
__device__ __forceinline__ void bitonic_block_steps(uint64_t& v0, uint64_t& v1, int base, int k, int jtop) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int i0 = base + lane, i1 = i0 + WAVE;
  for (int j = jtop; j > 0; j >>= 1) {
    if (j == WAVE) {  // the pair (base + l, base + 64 + l) lies in one lane
      const bool desc = (i0 & k) == 0;
      const uint64_t mx = v0 > v1 ? v0 : v1, mn = v0 > v1 ? v1 : v0;
      v0 = desc ? mx : mn;
      v1 = desc ? mn : mx;
    } else {
      v0 = bitonic_lane_step(v0, i0, k, j);
      v1 = bitonic_lane_step(v1, i1, k, j);
    }
  }
}

// Descending bitonic sort of buf[0, n) in LDS (n <= CAP); pads with zeros to
// a power of two P >= 128.  The steps of distance j <= 64 act within blocks
// of 128 entries: each wave loads a block into registers (two entries per
// lane), runs all such steps of one k there (lane exchanges by shuffles),
// and stores it back -- one LDS round trip where the network would take one
// per step.  Blocks of k <= 128 are sorted whole in one such pass.  Steps of
// distance >= 128 go through LDS, one pair per thread, between block
// barriers.
__device__ void bitonic_desc(uint64_t* buf, int n) {
  int P = 128;
  while (P < n) P <<= 1;
  for (int i = n + threadIdx.x; i < P; i += NT) buf[i] = 0;
  __syncthreads();
  const int lane = threadIdx.x & (WAVE - 1);
  const int wave = threadIdx.x / WAVE;
  const int nblk = P / (2 * WAVE);
  // blocks sorted whole: k = 2 .. 128
  for (int blk = wave; blk < nblk; blk += NWAVE) {
    const int base = blk * 2 * WAVE;
    uint64_t v0 = buf[base + lane], v1 = buf[base + WAVE + lane];
    for (int k = 2; k <= 2 * WAVE; k <<= 1) bitonic_block_steps(v0, v1, base, k, k >> 1);
    buf[base + lane] = v0;
    buf[base + WAVE + lane] = v1;
  }
  for (int k = 4 * WAVE; k <= P; k <<= 1) {
    for (int j = k >> 1; j > WAVE; j >>= 1) {
      __syncthreads();
      for (int i = threadIdx.x; i < (P >> 1); i += NT) {
        const int a = ((i & ~(j - 1)) << 1) | (i & (j - 1));  // 2 j (i / j) + i % j (j a power of 2)
        const int c = a + j;
        const uint64_t x = buf[a], y = buf[c];
        const bool desc = (a & k) == 0;
        if (desc ? (x < y) : (x > y)) {
          buf[a] = y;
          buf[c] = x;
        }
      }
    }
    __syncthreads();
    for (int blk = wave; blk < nblk; blk += NWAVE) {
      const int base = blk * 2 * WAVE;
      uint64_t v0 = buf[base + lane], v1 = buf[base + WAVE + lane];
      bitonic_block_steps(v0, v1, base, k, WAVE);
      buf[base + lane] = v0;
      buf[base + WAVE + lane] = v1;
    }
  }
  __syncthreads();
}

// Descending order of buf[0, n), n <= RANK_SORT_MAX, whose nonzero entries
// are distinct (zeros sort last): each entry goes to its rank, the number of
// entries greater than it, counted over broadcast LDS reads -- independent
// loads, where a bitonic network for a few hundred entries is a chain of
// dependent LDS round trips.  Every wave counts: the waves holding an entry
// each take one slice of the others (rank: n counters, tmp: n entries of
// scratch).  Entries of rank >= the nonzero count are left unspecified.
__device__ void rank_sort_desc(uint64_t* buf, uint64_t* tmp, uint32_t* rank, int n) {
  const int t = threadIdx.x;
  if (t < n) rank[t] = 0;
  __syncthreads();
  const int nw = (n + WAVE - 1) / WAVE;  // waves' worth of entries
  const int w = t / WAVE;
  if (nw > 0 && w < (NWAVE / nw) * nw) {
    const int i = (w % nw) * WAVE + (t & (WAVE - 1));
    const int np = NWAVE / nw, p = w / nw;
    const int j0 = (n * p) / np, j1 = (n * (p + 1)) / np;
    const uint64_t mine = i < n ? buf[i] : ~0ull;
    uint32_t r = 0;
    int j = j0;
    for (; j + 4 <= j1; j += 4) {
      const uint64_t a0 = buf[j], a1 = buf[j + 1], a2 = buf[j + 2], a3 = buf[j + 3];
      r += (a0 > mine ? 1u : 0u) + (a1 > mine ? 1u : 0u) + (a2 > mine ? 1u : 0u) + (a3 > mine ? 1u : 0u);
    }
    for (; j < j1; ++j) r += buf[j] > mine ? 1u : 0u;
    if (i < n && r) atomicAdd(&rank[i], r);
  }
  __syncthreads();
  if (t < n && buf[t] != 0ull) tmp[rank[t]] = buf[t];
  __syncthreads();
  if (t < n) buf[t] = tmp[t];
  __syncthreads();
}

enum Crit { CRIT_COUNT = 0, CRIT_PRED = 1, CRIT_MASS = 2 };

// The bin holding a decision point, scanning bins in descending key order
// with exact running totals.  Bins lying wholly below key `tau` are skipped
// (their elements are already removed) except by CRIT_COUNT.
//   CRIT_COUNT: first bin whose inclusive count exceeds `rank`
//   CRIT_PRED : first bin whose smallest possible value fails exp(y - M) >= mp
//   CRIT_MASS : first bin whose inclusive mass reaches `thr`
struct Pick {
  int bin;        // -1 when no bin qualifies
  uint32_t n_ex;  // elements before the bin (whole row order)
  uint64_t m_ex;  // their mass
};

__device__ Pick choose_bin(Shared32& sh, const uint32_t* cnt, const uint64_t* mass, int nbins, uint32_t klo, int shift,
                           uint32_t n_ab, uint64_t m_ab, int crit, uint32_t rank, float mp, float M, uint64_t thr,
                           uint32_t tau) {
  const int per = (nbins + NT - 1) / NT;
  const int p0 = threadIdx.x * per;
  uint32_t ln = 0;
  uint64_t lm = 0;
  for (int k = 0; k < per; ++k) {
    const int pos = p0 + k;
    if (pos < nbins) {
      ln += cnt[nbins - 1 - pos];
      lm += mass[nbins - 1 - pos];
    }
  }
  uint32_t tn;
  uint64_t tm;
  const uint32_t en = block_excl_scan<uint32_t>(ln, sh.redu, &tn);
  const uint64_t em = block_excl_scan<uint64_t>(lm, sh.redq, &tm);
  uint32_t cn = n_ab + en;
  uint64_t cm = m_ab + em;
  int first = INT_MAX;
  uint32_t fn = 0;
  uint64_t fm = 0;
  for (int k = 0; k < per; ++k) {
    const int pos = p0 + k;
    if (pos >= nbins) break;
    const int bin = nbins - 1 - pos;
    const uint32_t c = cnt[bin];
    const uint64_t m = mass[bin];
    if (c > 0 && first == INT_MAX) {
      const uint32_t lo = klo + (static_cast<uint32_t>(bin) << shift);
      const uint32_t hi = lo + ((1u << shift) - 1u);
      bool hit;
      if (crit == CRIT_COUNT) hit = cn + c > rank;
      else if (crit == CRIT_PRED) hit = hi >= tau && !(expf(f32_of_key(lo) - M) >= mp);
      else hit = hi >= tau && cm + m >= thr;
      if (hit) {
        first = pos;
        fn = cn;
        fm = cm;
      }
    }
    cn += c;
    cm += m;
  }
  const int w = block_reduce<int32_t>(first, OpMin(), sh.redi);
  if (w == INT_MAX) return {-1, 0, 0};
  if (first == w) {
    sh.pick_bin = nbins - 1 - w;
    sh.pick_n = fn;
    sh.pick_m = fm;
  }
  __syncthreads();
  Pick p = {sh.pick_bin, sh.pick_n, sh.pick_m};
  __syncthreads();
  return p;
}

// Outcome of a narrowing
enum Outcome {
  OUT_NONE = 0,     // no bin qualifies: the decision point lies past the row
  OUT_CAND = 1,     // candidates sorted in sh.cand[0, n)
  OUT_VALUE = 2,    // a single key with more than CAP elements
  OUT_ALLKEPT = 3,  // the qualifying range splits into bins none of which qualifies
};
struct Narrow {
  int out;
  uint32_t klo, khi;  // key range
  uint32_t n_ab;      // elements before the range (whole-row order)
  uint64_t m_ab;      // their mass
  uint32_t count;     // elements in the range
  uint64_t rmass;     // their mass
  int n;              // candidates gathered (OUT_CAND)
};

// ------------------------------------------------------------ two-read path
struct OpOr { template <typename T> __device__ T operator()(T a, T b) const { return a | b; } };

// Bin of a value y <= c (c = anchor + ANCHOR_UP): floor((c - y) * 64), the
// last bin for everything lower (-inf included); values above c give 0 or -1.
// Non-increasing in y, so the bins cut the value order into contiguous ranges.
__device__ __forceinline__ int fbin(float y, float c) {
  return static_cast<int>(fminf(fmaxf((c - y) * BPU, -1.0f), static_cast<float>(NBF - 1)));
}
// Upper bound of bin b's values (up to rounding).
__device__ __forceinline__ float fub(int b, float c) { return c - static_cast<float>(b) * (1.0f / BPU); }
// exp(y - ub_b) * 2^26, truncated to an integer, for y in bin b.  With
// u = (c - y) * 64, whose integer part is b (fbin), y - ub_b = -fract(u) / 64
// lies in (-1/64, 0]; the degree-3 Taylor polynomial of exp(-f / 64) in
// f = fract(u) is within 2.5e-9 of it there, 0.17 units of 2^-26 where the
// float result's own unit is 4 of them (one v_fract_f32 and three FMAs per
// value; rebuilding the bound from b took four more), and 2^18 terms of at
// most 2^26 fit the bin word's 45-bit field.
// Terms of the last bin are summed like the others (a value there is finite
// or -inf, whose fraction is NaN and converts to 0) and dropped by fmass.
// (The coefficients carry the factor 2^26: scaling by a power of two commutes
// with each rounding of the Horner chain, so this is t * 2^26 exactly.)
__device__ __forceinline__ uint32_t fterm(float y, float c) {
  const float f = __builtin_amdgcn_fractf((c - y) * BPU);
  const float t26 = fmaf(f, fmaf(f, fmaf(f, -67108864.0f / 1572864.0f, 67108864.0f / 8192.0f), -67108864.0f / 64.0f),
                         67108864.0f);
  return static_cast<uint32_t>(t26);
}
// Mass in 2^-45 fixed point relative to M of term sum F (2^-26 units) in bin b:
// round(F * exp(ub_b - M) * 2^19).  Bin totals and in-bin prefixes both use it,
// so the prefixes of a bin end exactly at its total.  The last bin adds no
// mass: its values lie more than 40 below the anchor, so their weights are
// below e^-40 of the largest.
__device__ __forceinline__ uint64_t fmass(uint64_t F, int b, float c, float M) {
  if (F == 0 || b == NBF - 1) return 0;
  const double g = exp(static_cast<double>(fub(b, c)) - static_cast<double>(M)) * 524288.0;
  return static_cast<uint64_t>(static_cast<double>(F) * g + 0.5);
}

struct RowCfg {
  int V, K;
  float T, TP, MP, U;
  bool select;
};
struct RowOut {
  uint32_t kmax;
  int32_t status;
  uint32_t tau;
  uint64_t CK;
  uint64_t keep_mass;
  uint32_t keep_n;
  int64_t tok;
};

// ------------------------------------------------------------ top-k path
// Rows with top-k on, up to TK_MAX (a request's default keeps 50,
// inference/requests.py:26): every decision of sampling.py:36-61 acts on
// the top-k survivors, which a histogram finds without the filtered values of
// the whole row.  The value
// y = RN(z / t) + 0 (sampling.py:33-34) is a non-decreasing function f of the
// penalised value z (sampling.py:30), so the K-th largest y is f of the K-th
// largest z, and only candidates need y:
//   read 1   s = soft-cap(x) (x without soft-cap) adds one to a TK_NB-bin
//            histogram on bits 31..TK_SH of its order-preserving key (16 bins
//            per binade); the row's first 4 * TK_TILE * NT keys stay in
//            registers
//   history  each element of the history bitmap moves from the bin of s to
//            the bin of z = penalty(s)
//   scan     the bin of the K-th largest z (a descending block scan)
//   read 2   every element in that bin or above becomes a candidate
//            (key(z) << 32 | ~index, then key(y)); more than TK_CAND of them,
//            a K-th value at -inf, or one that rounding could tie with a
//            value below the bin, leave the row to the two-read path, as do
//            NaN values
//   decide   one wave over the sorted candidates at or above the K-th value,
//            64 at a time: min-p, top-p and the inverse CDF on exact 2^-45
//            masses fx45(exp(y - M)) -- the multi-pass path's arithmetic,
//            element by element.
constexpr int TK_CAND = RANK_SORT_MAX;  // candidates it sorts and decides
constexpr int TK_MAX = TK_CAND;         // top-k values it serves (a row has at least K candidates)
constexpr int TK_TILE = 8;              // chunks per thread whose keys read 1 keeps in registers
constexpr int TK_SH = 19;               // bin of a key: key >> TK_SH
constexpr int TK_NB = 1 << (32 - TK_SH);
constexpr int TK_BPT = TK_NB / NT;      // bins per thread in the scan
static_assert(TK_CAND <= NT && TK_BPT * NT == TK_NB && TK_BPT % 4 == 0, "top-k shapes");
static_assert(sizeof(Shared32::tkc) == TK_NB * 4 && TK_NB * 4 <= NB * 24,
              "the top-k bins share the level-1 and level-2 bins' memory");

// s: the soft-capped logit, the logit itself without soft-cap
template <bool SC>
__device__ __forceinline__ float topk_s(const Xform& X, float x) {
  return SC ? softcap_val<F32>(x, X.cap) : x;
}
// y of a penalised value z, as Xform::yt computes it
template <bool TDIV>
__device__ __forceinline__ float topk_y(const Xform& X, float z) {
  return (TDIV ? div_rt(z, X.t, X.rt) : z) + 0.0f;
}

// Read 1 of four values (chunk ch): bin counts of their s keys, the keys in k
// (0 past the row's end), bad set on a NaN (or +inf and -inf together).
// Returns the largest key.
template <bool SC>
__device__ __forceinline__ uint32_t topk_count4(Shared32& sh, const Xform& X, int V, int ch, const float4& q,
                                                uint32_t (&k)[4], bool& bad) {
  const float s[4] = {topk_s<SC>(X, q.x), topk_s<SC>(X, q.y), topk_s<SC>(X, q.z), topk_s<SC>(X, q.w)};
  const float sm = (s[0] + s[1]) + (s[2] + s[3]);
  if (4 * ch + 3 < V) {
    bad |= sm != sm;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      k[e] = f32_key(s[e]);
      atomicAdd(&sh.tkc[k[e] >> TK_SH], 1u);
    }
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      k[e] = 0u;
      if (4 * ch + e >= V) continue;
      bad |= s[e] != s[e];
      k[e] = f32_key(s[e]);
      atomicAdd(&sh.tkc[k[e] >> TK_SH], 1u);
    }
  }
  return max(max(k[0], k[1]), max(k[2], k[3]));
}

// The register tile: chunk u * NT + tid for u < TK_TILE (one memory round
// trip for rows up to 4 * TK_TILE * NT values).  Chunks U0 .. U1 - 1; a chunk
// past the row reads 0 (the buffer's bound).  The first TK_EARLY go out before
// the row's history is read, the rest after its barriers: a wave waits at a
// barrier until the memory pipeline has taken every load it issued before
// it (16 waves of 8 16-byte loads take ~0.85 us per CU).
#ifndef FL_TK_EARLY
#define FL_TK_EARLY 4
#endif
constexpr int TK_EARLY = FL_TK_EARLY;
template <int U0, int U1>
__device__ __forceinline__ void topk_tile_load(const Src& S, float4 (&q)[TK_TILE]) {
  const int tid = threadIdx.x;
  if (S.aligned && (U1 * NT <= S.nfull || 4 * S.nfull == S.V)) {
#pragma unroll
    for (int u = U0; u < U1; ++u) {
      const uint4 v = buf_load16(S.rs, 16u * static_cast<uint32_t>(u * NT + tid), 0u);
      q[u] = make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
    }
  } else {
#pragma unroll
    for (int u = U0; u < U1; ++u) q[u] = S.chunk(u * NT + tid);
  }
}

// Read 1: the register tile q (keys kept in kt, the largest of chunk u in
// cmx[u]), then the rest of the row.
template <bool SC>
__device__ __forceinline__ void topk_read1(Shared32& sh, const Src& S, const Xform& X, int V,
                                           const float4 (&q)[TK_TILE], uint32_t (&kt)[TK_TILE][4],
                                           uint32_t (&cmx)[TK_TILE], bool& bad) {
  const int tid = threadIdx.x;
#pragma unroll
  for (int u = 0; u < TK_TILE; ++u) {
    cmx[u] = topk_count4<SC>(sh, X, V, u * NT + tid, q[u], kt[u], bad);
    __builtin_amdgcn_sched_barrier(0);
  }
  // (past the tile: chunk groups claimed wave by wave, as in the two-read path)
  const int ng = X.nch > TK_TILE * NT ? (X.nch - TK_TILE * NT + 4 * WAVE - 1) / (4 * WAVE) : 0;
  wave_groups(S, &sh.grp[2], TK_TILE * NT, ng, false, [&](int ch, const float4& q) __attribute__((always_inline)) {
    uint32_t k[4];
    topk_count4<SC>(sh, X, V, ch, q, k, bad);
  });
}

// History elements (bits of the bitmap X.hbits; thread t takes words t,
// t + NT, ...).  The first TK_HP of a thread are prefetched before read 1 and
// kept in registers (index hi, logit hx, then z key hk); the rest, rare, are
// loaded again by each pass that needs them.
constexpr int TK_HP = 4;
struct TopkHist {
  int hi[TK_HP];
  float hx[TK_HP];
  uint32_t hk[TK_HP];
  bool more;  // the thread's words hold more than TK_HP elements
};

__device__ __forceinline__ void topk_hist_prefetch(const Src& S, const Xform& X, int V, TopkHist& h) {
#pragma unroll
  for (int j = 0; j < TK_HP; ++j) h.hi[j] = -1;
  h.more = false;
  const int nw = (V + 31) >> 5;
  int n = 0;
  for (int w = threadIdx.x; w < nw && !h.more; w += NT) {
    uint32_t bits = X.hbits[w];
    while (bits) {
      if (n == TK_HP) {
        h.more = true;
        break;
      }
      const int i = 32 * w + __ffs(bits) - 1;
      bits &= bits - 1u;
#pragma unroll
      for (int j = 0; j < TK_HP; ++j)
        if (j == n) h.hi[j] = i;  // (static indices: the slots stay in registers)
      ++n;
    }
  }
#pragma unroll
  for (int j = 0; j < TK_HP; ++j)
    h.hx[j] = h.hi[j] >= 0 ? __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(S.rs, 4 * h.hi[j], 0, 0)) : 0.0f;
}

// The history elements past a thread's first TK_HP: f(i, x) for each.
template <class F>
__device__ __forceinline__ void topk_hist_rest(const Src& S, const Xform& X, int V, F&& f) {
  const int nw = (V + 31) >> 5;
  int n = 0;
  for (int w = threadIdx.x; w < nw; w += NT) {
    uint32_t bits = X.hbits[w];
    while (bits) {
      const int i = 32 * w + __ffs(bits) - 1;
      bits &= bits - 1u;
      if (n++ < TK_HP) continue;
      f(i, __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(S.rs, 4 * i, 0, 0)));
    }
  }
}

// Each history element moves from the bin of s to the bin of z = penalty(s)
// (bad set on a NaN z); the z keys of the prefetched ones stay in h.hk.
template <bool SC>
__device__ __forceinline__ void topk_hist_move(Shared32& sh, const Src& S, const Xform& X, int V, TopkHist& h,
                                               bool& bad) {
  auto move = [&](float x) -> uint32_t {
    const float s = topk_s<SC>(X, x);
    const float z = penalty_val<F32>(s, X.rp, X.rpr);
    bad |= z != z;
    const uint32_t ks = f32_key(s), kz = f32_key(z);
    if ((ks >> TK_SH) != (kz >> TK_SH)) {
      atomicSub(&sh.tkc[ks >> TK_SH], 1u);
      atomicAdd(&sh.tkc[kz >> TK_SH], 1u);
    }
    return kz;
  };
#pragma unroll
  for (int j = 0; j < TK_HP; ++j) h.hk[j] = h.hi[j] >= 0 ? move(h.hx[j]) : 0u;
  if (h.more) topk_hist_rest(S, X, V, [&](int, float x) { move(x); });
}

// One slot per candidate: (z key << 32) | ~index, z keys turned into y keys
// before the sort.  A wave's candidates take one atomic: lane l writes its c
// candidates from the wave's base plus the candidates of lanes below l.
__device__ __forceinline__ uint32_t topk_slots(Shared32& sh, uint32_t c) {
  const uint32_t incl = wave_incl_scan(c);
  const uint32_t tot = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(incl), WAVE - 1));
  uint32_t base = 0;
  if (tot) {
    if ((threadIdx.x & (WAVE - 1)) == WAVE - 1) base = atomicAdd(&sh.ncand, tot);
    base = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(base), WAVE - 1));
  }
  return base + incl - c;
}
__device__ __forceinline__ void topk_put(Shared32& sh, uint32_t& pos, uint32_t kz, int i) {
  if (pos < static_cast<uint32_t>(CAP))
    sh.cand[pos] = (static_cast<uint64_t>(kz) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(i));
  ++pos;
}

// Read 2: the elements in bin kbin or above (kbin > 0: the zero keys past the
// row stay out), history elements taken from their own list.
template <bool SC>
__device__ __forceinline__ void topk_read2(Shared32& sh, const Src& S, const Xform& X, int V,
                                           const uint32_t (&kt)[TK_TILE][4], const uint32_t (&cmx)[TK_TILE],
                                           const TopkHist& h, uint32_t kbin) {
  const int tid = threadIdx.x;
  {
    // the tile: bit 4u + e of m for chunk u, element e (chunks without a
    // candidate in the whole wave skipped)
    uint32_t m = 0;
#pragma unroll
    for (int u = 0; u < TK_TILE; ++u) {
      if (__ballot((cmx[u] >> TK_SH) >= kbin)) {
        uint32_t mu = 0;
#pragma unroll
        for (int e = 0; e < 4; ++e) mu |= ((kt[u][e] >> TK_SH) >= kbin ? 1u : 0u) << e;
        if (mu) mu &= ~X.nibble(u * NT + tid);
        m |= mu << (4 * u);
      }
    }
    uint32_t pos = topk_slots(sh, static_cast<uint32_t>(__popc(m)));
#pragma unroll
    for (int u = 0; u < TK_TILE; ++u) {
      if ((m >> (4 * u)) & 0xFu) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((m >> (4 * u + e)) & 1u) topk_put(sh, pos, kt[u][e], 4 * (u * NT + tid) + e);
      }
    }
  }
  // (past the tile: claimed chunk groups, the row's last chunks first)
  const int ng = X.nch > TK_TILE * NT ? (X.nch - TK_TILE * NT + 4 * WAVE - 1) / (4 * WAVE) : 0;
  wave_groups(S, &sh.grp[3], TK_TILE * NT, ng, true, [&](int ch, const float4& q) __attribute__((always_inline)) {
      const float xs[4] = {q.x, q.y, q.z, q.w};
      uint32_t k[4], m = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        k[e] = f32_key(topk_s<SC>(X, xs[e]));
        m |= (4 * ch + e < V && (k[e] >> TK_SH) >= kbin ? 1u : 0u) << e;
      }
      if (m) m &= ~X.nibble(ch);
      if (__ballot(m != 0u)) {
        uint32_t pos = topk_slots(sh, static_cast<uint32_t>(__popc(m)));
#pragma unroll
        for (int e = 0; e < 4; ++e)
          if ((m >> e) & 1u) topk_put(sh, pos, k[e], 4 * ch + e);
      }
  });
  if (X.pen) {
    uint32_t m = 0;
#pragma unroll
    for (int j = 0; j < TK_HP; ++j) m |= (h.hi[j] >= 0 && (h.hk[j] >> TK_SH) >= kbin ? 1u : 0u) << j;
    if (__ballot(m != 0u)) {
      uint32_t pos = topk_slots(sh, static_cast<uint32_t>(__popc(m)));
#pragma unroll
      for (int j = 0; j < TK_HP; ++j)
        if ((m >> j) & 1u) topk_put(sh, pos, h.hk[j], h.hi[j]);
    }
    if (h.more)
      topk_hist_rest(S, X, V, [&](int i, float x) {
        const uint32_t kz = f32_key(penalty_val<F32>(topk_s<SC>(X, x), X.rp, X.rpr));
        if ((kz >> TK_SH) >= kbin) {
          uint32_t pos = atomicAdd(&sh.ncand, 1u);
          topk_put(sh, pos, kz, i);
        }
      });
  }
}

// The bins, zeroed (and the candidate count) before the first barrier of a
// top-k row.
__device__ __forceinline__ void topk_init(Shared32& sh) {
  uint4* z4 = reinterpret_cast<uint4*>(sh.tkc);
  for (int i = threadIdx.x; i < TK_NB / 4; i += NT) z4[i] = make_uint4(0u, 0u, 0u, 0u);
  if (threadIdx.x == 0) {
    sh.ncand = 0;
    sh.pick_bin = -1;
  }
}

// The top-k path, after topk_init, the tile's first TK_EARLY chunks and the
// history barriers.
// Returns false, with nothing decided, when the row needs another path.
// Called by all threads (block-uniform control flow).
__device__ __forceinline__ bool topk_path(Shared32& sh, const Src& S, const Xform& X, const RowCfg& R, RowOut& o,
                                          float4 (&q)[TK_TILE]) {
  const int tid = threadIdx.x;
  const int lane = tid & (WAVE - 1);
  const int V = R.V, K = R.K;
  if constexpr (TK_EARLY < TK_TILE) topk_tile_load<TK_EARLY, TK_TILE>(S, q);
  if (sh.status != 0) return false;  // (rows with an error status: the two-read path reports them)
  const bool sc = X.cap > 0.0f, tdiv = X.t > 0.0f;
  TopkHist h;
  if (X.pen) topk_hist_prefetch(S, X, V, h);
  FL_MARK(16);
  uint32_t kt[TK_TILE][4], cmx[TK_TILE];
  bool bad = false;
  if (sc) topk_read1<true>(sh, S, X, V, q, kt, cmx, bad);
  else topk_read1<false>(sh, S, X, V, q, kt, cmx, bad);
  FL_MARK(1);
  // (no barrier before the moves: they commute with read 1's adds, since the
  // bin counters add modulo 2^32 and a count taken below zero is repaid by
  // the adds still to come; nothing reads the bins before the barrier below)
  if (X.pen) {
    FL_MARK(10);
    if (sc) topk_hist_move<true>(sh, S, X, V, h, bad);
    else topk_hist_move<false>(sh, S, X, V, h, bad);
  }
  FL_MARK(13);
  __syncthreads();  // (every add and move before the scan reads the bins)
  FL_MARK(11);

  // ---------------------------------------------- bin of the K-th largest value
  // (thread t takes bins TK_NB - 1 - TK_BPT t down to TK_NB - TK_BPT (t + 1):
  // the scan runs down the values)
  {
    const int b0 = TK_NB - TK_BPT * (tid + 1);
    uint32_t c[TK_BPT];
#pragma unroll
    for (int q = 0; q < TK_BPT / 4; ++q) {
      const uint4 v = reinterpret_cast<const uint4*>(sh.tkc + b0)[q];
      c[4 * q] = v.x;
      c[4 * q + 1] = v.y;
      c[4 * q + 2] = v.z;
      c[4 * q + 3] = v.w;
    }
    uint32_t sum = 0;
#pragma unroll
    for (int q = 0; q < TK_BPT; ++q) sum += c[q];
    // (the scan also counts the threads that saw a NaN, in bits 20 and up:
    // a row holds at most 2^18 values and a block 1024 threads)
    uint32_t tot;
    const uint32_t ex = block_excl_scan<uint32_t>(sum | (bad ? 1u << 20 : 0u), sh.redu, &tot) & 0xFFFFFu;
    // (with a NaN no bin is picked: pick_bin stays -1 and the two-read path
    // reports the row)
    const uint32_t k = static_cast<uint32_t>(K);
    if ((tot >> 20) == 0u && ex < k && ex + sum >= k) {
      uint32_t run = ex;
      bool done = false;
#pragma unroll
      for (int q = TK_BPT - 1; q >= 0; --q) {
        if (!done && run + c[q] >= k) {
          sh.pick_bin = b0 + q;
          sh.pick_n = run + c[q];  // members of that bin and above
          done = true;
        }
        run += c[q];
      }
    }
  }
  __syncthreads();
  const int kbin = sh.pick_bin;
  const uint32_t nc = sh.pick_n;
  // (a K-th value at -inf keeps every finite value: not a few candidates)
  if (kbin <= static_cast<int>(KEY_NEG_INF >> TK_SH) || nc > static_cast<uint32_t>(TK_CAND)) return false;
  FL_MARK(2);

  // ---------------------------------------------- read 2: the candidates
  if (sc) topk_read2<true>(sh, S, X, V, kt, cmx, h, static_cast<uint32_t>(kbin));
  else topk_read2<false>(sh, S, X, V, kt, cmx, h, static_cast<uint32_t>(kbin));
  __syncthreads();
  const int n = static_cast<int>(sh.ncand);
  if (n != static_cast<int>(nc)) return false;  // (cannot happen: the reads compute the same values)
  // z keys -> y keys (y = f(z), f non-decreasing: the order of the candidates stays)
  if (tid < n) {
    const uint64_t c = sh.cand[tid];
    const float z = f32_of_key(static_cast<uint32_t>(c >> 32));
    const float y = tdiv ? topk_y<true>(X, z) : topk_y<false>(X, z);
    sh.cand[tid] = (static_cast<uint64_t>(f32_key(y)) << 32) | static_cast<uint32_t>(c);
  }
  FL_MARK(3);
  rank_sort_desc(sh.cand, sh.cscan, reinterpret_cast<uint32_t*>(sh.cscan + RANK_SORT_MAX), n);
  FL_MARK(4);
  // The K-th largest y and the largest: a K-th value at -inf, or one that an
  // element below the bin could round to (f of the largest z below the bin
  // equals it), leaves the row to the two-read path; a maximum at +inf is the
  // row's status.
  const uint32_t kmx = static_cast<uint32_t>(sh.cand[0] >> 32);
  const uint32_t tau = static_cast<uint32_t>(sh.cand[K - 1] >> 32);  // the K-th largest value; ties stay
  if (kmx < KEY_POS_INF) {
    const float zb = f32_of_key((static_cast<uint32_t>(kbin) << TK_SH) - 1u);
    const uint32_t kb = f32_key(tdiv ? topk_y<true>(X, zb) : topk_y<false>(X, zb));
    if (tau <= KEY_NEG_INF || kb >= tau) return false;
  }
  o.kmax = kmx;
  o.status = kmx >= KEY_POS_INF ? FL_ROW_INF : 0;
  o.tau = KEY_MIN_FINITE;
  o.CK = static_cast<uint64_t>(KEY_MIN_FINITE) << 32;
  o.keep_mass = 0;
  o.keep_n = 0;
  o.tok = -1;
  if (o.status != 0) return true;

  // ---------------------------------------------- decisions (wave 0)
  // Kept by top-k: the nt candidates at or above tau, a prefix of the sorted
  // ones; min-p keeps a prefix of those (exp(y - M) falls along the order).
  // sh.cscan[i]: the inclusive mass prefix at sorted position i.
  if (tid < WAVE) {
    const float M = f32_of_key(kmx);
    const bool mp_on = R.MP > 0.0f, tp_on = R.TP > 0.0f && R.TP < 1.0f;
    int nt = K;
    while (nt < n && static_cast<uint32_t>(sh.cand[nt] >> 32) >= tau) ++nt;  // (ties with the K-th value)
    uint32_t keep_n = 0;
    uint64_t keep_mass = 0;
    for (int r0 = 0; r0 < nt; r0 += WAVE) {
      const int i = r0 + lane;
      const bool valid = i < nt;
      const float e = valid ? expf(f32_of_key(static_cast<uint32_t>(sh.cand[i] >> 32)) - M) : 0.0f;
      const bool kept = valid && (!mp_on || e >= R.MP);  // (sampling.py:40-43 with the common 1/S cancelled)
      const uint64_t f = kept ? fx45(e) : 0ull;
      const uint64_t incl = keep_mass + wave_incl_scan(f);
      if (valid) sh.cscan[i] = incl;
      keep_n += static_cast<uint32_t>(__popcll(__ballot(kept)));
      keep_mass = readlane64(incl, WAVE - 1);
    }
    __builtin_amdgcn_wave_barrier();  // (the prefixes above before the reads below)
    // (the first sorted position i < keep_n where pred(i) holds, or -1)
    auto first = [&](auto pred) -> int {
      for (int r0 = 0; r0 < static_cast<int>(keep_n); r0 += WAVE) {
        const int i = r0 + lane;
        const uint64_t m = __ballot(i < static_cast<int>(keep_n) && pred(i));
        if (m) return r0 + __ffsll(static_cast<unsigned long long>(m)) - 1;
      }
      return -1;
    };
    bool cut = false;
    if (tp_on && keep_n > 0) {
      // first kept position whose exclusive mass reaches ceil(top_p * kept mass)
      const uint64_t thr = static_cast<uint64_t>(ceil(static_cast<double>(R.TP) * static_cast<double>(keep_mass)));
      const int p = first([&](int i) { return (i == 0 ? 0ull : sh.cscan[i - 1]) >= thr; });
      if (p >= 0) {
        keep_n = static_cast<uint32_t>(p);
        keep_mass = p == 0 ? 0ull : sh.cscan[p - 1];
        cut = true;
      }
    }
    int64_t tok = -1;
    uint64_t CK = static_cast<uint64_t>(KEY_MIN_FINITE) << 32;
    uint32_t tau_out = KEY_MIN_FINITE;
    int32_t st = 0;
    if (keep_n == 0) {
      st |= FL_ROW_ALL_MASKED;
    } else {
      const uint64_t last = sh.cand[keep_n - 1];
      tau_out = static_cast<uint32_t>(last >> 32);
      CK = cut ? last : static_cast<uint64_t>(tau_out) << 32;
      if (R.select) {
        int is = 0;
        if (R.T > 0.0f) {
          // inverse CDF: first kept candidate whose inclusive mass exceeds
          // floor(u * kept mass) (the last kept one when none does)
          const uint64_t target = static_cast<uint64_t>(floor(static_cast<double>(R.U) * static_cast<double>(keep_mass)));
          is = first([&](int i) { return sh.cscan[i] > target; });
          if (is < 0) is = static_cast<int>(keep_n) - 1;
        }
        tok = static_cast<int64_t>(~static_cast<uint32_t>(sh.cand[is]));
      }
    }
    if (lane == 0) {
      sh.bcast_u = static_cast<uint32_t>(st);
      sh.fkey[0] = tau_out;
      sh.fck = CK;
      sh.fmass_out = keep_mass;
      sh.pick_n = keep_n;
      sh.ftok = tok;
    }
  }
  __syncthreads();
  o.status = static_cast<int32_t>(sh.bcast_u);
  o.tau = sh.fkey[0];
  o.CK = sh.fck;
  o.keep_mass = sh.fmass_out;
  o.keep_n = sh.pick_n;
  o.tok = sh.ftok;
  FL_MARK(7);
  return true;
}

// Read 1 of the two-read path: anchor the bins on the largest value among the
// first 4 chunks per thread, then add every element to its bin.  Returns false
// (uniformly) when the anchor is not a finite value below 2^20 in magnitude.
template <bool TDIV, bool PEN, bool SC>
__device__ __forceinline__ bool read1(Shared32& sh, const Src& S, const Xform& X, int V, float& c, uint32_t& km,
                                      uint32_t& nfin, uint32_t& bad) {
  const int tid = threadIdx.x;
  for (int i = tid; i < NBF; i += NT) sh.acc[i] = 0;
  float yb[16];
  {
    float4 q[4];
    S.chunks(0, q);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int ch = u * NT + tid;
      const uint32_t hb = PEN ? X.nibble(ch) : 0u;
      const float xs[4] = {q[u].x, q[u].y, q[u].z, q[u].w};
      float y4[4];
      X.yt4<TDIV, PEN, SC>(xs, hb, y4);
#pragma unroll
      for (int e = 0; e < 4; ++e) yb[4 * u + e] = y4[e];
    }
  }
#pragma unroll
  for (int j = 0; j < 16; ++j) {
    const int idx = 4 * ((j >> 2) * NT + tid) + (j & 3);
    if (idx < V && yb[j] == yb[j]) km = max(km, f32_key(yb[j]));
  }
  const uint32_t ka = block_reduce<uint32_t>(km, OpMax(), sh.redu);  // also orders the bin clearing
  const float A = f32_of_key(ka);
  if (!(ka > KEY_NEG_INF && ka < KEY_POS_INF && fabsf(A) < 1048576.0f)) return false;
  c = A + ANCHOR_UP;

  // branch-free: an element outside the bins adds 0 to the discard slot
  auto add = [&](int idx, float y) __attribute__((always_inline)) {
    const bool valid = idx < V;
    bad |= (valid && y != y) ? 2u : 0u;
    bad |= (valid && y > c) ? 1u : 0u;
    const bool ok = valid && y <= c;
    km = max(km, ok ? f32_key(y) : 0u);
    nfin += (ok && y > -__builtin_inff()) ? 1u : 0u;
    const int b = fbin(y, c);
    const uint64_t w = (1ull << CNT_SH) | fterm(y, c);
    atomicAdd(reinterpret_cast<unsigned long long*>(&sh.acc[ok ? b : NBF]),
              static_cast<unsigned long long>(ok ? w : 0ull));
  };
  // A chunk of 4 whose values are all valid, finite and inside the bins (the
  // usual case) needs no per-element test: its maximum, minimum and sum
  // (NaN if any value is) decide it once; any other chunk goes element by
  // element.  (fmaxf / fminf skip NaN, the sum does not.)
  auto add4 = [&](int ch, const float (&y)[4]) __attribute__((always_inline)) {
    const float mx = fmaxf(fmaxf(y[0], y[1]), fmaxf(y[2], y[3]));
    const float mn = fminf(fminf(y[0], y[1]), fminf(y[2], y[3]));
    const float sm = (y[0] + y[1]) + (y[2] + y[3]);
    if (4 * ch + 3 < V && mx <= c && mn > -__builtin_inff() && sm == sm) {
      km = max(km, f32_key(mx));
      nfin += 4u;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int b = fbin(y[e], c);
        const uint64_t w = (1ull << CNT_SH) | fterm(y[e], c);
        atomicAdd(reinterpret_cast<unsigned long long*>(&sh.acc[b]), static_cast<unsigned long long>(w));
      }
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) add(4 * ch + e, y[e]);
    }
  };
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const float y4[4] = {yb[4 * u], yb[4 * u + 1], yb[4 * u + 2], yb[4 * u + 3]};
    add4(u * NT + tid, y4);
  }
  const int nch = X.nch;
  const int ng = nch > 4 * NT ? (nch - 4 * NT + 4 * WAVE - 1) / (4 * WAVE) : 0;
  wave_groups(S, &sh.grp[0], 4 * NT, ng, false, [&](int ch, const float4& q) __attribute__((always_inline)) {
    const uint32_t hb = PEN ? X.nibble(ch) : 0u;
    const float xs[4] = {q.x, q.y, q.z, q.w};
    float y4[4];
    X.yt4<TDIV, PEN, SC>(xs, hb, y4);
    add4(ch, y4);
    __builtin_amdgcn_sched_barrier(0);
  });
  return true;
}

// The two-read path.  Returns false, with nothing decided, when the row needs
// the multi-pass path.  Called by all threads (block-uniform control flow).
__device__ __forceinline__ bool two_read(Shared32& sh, const Src& S, const Xform& X, const RowCfg& R, RowOut& o) {
  const int tid = threadIdx.x;
  const int lane = tid & (WAVE - 1);
  const int V = R.V;
  o.kmax = 0;
  o.status = 0;
  o.tau = KEY_MIN_FINITE;
  o.CK = static_cast<uint64_t>(KEY_MIN_FINITE) << 32;
  o.keep_mass = 0;
  o.keep_n = 0;
  o.tok = -1;

  // ---------------------------------------------- read 1
  uint32_t km = 0, nfin = 0, bad = 0;  // bad: 1 a value above the bins, 2 NaN
  float c = 0.0f;
  bool anchored;
  const bool tdiv = X.t > 0.0f;
  auto r1 = [&](auto tdiv_c, auto pen_c, auto sc_c) -> bool {
    return read1<decltype(tdiv_c)::value, decltype(pen_c)::value, decltype(sc_c)::value>(sh, S, X, V, c, km, nfin,
                                                                                         bad);
  };
  using T_ = std::true_type;
  using F_ = std::false_type;
  if (X.cap > 0.0f) {
    if (X.pen) anchored = tdiv ? r1(T_{}, T_{}, T_{}) : r1(F_{}, T_{}, T_{});
    else anchored = tdiv ? r1(T_{}, F_{}, T_{}) : r1(F_{}, F_{}, T_{});
  } else {
    if (X.pen) anchored = tdiv ? r1(T_{}, T_{}, F_{}) : r1(F_{}, T_{}, F_{});
    else anchored = tdiv ? r1(T_{}, F_{}, F_{}) : r1(F_{}, F_{}, F_{});
  }
  if (!anchored) return false;
  FL_MARK(1);
  const uint32_t kmx = block_reduce<uint32_t>(km, OpMax(), sh.redu);
  const uint32_t bad_all = block_reduce<uint32_t>(bad, OpOr(), sh.redu);
  const uint32_t nf = block_reduce<uint32_t>(nfin, OpAdd(), sh.redu);
  int32_t status = sh.status;
  if (bad_all & 2u) status |= FL_ROW_NAN;
  else if (bad_all & 1u) {
    // +inf values are above every bin
    if (status == 0) return false;
  }
  o.kmax = kmx;
  o.status = status;
  if (status != 0) return true;
  const float M = f32_of_key(kmx);

  // ---------------------------------------------- bin prefixes
  uint32_t tc;
  uint64_t tm;
  {
    uint32_t cb[4];
    uint64_t mb[4];
    uint32_t lc = 0;
    uint64_t lm = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = 4 * tid + j;
      const uint64_t w = sh.acc[b];
      cb[j] = static_cast<uint32_t>(w >> CNT_SH);
      mb[j] = fmass(w & TERM_MASK, b, c, M);
      lc += cb[j];
      lm += mb[j];
    }
    uint32_t ec;
    uint64_t em;
    block_excl_scan2(lc, lm, sh.redu, sh.redq, ec, em, tc, tm);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int b = 4 * tid + j;
      sh.pc[b] = ec;
      sh.acc[b] = em;
      ec += cb[j];
      em += mb[j];
    }
  }
  __syncthreads();
  FL_MARK(2);
  auto Pn = [&](int b) -> uint32_t { return b < NBF ? sh.pc[b] : tc; };
  auto Qm = [&](int b) -> uint64_t { return b < NBF ? sh.acc[b] : tm; };

  const bool tk_on = R.K > 0 && R.K < V;
  const bool mp_on = R.MP > 0.0f;
  const bool tp_on = R.TP > 0.0f && R.TP < 1.0f;

  // ---------------------------------------------- plan (wave 0)
  // fplan: 0 ok, 1 status, 2 bk, 3 bc, 4 ranges, 5 gathered count
  if (tid < WAVE) {
    int ok = 1;
    int32_t st = 0;
    int bk = NBF, bm = NBF;
    uint32_t kp = 0;
    if (tk_on) bk = wave_first(0, NBF, [&](int b) { return Pn(b + 1) > static_cast<uint32_t>(R.K - 1); });
    if (mp_on) {
      if (!(1.0f >= R.MP)) {
        st |= FL_ROW_ALL_MASKED;  // min_p > 1 removes every value
      } else {
        // smallest key whose value passes exp(y - M) >= min_p (kmx passes): a
        // 64-way search of the wave over the monotone predicate
        kp = wave_first_key(KEY_MIN_FINITE, kmx, [&](uint32_t k) { return expf(f32_of_key(k) - M) >= R.MP; });
        bm = fbin(f32_of_key(kp), c);
      }
    }
    const int bc = min(bk, bm);  // bin of the binding value cut (NBF: none)
    if (bc == NBF - 1) ok = 0;
    int lo_[NRANGE], hi_[NRANGE];
    int nr = 0;
    if (bc < NBF) {
      lo_[nr] = bc;
      hi_[nr] = bc;
      ++nr;
    }
    uint64_t kmlo = tm, kmhi = tm;  // bounds of the mass kept by the value cuts
    if (bc < NBF) {
      kmlo = Qm(bc);
      kmhi = Qm(bc + 1);
    }
    int blast = bc < NBF ? bc : NBF - 1;  // last bin holding kept values
    uint64_t k2lo = kmlo, k2hi = kmhi;
    if (tp_on) {
      const uint64_t tlo = static_cast<uint64_t>(ceil(static_cast<double>(R.TP) * static_cast<double>(kmlo)));
      const uint64_t thi = static_cast<uint64_t>(ceil(static_cast<double>(R.TP) * static_cast<double>(kmhi)));
      const int plo = min(blast, wave_first(0, NBF, [&](int b) { return Qm(b + 1) >= tlo; }));
      const int phi = min(blast, wave_first(0, NBF, [&](int b) { return Qm(b + 1) >= thi; }));
      if (phi >= NBF - 1) ok = 0;
      lo_[nr] = plo;
      hi_[nr] = phi;
      ++nr;
      // the kept mass ends at the crossing member: at least thr, at most the
      // inclusive mass of its bin
      k2lo = tlo;
      k2hi = min(kmhi, Qm(phi + 1));
      blast = phi;
    }
    if (R.select) {
      int s0, s1;
      if (R.T > 0.0f) {
        const uint64_t tlo = static_cast<uint64_t>(floor(static_cast<double>(R.U) * static_cast<double>(k2lo)));
        const uint64_t thi = static_cast<uint64_t>(floor(static_cast<double>(R.U) * static_cast<double>(k2hi)));
        s0 = min(blast, wave_first(0, NBF, [&](int b) { return Qm(b + 1) > tlo; }));
        s1 = min(blast, wave_first(0, NBF, [&](int b) { return Qm(b + 1) > thi; }));
      } else {
        s0 = s1 = wave_first(0, NBF, [&](int b) { return Pn(b + 1) > 0u; });  // the maximum's bin
      }
      if (s1 >= NBF - 1) ok = 0;
      lo_[nr] = s0;
      hi_[nr] = s1;
      ++nr;
    }
    // sort the ranges by their first bin and merge overlapping or adjacent ones
    for (int i = 1; i < nr; ++i)
      for (int j = i; j > 0 && lo_[j] < lo_[j - 1]; --j) {
        const int tl = lo_[j], th = hi_[j];
        lo_[j] = lo_[j - 1];
        hi_[j] = hi_[j - 1];
        lo_[j - 1] = tl;
        hi_[j - 1] = th;
      }
    int m = 0;
    for (int i = 0; i < nr; ++i) {
      if (m > 0 && lo_[i] <= hi_[m - 1] + 1) {
        hi_[m - 1] = max(hi_[m - 1], hi_[i]);
      } else {
        lo_[m] = lo_[i];
        hi_[m] = hi_[i];
        ++m;
      }
    }
    uint32_t total = 0;
    for (int i = 0; i < m; ++i) {
      if (lane == 0) {
        sh.rlo[i] = lo_[i];
        sh.rhi[i] = hi_[i];
        sh.rbase[i] = static_cast<int32_t>(total);
      }
      total += Pn(hi_[i] + 1) - Pn(lo_[i]);
    }
    if (total > static_cast<uint32_t>(CAP)) ok = 0;
    if (lane == 0) {
      for (int i = m; i < NRANGE; ++i) {
        sh.rlo[i] = 1;
        sh.rhi[i] = 0;
        sh.rbase[i] = 0;
      }
      sh.fplan[0] = ok;
      sh.fplan[1] = st;
      sh.fplan[2] = bk;
      sh.fplan[3] = bc;
      sh.fplan[4] = m;
      sh.fplan[5] = static_cast<int32_t>(total);
      sh.fplan[6] = bm;
      sh.fkey[0] = kp;
      sh.ncand = 0;
    }
  }
  __syncthreads();
  FL_MARK(3);
  const int32_t st = sh.fplan[1];
  if (st != 0) {
    o.status = st;
    return true;
  }
  if (!sh.fplan[0]) return false;
  const int bk = sh.fplan[2], bc = sh.fplan[3], nr = sh.fplan[4], ngath = sh.fplan[5], bm = sh.fplan[6];
  const uint32_t kp = sh.fkey[0];
  int rl[NRANGE], rh[NRANGE], rb[NRANGE];
#pragma unroll
  for (int i = 0; i < NRANGE; ++i) {
    rl[i] = sh.rlo[i];
    rh[i] = sh.rhi[i];
    rb[i] = sh.rbase[i];
  }
  auto gathered = [&](int b) {
    bool in = false;
#pragma unroll
    for (int i = 0; i < NRANGE; ++i) in |= b >= rl[i] && b <= rh[i];
    return in;
  };
  // index of bin b's first member among the candidates (b gathered)
  auto cstart = [&](int b) {
    int s = 0;
#pragma unroll
    for (int i = 0; i < NRANGE; ++i)
      if (b >= rl[i] && b <= rh[i]) s = rb[i] + static_cast<int>(Pn(b) - Pn(rl[i]));
    return s;
  };

  uint32_t tau = KEY_MIN_FINITE;
  uint64_t CK = static_cast<uint64_t>(tau) << 32;
  uint32_t keep_n = nf;
  uint64_t keep_mass = tm;
  int64_t tok = -1;
  if (nr > 0) {
    // ---------------------------------------------- read 2
    // y is non-decreasing in the raw logit x within each class (history
    // members or not), so the values of a bin range come from one interval
    // of x per class.  One wave per interval end finds it by a 64-way search
    // over the float order; the second read then stages only the elements
    // whose raw logit lies in an interval, and y is evaluated for those alone.
    // A non-monotone rounding would lose members, which the count check below
    // catches (the row then takes the multi-pass path).
    {
      const int w = tid / WAVE;
      const int nb = 2 * nr * (X.pen ? 2 : 1);
      if (w < nb) {
        const int r = (w >> 1) % nr;
        const bool hist = w >= 2 * nr;
        const bool upper = w & 1;
        auto bin_of_x = [&](uint32_t kx) { return fbin(X.y(f32_of_key(kx), hist), c); };
        auto pred = [&](uint32_t kx) { return upper ? bin_of_x(kx) < rl[r] : bin_of_x(kx) <= rh[r]; };
        // finite x only: +-inf map to +-inf (a non-finite y is never gathered)
        const uint32_t k0 = f32_key(-FLT_MAX), k1 = f32_key(FLT_MAX) + 1u;
        // First a window of 2^13 keys around an approximate inverse of the
        // bin bound (temperature, penalty and soft-cap undone); if the
        // predicate does not change inside it (checked at its two ends), the
        // whole range.  Either way the result is the first key where the
        // monotone predicate holds.
        constexpr uint32_t HALF = 4096;
        float xa = upper ? fub(rl[r], c) : fub(rh[r] + 1, c);
        if (X.t > 0.0f) xa *= X.t;
        if (hist) xa = xa > 0.0f ? xa * X.rp : xa / X.rp;
        if (X.cap > 0.0f) xa = fabsf(xa) < X.cap ? atanhf(xa / X.cap) * X.cap : __builtin_nanf("");
        uint32_t k = k1;
        bool found = false;
        if (fabsf(xa) <= FLT_MAX) {   // (false for NaN)
          const uint32_t ka = f32_key(xa);
          const uint32_t a0 = ka > k0 + HALF ? ka - HALF : k0;
          const uint32_t b0 = ka + HALF < k1 ? ka + HALF : k1;
          if ((a0 == k0 || !pred(a0 - 1u)) && pred(b0 - 1u)) {
            k = wave_first_key(a0, b0, pred);
            found = true;
          }
        }
        if (!found) k = wave_first_key(k0, k1, pred);
        if (lane == 0) {
          // empty interval: lower end +inf or upper end -inf
          if (!upper) sh.xlo[hist][r] = k == k1 ? __builtin_inff() : f32_of_key(k);
          else sh.xhi[hist][r] = k == k0 ? -__builtin_inff() : f32_of_key(k - 1u);
        }
      }
      __syncthreads();
    }
    FL_MARK(4);
    // interval ends of the plain (0) and history (1) classes; unused ranges empty
    float xl0[NRANGE], xh0[NRANGE], xl1[NRANGE], xh1[NRANGE];
#pragma unroll
    for (int i = 0; i < NRANGE; ++i) {
      xl0[i] = i < nr ? sh.xlo[0][i] : __builtin_inff();
      xh0[i] = i < nr ? sh.xhi[0][i] : -__builtin_inff();
      xl1[i] = i < nr && X.pen ? sh.xlo[1][i] : __builtin_inff();
      xh1[i] = i < nr && X.pen ? sh.xhi[1][i] : -__builtin_inff();
    }
    // (instantiated per range count and history: each element is tested
    // against the ranges the plan uses, and a chunk takes one ballot)
    auto stage = [&](auto pen_tag, auto nr_tag) __attribute__((always_inline)) {
      constexpr bool PEN = decltype(pen_tag)::value;
      constexpr int NR = decltype(nr_tag)::value;
      // (claimed groups, the row's last chunks first: read 1 went first to
      // last, so the bytes it read most recently, the likeliest still in
      // the caches, are read again first)
      wave_groups(S, &sh.grp[1], 0, (X.nch + 4 * WAVE - 1) / (4 * WAVE), true,
                  [&](int c, const float4& q) __attribute__((always_inline)) {
        const float xs[4] = {q.x, q.y, q.z, q.w};
        const uint32_t hb = X.nibble(c);
        bool in[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float x = xs[e];
          bool a = false;
#pragma unroll
          for (int i = 0; i < NR; ++i) a |= x >= xl0[i] && x <= xh0[i];
          if constexpr (PEN) {
            bool ah = false;
#pragma unroll
            for (int i = 0; i < NR; ++i) ah |= x >= xl1[i] && x <= xh1[i];
            a = ((hb >> e) & 1u) ? ah : a;
          }
          in[e] = a && 4 * c + e < V;
        }
        if (__ballot(in[0] || in[1] || in[2] || in[3])) {
#pragma unroll
          for (int e = 0; e < 4; ++e)
            wave_append(in[e],
                        (static_cast<uint64_t>(__float_as_uint(xs[e])) << 32) |
                            static_cast<uint32_t>(~static_cast<uint32_t>(4 * c + e)),
                        &sh.ncand, sh.cand);
        }
      });
    };
    using I1 = std::integral_constant<int, 1>;
    using I2 = std::integral_constant<int, 2>;
    using I3 = std::integral_constant<int, 3>;
    using I4 = std::integral_constant<int, 4>;
    auto stage_nr = [&](auto pen_tag) __attribute__((always_inline)) {
      if (nr <= 1) stage(pen_tag, I1{});
      else if (nr == 2) stage(pen_tag, I2{});
      else if (nr == 3) stage(pen_tag, I3{});
      else stage(pen_tag, I4{});
    };
    if (X.pen) stage_nr(std::true_type{});
    else stage_nr(std::false_type{});
    __syncthreads();
    FL_MARK(5);
    const int ns = static_cast<int>(sh.ncand);
    if (ns > CAP) return false;
    // staged raw logits -> candidates (key << 32 | ~index); non-members -> 0
    uint32_t nm = 0;
    for (int i = tid; i < ns; i += NT) {
      const uint64_t v = sh.cand[i];
      const int idx = static_cast<int>(~static_cast<uint32_t>(v));
      const float y = X.y(__uint_as_float(static_cast<uint32_t>(v >> 32)), (X.nibble(idx >> 2) >> (idx & 3)) & 1u);
      const bool mem = y <= c && gathered(fbin(y, c));
      nm += mem ? 1u : 0u;
      sh.cand[i] = mem ? (static_cast<uint64_t>(f32_key(y)) << 32) | (v & 0xFFFFFFFFull) : 0ull;
    }
    FL_MARK(10);
    nm = block_reduce<uint32_t>(nm, OpAdd(), sh.redu);
    if (nm != static_cast<uint32_t>(ngath)) return false;
    FL_MARK(11);
    // members first (every member word is nonzero)
    // (the rank sort's work grows as ns^2 / 16 cycles: 1.7 us at 256,
    // 27 us at 1024; the bitonic network's as its steps)
    if (ns <= RANK_SORT_MAX) rank_sort_desc(sh.cand, sh.cscan, reinterpret_cast<uint32_t*>(sh.cscan + RANK_SORT_MAX), ns);
    else bitonic_desc(sh.cand, ns);
    FL_MARK(6);
    const int n = ngath;

    // inclusive mass prefix at each candidate
    {
      uint64_t f[4];
      int bb[4];
      uint64_t ls = 0;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        f[j] = 0;
        bb[j] = 0;
        if (i < n) {
          const float y = f32_of_key(static_cast<uint32_t>(sh.cand[i] >> 32));
          bb[j] = fbin(y, c);
          f[j] = fterm(y, c);
          ls += f[j];
        }
      }
      uint64_t tot;
      uint64_t run = block_excl_scan<uint64_t>(ls, sh.redq, &tot);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        run += f[j];
        if (i < n) sh.cscan[i] = run;
      }
      __syncthreads();
      uint64_t incl[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        incl[j] = 0;
        if (i < n) {
          const int h = cstart(bb[j]);
          const uint64_t F = sh.cscan[i] - (h > 0 ? sh.cscan[h - 1] : 0ull);
          incl[j] = Qm(bb[j]) + fmass(F, bb[j], c, M);
        }
      }
      __syncthreads();
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int i = 4 * tid + j;
        if (i < n) sh.cscan[i] = incl[j];
      }
      __syncthreads();
    }

    // ---------------------------------------------- decisions (wave 0)
    if (tid < WAVE) {
      int ok = 1;
      int32_t st2 = 0;
      auto key_at = [&](int i) { return static_cast<uint32_t>(sh.cand[i] >> 32); };
      if (bc < NBF) {
        // value cuts: top-k keeps y >= the K-th largest, min-p keeps keys >= kp
        if (tk_on && bk == bc) tau = max(tau, key_at(cstart(bk) + (R.K - 1 - static_cast<int>(Pn(bk)))));
        if (mp_on && bm == bc) tau = max(tau, kp);
        const int h = cstart(bc), cnt = static_cast<int>(Pn(bc + 1) - Pn(bc));
        const int ck = wave_first(h, h + cnt, [&](int i) { return key_at(i) < tau; }) - h;
        keep_n = Pn(bc) + static_cast<uint32_t>(ck);
        keep_mass = ck > 0 ? sh.cscan[h + ck - 1] : Qm(bc);
      }
      CK = static_cast<uint64_t>(tau) << 32;
      if (keep_n == 0 || tau > o.kmax) st2 |= FL_ROW_ALL_MASKED;
      if (st2 == 0 && tp_on) {
        // first position whose inclusive mass reaches thr; it and all before are kept
        const uint64_t thr = static_cast<uint64_t>(ceil(static_cast<double>(R.TP) * static_cast<double>(keep_mass)));
        const int bp = wave_first(0, NBF, [&](int b) { return Qm(b + 1) >= thr; });
        if (bp >= NBF || !gathered(bp)) {
          ok = 0;
        } else {
          const int h = cstart(bp), cnt = static_cast<int>(Pn(bp + 1) - Pn(bp));
          const int j = wave_first(h, h + cnt, [&](int i) { return sh.cscan[i] >= thr; });
          if (j >= h + cnt) {
            ok = 0;
          } else {
            CK = sh.cand[j];
            keep_n = Pn(bp) + static_cast<uint32_t>(j - h) + 1u;
            keep_mass = sh.cscan[j];
          }
        }
      }
      if (st2 == 0 && ok && R.select) {
        if (R.T > 0.0f) {
          const uint64_t target = static_cast<uint64_t>(floor(static_cast<double>(R.U) * static_cast<double>(keep_mass)));
          const int bs = wave_first(0, NBF, [&](int b) { return Qm(b + 1) > target; });
          if (bs >= NBF || !gathered(bs)) {
            ok = 0;
          } else {
            const int h = cstart(bs), cnt = static_cast<int>(Pn(bs + 1) - Pn(bs));
            const int j = wave_first(h, h + cnt, [&](int i) { return sh.cscan[i] > target; });
            if (j >= h + cnt || Pn(bs) + static_cast<uint32_t>(j - h) >= keep_n) ok = 0;
            else tok = static_cast<uint32_t>(~static_cast<uint32_t>(sh.cand[j]));
          }
        } else {
          tok = static_cast<uint32_t>(~static_cast<uint32_t>(sh.cand[0]));  // first index of the maximum
        }
      }
      if (lane == 0) {
        sh.fplan[0] = ok;
        sh.fplan[1] = st2;
        sh.fkey[1] = tau;
        sh.fplan[7] = static_cast<int32_t>(keep_n);
        sh.fmass_out = keep_mass;
        sh.ftok = tok;
        sh.fck = CK;
      }
    }
    __syncthreads();
    FL_MARK(7);
    if (!sh.fplan[0]) return false;
    o.status = sh.fplan[1];
    tau = sh.fkey[1];
    keep_n = static_cast<uint32_t>(sh.fplan[7]);
    keep_mass = sh.fmass_out;
    tok = sh.ftok;
    CK = sh.fck;
    __syncthreads();
  }
  o.tau = tau;
  o.CK = CK;
  o.keep_n = keep_n;
  o.keep_mass = keep_mass;
  o.tok = tok;
  return true;
}

}  // namespace

__global__ __launch_bounds__(NT) void k_sample_rows32(const fl_sample_args a) {
  __shared__ Shared32 sh;
  extern __shared__ uint32_t hbits_dyn[];
  FL_MARK(12);  // (kernel entry)
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int V = static_cast<int>(a.vocab);
  const float* row = static_cast<const float*>(a.logits) + b * a.ld;
  const bool select = (a.flags & FL_FLAG_NO_SELECT) == 0;

  const float T = a.temperature[b];
  const int K = a.top_k[b];
  const float TP = a.top_p[b];
  const float MP = a.min_p[b];
  const float RP = a.rep_penalty[b];
  const float U_in = select ? a.uniforms[a.uniform_div > 1 ? b / a.uniform_div : b] : 0.0f;
  const int H_in = a.hist_ids ? a.hist_len[b] : 0;
  // Each thread's first history id, requested by row stride before the row's
  // length is known, so that the id arrives with the parameters rather than
  // one memory round trip after them (the temperature array stands in when
  // there is no per-row id list, keeping the load unconditional).
  const bool hist_rows = a.hist_ids != nullptr && a.hist_ld > 0;
  const int32_t* hid = a.hist_ids ? a.hist_ids + b * a.hist_ld : nullptr;
  const int32_t hid0 = (hist_rows ? hid : reinterpret_cast<const int32_t*>(a.temperature))
      [hist_rows ? min(tid, static_cast<int>(min(a.hist_ld, static_cast<int64_t>(NT))) - 1) : 0];
  const float U = select ? fminf(fmaxf(U_in, 0.0f), 0.99999994f) : 0.0f;
  const bool hist_too_long = H_in > FL_MAX_HISTORY;
  const int H = (a.hist_ids != nullptr && RP != 1.0f && !hist_too_long) ? max(H_in, 0) : 0;
  const bool pen = H > 0;
  const int nch = (V + 3) >> 2;
  FL_MARK(0);

  Src S;
  S.rs = row_rsrc(row, 4u * static_cast<uint32_t>(V));
  S.V = V;
  S.nfull = V >> 2;
  S.aligned = (reinterpret_cast<uintptr_t>(row) & 15u) == 0;
  // top-k rows: the first loads of the row go out before the history is read
  const bool topk_first = K > 0 && K < V && K <= TK_MAX;
  float4 q[TK_TILE];
  if (topk_first) {
    topk_tile_load<0, TK_EARLY>(S, q);
    topk_init(sh);
  }

  if (tid == 0) {
    sh.status = hist_too_long ? FL_ROW_LIMIT : 0;
    sh.result = -1;
    sh.grp[0] = sh.grp[1] = sh.grp[2] = sh.grp[3] = 0;
  }
  // ------------------------------------------------ history bitmap
  if (pen) {
    for (int i = tid; i < (V + 31) / 32; i += NT) hbits_dyn[i] = 0;
  }
  __syncthreads();
  FL_MARK(14);
  if (pen) {
    for (int i = tid; i < H; i += NT) {
      const int id = (hist_rows && i == tid) ? hid0 : hid[i];
      if (id < 0 || id >= V) atomicOr(&sh.status, FL_ROW_BAD_HISTORY);
      else atomicOr(&hbits_dyn[id >> 5], 1u << (id & 31));
    }
  }
  __syncthreads();
  FL_MARK(15);

  Xform X;
  X.cap = a.softcap;
  X.rp = RP;
  X.t = T == 1.0f ? 0.0f : T;  // x / 1 == x exactly: skip the division
  X.rt = X.t > 0.0f ? recip_rt(X.t) : 0.0f;
  X.rpr = recip_rt(RP);
  X.rcap = a.softcap > 0.0f ? 1.0f / a.softcap : 0.0f;
  X.pen = pen;
  X.hbits = hbits_dyn;
  X.nch = nch;

  RowCfg R;
  R.V = V;
  R.K = K;
  R.T = T;
  R.TP = TP;
  R.MP = MP;
  R.U = U;
  R.select = select;
  RowOut o;
  if (!(topk_first && topk_path(sh, S, X, R, o, q)) && !two_read(sh, S, X, R, o)) {
  // ------------------------------------------------ first read: max, NaN
  uint32_t kmax = 0;
  int nan = 0;
  row_pass(S, X, [&](int, float y, bool valid) {
    if (valid) {
      if (y != y) nan = 1;
      else kmax = max(kmax, f32_key(y));
    }
  });
  kmax = block_reduce<uint32_t>(kmax, OpMax(), sh.redu);
  nan = block_reduce<int32_t>(nan, OpMax(), sh.redi);
  if (tid == 0) {
    if (nan) sh.status |= FL_ROW_NAN;
    else if (kmax >= KEY_POS_INF) sh.status |= FL_ROW_INF;
    else if (kmax <= KEY_NEG_INF) sh.status |= FL_ROW_ALL_MASKED;
  }
  __syncthreads();
  int32_t status = sh.status;
  const float M = f32_of_key(kmax);

  // ------------------------------------------------ helpers
  auto hist_pass = [&](uint32_t* cnt, uint64_t* mass, uint32_t klo, int shift, int nb) __attribute__((always_inline)) {
    for (int i = tid; i < nb; i += NT) {
      cnt[i] = 0;
      mass[i] = 0;
    }
    __syncthreads();
    row_pass(S, X, [&](int, float y, bool valid) {
      const uint32_t bin = (f32_key(y) - klo) >> shift;
      if (valid && bin < static_cast<uint32_t>(nb)) {
        atomicAdd(&cnt[bin], 1u);
        const uint64_t f = fx45(expf(y - M));
        if (f) atomicAdd(reinterpret_cast<unsigned long long*>(&mass[bin]), static_cast<unsigned long long>(f));
      }
    });
    __syncthreads();
  };
  auto collect = [&](uint32_t klo, uint32_t khi) -> int __attribute__((always_inline)) {
    int n;
    if (tid == 0) sh.ncand = 0;
    __syncthreads();
    row_pass(S, X, [&](int idx, float y, bool valid) {
      const uint32_t k = f32_key(y);
      const bool in = valid && (k - klo) <= (khi - klo);
      wave_append(in, (static_cast<uint64_t>(k) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(idx)),
                  &sh.ncand, sh.cand);
    });
    __syncthreads();
    n = min(static_cast<int>(sh.ncand), CAP);

    bitonic_desc(sh.cand, n);
    return n;
  };
  // Narrow the whole row down to the decision point of a criterion.
  auto narrow = [&](int crit, uint32_t rank, float mp, uint64_t thr, uint32_t tau) -> Narrow __attribute__((always_inline)) {
    Narrow r = {OUT_NONE, 0, 0, 0, 0, 0, 0, 0};
    Pick p = choose_bin(sh, sh.cnt1, sh.mass1, NB, 0u, 21, 0u, 0ull, crit, rank, mp, M, thr, tau);
    if (p.bin < 0) return r;
    uint32_t klo = static_cast<uint32_t>(p.bin) << 21;
    int shift = 21;
    uint32_t count = sh.cnt1[p.bin];
    uint64_t rmass = sh.mass1[p.bin];
    for (;;) {
      const uint32_t khi = klo + ((1u << shift) - 1u);
      r.klo = klo;
      r.khi = khi;
      r.n_ab = p.n_ex;
      r.m_ab = p.m_ex;
      r.count = count;
      r.rmass = rmass;
      if (count <= static_cast<uint32_t>(CAP)) {
        r.n = collect(klo, khi);
        r.out = OUT_CAND;
        return r;
      }
      if (shift == 0) {
        r.out = OUT_VALUE;
        return r;
      }
      const int nshift = shift == 21 ? 10 : 0;
      const int nb = shift == 21 ? NB : NB3;
      hist_pass(sh.cnt, sh.mass, klo, nshift, nb);
      const Pick q = choose_bin(sh, sh.cnt, sh.mass, nb, klo, nshift, p.n_ex, p.m_ex, crit, rank, mp, M, thr, tau);
      if (q.bin < 0) {
        r.out = OUT_ALLKEPT;
        return r;
      }
      klo = klo + (static_cast<uint32_t>(q.bin) << nshift);
      shift = nshift;
      count = sh.cnt[q.bin];
      rmass = sh.mass[q.bin];
      p = q;
      __syncthreads();
    }
  };
  // Count and mass of the candidates [0, n) with key >= tau.
  auto cand_sum = [&](int n, uint32_t tau, uint32_t& cnt_out, uint64_t& mass_out) __attribute__((always_inline)) {
    uint32_t c = 0;
    uint64_t m = 0;
    for (int i = tid; i < n; i += NT) {
      const uint64_t v = sh.cand[i];
      const uint32_t k = static_cast<uint32_t>(v >> 32);
      if (k >= tau) {
        ++c;
        m += fx45(expf(f32_of_key(k) - M));
      }
    }
    cnt_out = block_reduce<uint32_t>(c, OpAdd(), sh.redu);
    mass_out = block_reduce<uint64_t>(m, OpAdd(), sh.redq);
  };
  // Index of the member of rank r (ascending index) among elements with key v.
  auto find_rank = [&](uint32_t v, uint32_t r) -> int __attribute__((always_inline)) {
    if (tid == 0) sh.result = -1;
    __syncthreads();
    uint32_t base = 0;
    auto round = [&](uint32_t mbits, int c) -> bool {
      uint32_t tot;
      const uint32_t n = static_cast<uint32_t>(__popc(mbits));
      const uint32_t ex = block_excl_scan<uint32_t>(n, sh.redu, &tot);
      if (base + ex <= r && r < base + ex + n) {
        uint32_t need = r - base - ex;
        for (int e = 0; e < 4; ++e) {
          if ((mbits >> e) & 1u) {
            if (need == 0) {
              sh.result = 4 * c + e;
              break;
            }
            --need;
          }
        }
      }
      base += tot;
      return base > r;
    };
    for (int c0 = 0; c0 < nch; c0 += NT) {
      const int c = c0 + tid;
      const float4 q = S.chunk(c);
      const uint32_t hb = X.nibble(c);
      const float xs[4] = {q.x, q.y, q.z, q.w};
      uint32_t mb = 0;
#pragma unroll
      for (int e = 0; e < 4; ++e)
        mb |= static_cast<uint32_t>(4 * c + e < V && f32_key(X.y(xs[e], (hb >> e) & 1u)) == v) << e;
      if (round(mb, c)) break;
    }

    __syncthreads();
    const int res = sh.result;
    __syncthreads();
    return res;
  };

  // ------------------------------------------------ decisions
  // The kept set is a prefix of the order (descending key, ascending index):
  // composite (key << 32 | ~index) >= CK.  tau = key bound of the value cuts.
  uint32_t tau = KEY_MIN_FINITE;  // -inf entries are never kept
  uint64_t CK = static_cast<uint64_t>(tau) << 32;
  uint64_t keep_mass = 0;
  uint32_t keep_n = 0;
  int64_t tok = -1;

  if (status == 0) {
    hist_pass(sh.cnt1, sh.mass1, 0u, 21, NB);
    uint32_t c = 0;
    uint64_t m = 0;
    for (int i = tid; i < NB; i += NT) {
      m += sh.mass1[i];
      if (static_cast<uint32_t>(i) >= (KEY_MIN_FINITE >> 21)) c += sh.cnt1[i];
    }
    keep_n = block_reduce<uint32_t>(c, OpAdd(), sh.redu);
    keep_mass = block_reduce<uint64_t>(m, OpAdd(), sh.redq);
  }

  // Stages, in the reference's order: 0 top-k (sampling.py:36-38), 1 min-p
  // (:40-43), 2 top-p (:45-51), 3 selection (:56-61).  One narrowing per
  // stage; a stage whose decision falls inside a run of more than CAP equal
  // values asks for the index of one member by rank.
  for (int stage = 0; stage < 4; ++stage) {
    if (stage == 2) {
      CK = static_cast<uint64_t>(tau) << 32;
      if (tau > kmax || keep_n == 0) status |= FL_ROW_ALL_MASKED;
    }
    if (status != 0) break;
    bool active = false;
    int crit = CRIT_COUNT;
    uint32_t rank = 0, tr = 0;
    float mp = 0.0f;
    uint64_t thr = 0, target = 0;
    if (stage == 0) {
      active = K > 0 && K < V;
      rank = static_cast<uint32_t>(K - 1);
    } else if (stage == 1) {
      active = MP > 0.0f;
      crit = CRIT_PRED;
      mp = MP;
      tr = tau;
    } else if (stage == 2) {
      active = TP > 0.0f && TP < 1.0f;
      crit = CRIT_MASS;
      thr = static_cast<uint64_t>(ceil(static_cast<double>(TP) * static_cast<double>(keep_mass)));
      tr = tau;
    } else {
      active = select;
      if (T > 0.0f) {
        crit = CRIT_MASS;
        target = static_cast<uint64_t>(floor(static_cast<double>(U) * static_cast<double>(keep_mass)));
        thr = target + 1u;
        tr = static_cast<uint32_t>(CK >> 32);
      }
    }
    if (!active) continue;
    const Narrow n = narrow(crit, rank, mp, thr, tr);

    bool need_rank = false;
    uint32_t rv = 0, rr = 0;
    if (stage == 0) {
      // k-th largest value; every element equal to it survives
      uint32_t tk = 0;
      if (n.out == OUT_CAND) tk = static_cast<uint32_t>(sh.cand[K - 1 - static_cast<int>(n.n_ab)] >> 32);
      else if (n.out == OUT_VALUE) tk = n.klo;
      if (tk > tau) {
        tau = tk;
        if (n.out == OUT_CAND) {
          uint32_t c;
          uint64_t m;
          cand_sum(n.n, tau, c, m);
          keep_n = n.n_ab + c;
          keep_mass = n.m_ab + m;
        } else {
          keep_n = n.n_ab + n.count;
          keep_mass = n.m_ab + n.rmass;
        }
      }
    } else if (stage == 1) {
      // smallest kept value: the passing candidates form a prefix
      uint32_t tm = 0;
      bool whole_range = false;
      if (n.out == OUT_CAND) {
        uint32_t c = 0;
        for (int i = tid; i < n.n; i += NT) {
          const uint32_t k = static_cast<uint32_t>(sh.cand[i] >> 32);
          c += (k >= tau && expf(f32_of_key(k) - M) >= MP) ? 1u : 0u;
        }
        c = block_reduce<uint32_t>(c, OpAdd(), sh.redu);
        tm = c > 0 ? static_cast<uint32_t>(sh.cand[c - 1] >> 32) : n.khi + 1u;
      } else if (n.out == OUT_VALUE) {
        tm = (expf(f32_of_key(n.klo) - M) >= MP) ? n.klo : n.klo + 1u;
        whole_range = tm == n.klo;
      } else if (n.out == OUT_ALLKEPT) {
        tm = n.klo;
        whole_range = true;
      }
      if (tm > tau) {
        tau = tm;
        if (n.out == OUT_CAND) {
          uint32_t c;
          uint64_t m;
          cand_sum(n.n, tau, c, m);
          keep_n = n.n_ab + c;
          keep_mass = n.m_ab + m;
        } else {
          keep_n = n.n_ab + (whole_range ? n.count : 0u);
          keep_mass = n.m_ab + (whole_range ? n.rmass : 0ull);
        }
      }
    } else if (stage == 2) {
      // first kept position whose exclusive mass reaches thr
      if (n.out == OUT_CAND) {
        const int per = (n.n + NT - 1) / NT;
        const int i0 = min(n.n, tid * per), i1 = min(n.n, i0 + per);
        uint64_t lm = 0;
        for (int i = i0; i < i1; ++i) {
          const uint32_t k = static_cast<uint32_t>(sh.cand[i] >> 32);
          if (k >= tau) lm += fx45(expf(f32_of_key(k) - M));
        }
        uint64_t tot;
        const uint64_t ex = block_excl_scan<uint64_t>(lm, sh.redq, &tot);
        int first = INT_MAX;
        uint64_t mass_before = 0;
        uint64_t c = n.m_ab + ex;
        for (int i = i0; i < i1; ++i) {
          const uint32_t k = static_cast<uint32_t>(sh.cand[i] >> 32);
          if (k < tau) break;  // candidates below tau follow every kept one
          if (c >= thr) {
            first = i;
            mass_before = c;
            break;
          }
          c += fx45(expf(f32_of_key(k) - M));
        }
        const int f = block_reduce<int32_t>(first, OpMin(), sh.redi);
        if (f != INT_MAX) {
          if (first == f) sh.bcast_q = mass_before;
          __syncthreads();
          CK = f == 0 ? static_cast<uint64_t>(n.khi + 1u) << 32 : sh.cand[f - 1];
          keep_n = n.n_ab + static_cast<uint32_t>(f);
          keep_mass = sh.bcast_q;
          __syncthreads();
        } else {
          // no kept candidate is removed: the bin's mass reaches thr, so the
          // first removed element is the next one after the bin
          uint32_t nk = 0;
          for (int i = tid; i < n.n; i += NT) nk += static_cast<uint32_t>(sh.cand[i] >> 32) >= tau ? 1u : 0u;
          nk = block_reduce<uint32_t>(nk, OpAdd(), sh.redu);
          if (nk > 0) {
            CK = sh.cand[nk - 1];
            keep_n = n.n_ab + nk;
            keep_mass = n.m_ab + tot;
          }
        }
      } else if (n.out == OUT_VALUE) {
        // members of one value, in index order, each of mass fv
        const uint32_t v = n.klo;
        const uint64_t fv = fx45(expf(f32_of_key(v) - M));
        uint64_t jstar = n.count;  // first removed member
        if (n.m_ab >= thr) jstar = 0;
        else if (fv > 0) jstar = (thr - n.m_ab + fv - 1) / fv;
        if (jstar > n.count) jstar = n.count;
        if (jstar == 0) CK = static_cast<uint64_t>(v + 1u) << 32;
        else if (jstar == n.count) CK = static_cast<uint64_t>(v) << 32;  // the whole value stays
        need_rank = jstar > 0 && jstar < n.count;
        rv = v;
        rr = static_cast<uint32_t>(jstar) - 1u;
        keep_n = n.n_ab + static_cast<uint32_t>(jstar);
        keep_mass = n.m_ab + jstar * fv;
      }
    } else {
      if (T <= 0.0f) {
        // greedy (sampling.py:59-60): first index of the maximal value
        if (n.out == OUT_CAND) tok = static_cast<uint32_t>(~static_cast<uint32_t>(sh.cand[0]));
        need_rank = n.out == OUT_VALUE;
        rv = n.klo;
        rr = 0;
      } else if (n.out == OUT_CAND) {
        // inverse CDF over the kept candidates
        const int per = (n.n + NT - 1) / NT;
        const int i0 = min(n.n, tid * per), i1 = min(n.n, i0 + per);
        uint64_t lm = 0;
        int last_kept = -1;
        for (int i = i0; i < i1; ++i) {
          if (sh.cand[i] >= CK) {
            lm += fx45(expf(f32_of_key(static_cast<uint32_t>(sh.cand[i] >> 32)) - M));
            last_kept = i;
          }
        }
        uint64_t tot;
        const uint64_t ex = block_excl_scan<uint64_t>(lm, sh.redq, &tot);
        int first = INT_MAX;
        uint64_t c = n.m_ab + ex;
        for (int i = i0; i < i1; ++i) {
          if (sh.cand[i] < CK) break;
          c += fx45(expf(f32_of_key(static_cast<uint32_t>(sh.cand[i] >> 32)) - M));
          if (c > target) {
            first = i;
            break;
          }
        }
        int f = block_reduce<int32_t>(first, OpMin(), sh.redi);
        // the target lies past the kept members of this bin only through the
        // ceiling of the top-p threshold: take the last kept candidate
        if (f == INT_MAX) f = block_reduce<int32_t>(last_kept, OpMax(), sh.redi);
        if (f >= 0) tok = static_cast<uint32_t>(~static_cast<uint32_t>(sh.cand[f]));
      } else if (n.out == OUT_VALUE) {
        const uint32_t v = n.klo;
        const uint64_t fv = fx45(expf(f32_of_key(v) - M));
        uint32_t kept_cnt = n.count;  // members of this value inside the kept set
        if (static_cast<uint32_t>(CK >> 32) == v && static_cast<uint32_t>(CK) != 0u) kept_cnt = keep_n - n.n_ab;
        uint64_t j = 0;
        if (fv > 0 && target >= n.m_ab) j = (target - n.m_ab) / fv;
        if (j + 1 > kept_cnt) j = kept_cnt > 0 ? kept_cnt - 1 : 0;
        need_rank = true;
        rv = v;
        rr = static_cast<uint32_t>(j);
      }
    }
    if (need_rank) {
      const int idx = find_rank(rv, rr);
      if (stage == 2) CK = (static_cast<uint64_t>(rv) << 32) | static_cast<uint32_t>(~static_cast<uint32_t>(idx));
      else tok = idx;
    }
    if (stage == 2 && keep_n == 0) status |= FL_ROW_ALL_MASKED;
    if (stage == 3 && tok < 0) status |= FL_ROW_LIMIT;
  }

  o.kmax = kmax;
  o.status = status;
  o.tau = tau;
  o.CK = CK;
  o.keep_mass = keep_mass;
  o.keep_n = keep_n;
  o.tok = tok;
  }  // multi-pass path

  const float M = f32_of_key(o.kmax);
  int32_t status = o.status;
  int64_t tok = o.tok;
  const uint64_t CK = o.CK;
  const uint32_t keep_n = o.keep_n;
  const double SK = from_fx45(o.keep_mass);
  const float rK = 1.0f / static_cast<float>(SK);
  // Greedy (sampling.py:59-60) is torch.argmax of the float32 probabilities:
  // the first index among equal probabilities.  Values a few ulp below the
  // maximum M (|M| small, so that exp(y - M) rounds to 1) can share the
  // maximum's probability; the token is then the lowest such kept index.
  // Rows whose next value below M already has a smaller probability (every
  // row with |M| >= 0.25) skip the pass.
  if (select && T <= 0.0f && status == 0 && tok >= 0) {
    const float below = f32_of_key(f32_key(M) - 1u);  // the next float below M (M is finite)
    if (expf(below - M) * rK == rK) {
      const float ycut = f32_of_key(static_cast<uint32_t>(CK >> 32));
      const uint32_t lowc = static_cast<uint32_t>(CK);
      const int icut = lowc == 0u ? INT_MAX : static_cast<int>(~lowc);
      int best = static_cast<int>(tok);
      row_pass(S, X, [&](int idx, float y, bool valid) {
        const bool kept = y > ycut || (y == ycut && idx <= icut);
        if (valid && kept && idx < best && y < M && expf(y - M) * rK == rK) best = idx;
      });
      best = block_reduce<int32_t>(best, OpMin(), sh.redi);
      tok = best;
    }
  }
  float y_sel = 0.0f;
  if (tid == 0 && status == 0 && tok >= 0 && a.out_logprob) {
    const int i = static_cast<int>(tok);
    y_sel = X.y(row[i], (X.nibble(i >> 2) >> (i & 3)) & 1u);
  }

  // ------------------------------------------------ outputs
  if (tid == 0) {
    if (status != 0) tok = -1;
    // (read before any output is written: out_finished may be finished_in)
    const bool was_finished = a.finished_in != nullptr && a.finished_in[b] != 0;
    if (a.out_token) a.out_token[b] = tok;
    if (a.out_status) a.out_status[b] = status;
    if (a.out_finished) {
      const bool fin = was_finished || (tok >= 0 && is_stop(a.stop_ids, a.stop_ld, a.n_stop, b, tok));
      a.out_finished[b] = fin ? 1 : 0;
    }
    if (a.out_logprob) {
      float lp = __builtin_nanf("");
      if (tok >= 0) lp = (y_sel - M) - logf(static_cast<float>(SK));
      a.out_logprob[b] = lp;
    }
    if ((a.flags & FL_FLAG_APPEND_HISTORY) && a.hist_ids != nullptr && a.hist_ld > 0 && tok >= 0 && !was_finished &&
        H_in >= 0 && H_in < a.hist_ld) {
      // (every read of this row's history, all below index H_in, finished
      // before the barriers that led here)
      const_cast<int32_t*>(a.hist_ids)[b * a.hist_ld + H_in] = static_cast<int32_t>(tok);
      const_cast<int32_t*>(a.hist_len)[b] = H_in + 1;
    }
    if (a.out_desc) {
      fl_row_desc dsc;
      dsc.status = status;
      dsc.shift = M;
      dsc.mass = SK;
      dsc.inv_mass = rK;
      if (status == 0) {
        const uint32_t low = static_cast<uint32_t>(CK);
        dsc.y_cut = f32_of_key(static_cast<uint32_t>(CK >> 32));
        dsc.idx_cut = low == 0u ? INT_MAX : static_cast<int32_t>(~low);
        dsc.n_kept = static_cast<int32_t>(keep_n);
      } else {
        dsc.y_cut = __builtin_inff();
        dsc.idx_cut = -1;
        dsc.n_kept = 0;
      }
      a.out_desc[b] = dsc;
    }
  }
  FL_MARK(9);
}

// ------------------------------------------------------------------ launch
hipError_t launch_sample_rows32(const fl_sample_args& a, hipStream_t s) {
  const size_t dyn = a.hist_ids != nullptr ? static_cast<size_t>((a.vocab + 31) / 32) * 4u : 0u;
  hipLaunchKernelGGL(k_sample_rows32, dim3(static_cast<unsigned>(a.batch)), dim3(NT), dyn, s, a);
  return hipGetLastError();
}

}  // namespace fl

#ifdef FL_PHASE_TIMES
// Tuning builds only: copy the phase timestamps this kernel recorded.
extern "C" int fl_debug_phase_ts32(uint64_t* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(fl_phase_ts), sizeof(uint64_t) * FL_PHASE_SLOTS, 0,
                             hipMemcpyDeviceToHost) == hipSuccess ? 0 : -1;
}
#endif
