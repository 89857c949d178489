// Fused per-row sampler for bf16 / fp16 logits on gfx950.
//
// One work-group of 1024 threads owns one row.  A 16-bit dtype has only 65536
// values, so the row is summarised exactly by a histogram of its bit patterns
// (65536 packed 16-bit counters = 128 KB of LDS).  Every filter of the
// reference sampler (src/forgeline/models/generation/sampling.py:26-61) is
// then decided once per *distinct value* instead of once per element, with the
// reference's dtype rounding reproduced value by value:
//
//   load     the row is read from HBM once (16-byte loads) and kept in VGPRs
//   count    each element: one LDS atomic on its pattern's counter
//   history  ids are de-duplicated through an LDS bitmap; each unique id moves
//            one count from its pattern to its penalised pattern (:27-31)
//   compact  non-empty counters, in descending value order, become the entry
//            list (pattern, count)
//   decide   temperature, top-k, min-p, top-p and the inverse-CDF target are
//            evaluated over the entries with block scans (:33-61)
//   find     a sweep over the VGPR-resident row picks the element of the
//            chosen value with the chosen rank by vocabulary index
//
// Order convention: descending filtered value, ties by ascending vocabulary
// index.  All sums are float64 in a fixed order, so results are deterministic.
#include <type_traits>

#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {

namespace {

constexpr int NCH = 16;                          // 16-byte chunks per thread
constexpr int HIST_WORDS = 32768;                // 65536 packed u16 counters
constexpr int TILE_V = NCH * NT * 8;              // the VGPR tile: rows up to this length stay in registers
constexpr int HBITS_WORDS = TILE_V / 32;          // history bitmap (penalty rows up to TILE_V values)
constexpr int NSLOT = FL_MAX_VOCAB_16 / (NT * 8);  // identification slots of NT chunks
constexpr int OWNER_WORDS = FL_MAX_HISTORY / 32;
constexpr int HLIST_CAP = HIST_WORDS / 8;         // history members listed per identification target
constexpr int SLICE_BASE = HIST_WORDS - 3 * NT;   // slice tables: count u32[NT], mass u64[NT]
constexpr int ENT_MAX = SLICE_BASE;               // entries (distinct values) a row may have
constexpr int CACHE_MAX = (SLICE_BASE - 4) / 6;   // entries with y, e, prefix count and mass kept per entry
constexpr int NSTEP = 512;                        // compaction steps of 128 orders
constexpr int SPW = NSTEP / NWAVE;                // steps per wave
constexpr int HPRE = 2;                          // history ids per thread loaded ahead of the row
constexpr int EARLY_CHUNKS = 4;                  // row chunks per thread requested before the LDS clear
#ifndef FL_LOOKAHEAD
#define FL_LOOKAHEAD 4
#endif
constexpr int LOOKAHEAD = FL_LOOKAHEAD;          // row chunks per thread in flight while counting
static_assert(LOOKAHEAD >= EARLY_CHUNKS && LOOKAHEAD <= NCH, "lookahead window");
constexpr int MAX_HEAVY = 8;                     // patterns with more than 65535 values (at most 5 exist)

static_assert(NSLOT * NT * 8 == FL_MAX_VOCAB_16 && NSLOT >= NCH, "identification slots cover the longest row");

struct Shared16 {
  uint32_t hist[HIST_WORDS + WAVE];  // pattern counts, then one -inf counter per lane
  uint32_t hbits[HBITS_WORDS];
  uint32_t owner[OWNER_WORDS];
  uint64_t redq[NWAVE];
  uint32_t redu[NWAVE];
  uint64_t scan_sum[NWAVE];
  uint64_t scan_excl[NWAVE];
  int32_t scan_idx[NWAVE];
  alignas(16) uint32_t stepc[NSTEP];
  int32_t status;
  int32_t result[2];
  struct {
    double S, SK;
    int32_t L, i0, cut_lo, cut_hi, sel_lo, sel_hi;
    uint32_t c0, cut_kept, cut_total, n_kept, sel_rank;
    uint32_t o_lo[2], o_hi[2];
    float y_sel, y_cut;
  } dec;  // results of the search wave
  uint32_t wc[2][NSLOT][NWAVE];  // identification: members per slot of NT chunks and wave
  uint32_t nh[2];         // identification: history members
  uint32_t inf_extra;     // soft-capped rows: -inf values beyond their pattern's 16-bit count
  // patterns with more than 65535 values (at most 5: V + unique history ids
  // <= 327680): their order, exact count and the part beyond the 16-bit field
  uint32_t n_heavy;
  uint32_t hv_order[MAX_HEAVY], hv_count[MAX_HEAVY], hv_extra[MAX_HEAVY];
};

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

constexpr int NO_HIT = 0x7FFFFFFF;

struct ScanHit {
  int idx;         // first index whose predicate holds (n when none does)
  uint64_t excl;   // sum of the terms before idx
  uint64_t total;  // sum of all terms (or the total passed in)
};

// Block-wide search along n terms in index order: the first i for which
// pred(i, excl_i, total) holds, excl_i being the sum of the terms before i
// (the predicate must be false, then true, along the indices).  The terms are
// taken NT per round, one per thread; a round is a block scan with two
// barriers, and the search stops at the first round with a hit.  `total` is
// the sum of all n terms: known within the round when n <= NT, else passed in
// (total_given).  Every thread of the block calls it with the same arguments.
template <class TermF, class PredF>
__device__ __forceinline__ ScanHit scan_first(Shared16& sh, int n, bool total_given, uint64_t total_in, TermF&& term,
                                              PredF&& pred) {
  const int lane = threadIdx.x & (WAVE - 1);
  const int w = __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) / WAVE);
  uint64_t carry = 0;
  for (int base = 0; base < n; base += NT) {
    const int i = base + static_cast<int>(threadIdx.x);
    const bool act = base + w * WAVE < n;  // wave-uniform: this wave holds terms in this pass
    uint64_t v = 0, inc = 0;
    if (act) {
      v = i < n ? term(i) : 0ull;
      inc = wave_incl_scan(v);
    }
    if (lane == WAVE - 1) sh.scan_sum[w] = inc;
    lds_barrier();
    const uint64_t wi = wave_incl_scan(lane < NWAVE ? sh.scan_sum[lane] : 0ull);
    const uint64_t rtot = readlane64(wi, NWAVE - 1);
    const uint64_t total = total_given ? total_in : carry + rtot;
    int first = NO_HIT;
    uint64_t fex = 0;
    if (act) {
      const uint64_t excl = carry + (w > 0 ? readlane64(wi, w - 1) : 0ull) + (inc - v);
      const uint64_t m = __ballot(i < n && pred(i, excl, total));
      if (m) {
        const int f = __ffsll(static_cast<unsigned long long>(m)) - 1;
        first = base + w * WAVE + f;
        fex = readlane64(excl, f);
      }
    }
    if (lane == 0) {
      sh.scan_idx[w] = first;
      sh.scan_excl[w] = fex;
    }
    lds_barrier();
    const uint64_t hm = __ballot(lane < NWAVE && sh.scan_idx[lane] != NO_HIT);
    carry += rtot;
    if (hm) {
      const int fw = __ffsll(static_cast<unsigned long long>(hm)) - 1;
      return {sh.scan_idx[fw], sh.scan_excl[fw], total};
    }
  }
  return {n, carry, total_given ? total_in : carry};
}

// 16-byte chunk c (elements 8c .. 8c+7) of a row; elements >= V read as 0.
__device__ __forceinline__ uint4 load_chunk16(const uint16_t* row, int c, int V, bool aligned) {
  const int e0 = c * 8;
  if (aligned && e0 + 8 <= V) return reinterpret_cast<const uint4*>(row)[c];
  uint32_t w[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const int i = e0 + 2 * k;
    const uint32_t lo = (i < V) ? row[i] : 0u;
    const uint32_t hi = (i + 1 < V) ? row[i + 1] : 0u;
    w[k] = lo | (hi << 16);
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

// Value transforms of the rarer paths (soft-cap, values rebuilt from orders)
// are kept out of line: inlined at every call site they would multiply the
// kernel's code.  The penalty is small and on the common path: inline.
template <class D>
__device__ __noinline__ uint32_t capped_bits(uint32_t raw, float cap) {
  return D::from_f32(softcap_val<D>(D::to_f32(raw), cap));
}
template <class D>
__device__ __forceinline__ uint32_t penalised_bits(uint32_t z, float rp) {
  return D::from_f32(penalty_val<D>(D::to_f32(z), rp));
}
// filtered value of a pattern given as an order index (soft-cap if `sc`)
template <class D>
__device__ __noinline__ float value_of_order(uint32_t order, float cap, float t, float rt, bool sc) {
  float z = D::to_f32(bits_of_order16(order));
  if (sc) z = softcap_val<D>(z, cap);
  return temperature_val<D>(z, t, rt);
}
template <class D>
__device__ __noinline__ float e_of_order(uint32_t order, float cap, float t, float rt, bool sc, float M) {
  return expf(value_of_order<D>(order, cap, t, rt, sc) - M);
}
// The same for a kernel instantiated with or without the soft-cap: without
// it the value is cheap and inline, and the kernel makes no calls (a call
// would keep most VGPRs from holding values across it).
template <class D, bool SC>
__device__ __forceinline__ float y_of_order(uint32_t order, float cap, float t, float rt, bool sc) {
  if constexpr (SC) return value_of_order<D>(order, cap, t, rt, sc);
  else return temperature_val<D>(D::to_f32(bits_of_order16(order)), t, rt);
}
template <class D, bool SC>
__device__ __forceinline__ float exp_of_order(uint32_t order, float cap, float t, float rt, bool sc, float M) {
  if constexpr (SC) return e_of_order<D>(order, cap, t, rt, sc, M);
  else return expf(y_of_order<D, false>(order, cap, t, rt, false) - M);
}

// ------------------------------------------------ more than 65535 equal values
// A 16-bit counter wraps past 65535 (a constant or all-zero row, a mask with
// a finite floor such as finfo.min): the compaction then sees fewer values
// than the row holds.  Such a row recounts exactly (a few microseconds):
//   1. 32-bit counts of each half of the orders in the histogram's memory:
//      the values plus the ids the penalty moves in (a pattern whose count can
//      pass 65535 at any time of the counting is flagged), then less the ids
//      moved out (the flagged patterns' final counts);
//   2. the 16-bit histogram rebuilt without the flagged patterns, which get
//      as much of their count as 16 bits hold; the rest is kept per pattern
//      (hv_extra) and added wherever an entry's count is read.
// It does all the counting of the recounting body: the -inf values go to
// their lanes' counters as in the first count.
template <class D>
__device__ __forceinline__ void heavy_recount(Shared16& sh, const uint16_t* row, int V, int nfull, bool aligned,
                                           bool sc_elem, float cap, const int32_t* hid, int H, bool pen, float rp) {
  const int tid = threadIdx.x;
  constexpr uint32_t NEG_INF_RAW = 0x8000u | D::INF_BITS;
  auto elem_bits = [&](uint32_t raw) -> uint32_t { return sc_elem ? capped_bits<D>(raw, cap) : raw; };
  const bool neg_inf_value = cap > 0.0f;  // -inf is a value (-cap) only under a soft-cap
  auto for_each_value = [&](auto&& f) {  // f(raw) for every element
    for (int c = tid; c < nfull; c += NT) {
      const uint4 q = load_chunk16(row, c, V, aligned);
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) f((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
    }
    if (tid == 0)
      for (int i = nfull * 8; i < V; ++i) f(static_cast<uint32_t>(row[i]));
  };
  auto for_each_unique_id = [&](auto&& f) {  // f(raw) for the logit of every unique history id
    if (!pen) return;
    for (int i = tid; i < H; i += NT)
      if ((sh.owner[i >> 5] >> (i & 31)) & 1u) f(static_cast<uint32_t>(row[hid[i]]));
  };
  auto is_heavy = [&](uint32_t bits) {
    const uint32_t o = order16(bits);
    bool h = false;
    for (uint32_t k = 0; k < sh.n_heavy; ++k) h |= sh.hv_order[k] == o;
    return h;
  };
  uint32_t* c32 = sh.hist;  // 32768 counters: orders 32768 h .. 32768 h + 32767
  for (int h = 0; h < 2; ++h) {
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 8; ++k) reinterpret_cast<uint4*>(c32)[tid + k * NT] = make_uint4(0, 0, 0, 0);
    __syncthreads();
    auto add_if = [&](uint32_t bits, uint32_t v) {
      const uint32_t o = order16(bits);
      if ((o >> 15) == static_cast<uint32_t>(h)) atomicAdd(&c32[o & 0x7FFFu], v);
    };
    for_each_value([&](uint32_t raw) {
      // (a soft-capped row's -inf values are counted under the pattern the
      // -inf counters join: elem_bits(-inf))
      if (raw != NEG_INF_RAW || neg_inf_value) add_if(elem_bits(raw), 1u);
    });
    for_each_unique_id([&](uint32_t raw) {
      const uint32_t z = elem_bits(raw), zp = penalised_bits<D>(z, rp);
      if (zp != z) add_if(zp, 1u);
    });
    __syncthreads();
    for (int k = 0; k < 32; ++k) {
      const int i = tid * 32 + ((k + tid) & 31);  // (staggered: no bank conflicts)
      if (c32[i] > 0xFFFFu) {
        const uint32_t slot = atomicAdd(&sh.n_heavy, 1u);
        if (slot < static_cast<uint32_t>(MAX_HEAVY)) sh.hv_order[slot] = 32768u * h + static_cast<uint32_t>(i);
      }
    }
    __syncthreads();
    for_each_unique_id([&](uint32_t raw) {
      const uint32_t z = elem_bits(raw), zp = penalised_bits<D>(z, rp);
      if (zp != z) add_if(z, 0xFFFFFFFFu);
    });
    __syncthreads();
    if (tid < static_cast<int>(min(sh.n_heavy, static_cast<uint32_t>(MAX_HEAVY))) &&
        (sh.hv_order[tid] >> 15) == static_cast<uint32_t>(h))
      sh.hv_count[tid] = c32[sh.hv_order[tid] & 0x7FFFu];
  }
  __syncthreads();
  if (tid == 0 && sh.n_heavy > static_cast<uint32_t>(MAX_HEAVY)) {  // cannot happen (at most 5 exist)
    sh.n_heavy = MAX_HEAVY;
    atomicOr(&sh.status, FL_ROW_LIMIT);
  }
#pragma unroll
  for (int k = 0; k < 8; ++k) reinterpret_cast<uint4*>(sh.hist)[tid + k * NT] = make_uint4(0, 0, 0, 0);
  __syncthreads();
  for_each_value([&](uint32_t raw) {
    if (raw == NEG_INF_RAW) {  // the -inf values in this lane's counter past the patterns
      atomicAdd(&sh.hist[HIST_WORDS + (tid & (WAVE - 1))], 1u);
      return;
    }
    const uint32_t bits = elem_bits(raw);
    if (!is_heavy(bits)) atomicAdd(&sh.hist[bits >> 1], 1u + (bits & 1u) * 0xFFFFu);
  });
  __syncthreads();
  for_each_unique_id([&](uint32_t raw) {
    const uint32_t z = elem_bits(raw), zp = penalised_bits<D>(z, rp);
    if (zp == z) return;
    // (a soft-capped raw -inf leaves its lane's -inf counter)
    if (neg_inf_value && raw == NEG_INF_RAW) atomicAdd(&sh.hist[HIST_WORDS + (tid & (WAVE - 1))], 0xFFFFFFFFu);
    else if (!is_heavy(z)) atomicAdd(&sh.hist[z >> 1], (z & 1u) ? 0xFFFF0000u : 0xFFFFFFFFu);
    if (!is_heavy(zp)) atomicAdd(&sh.hist[zp >> 1], (zp & 1u) ? 0x10000u : 1u);
  });
  __syncthreads();
  if (tid < static_cast<int>(sh.n_heavy)) {
    const uint32_t P = bits_of_order16(sh.hv_order[tid]);
    const uint32_t c = sh.hv_count[tid], f = min(c, 0xFFFFu);
    atomicAdd(&sh.hist[P >> 1], (P & 1u) ? (f << 16) : f);
    sh.hv_extra[tid] = c - f;
  }
  __syncthreads();
}

}  // namespace

// SC: the row has a soft-cap (applied per element when SC_ELEM, else per
// entry).  The instantiation without it keeps the first read's VGPR tile for
// the identification; the one with it reads the row again.
// HEAVY: the exact-count body -- no register tile, the histogram counted by
// heavy_recount, counts beyond 16 bits kept per pattern.
template <class D, bool SC, bool HEAVY>
__device__ __forceinline__ bool row_body(const fl_sample_args a, const int ALIGNED, const int SC_ELEM_IN,
                                         Shared16& sh) {
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  // (a repeat for the rows a first call left at FL_ROW_LIMIT: the others keep
  // their outputs; block-uniform, before any barrier)
  if constexpr (HEAVY)
    if ((a.flags & FL_FLAG_ONLY_LIMITED) && (a.out_status[b] & FL_ROW_LIMIT) == 0) return true;
  const int V = static_cast<int>(a.vocab);
  const uint16_t* row = static_cast<const uint16_t*>(a.logits) + b * a.ld;
  const bool SC_ELEM = SC && SC_ELEM_IN;
  const int nfull = V >> 3;                               // chunks holding 8 valid elements
  const bool fast_row = !HEAVY && ALIGNED && !SC_ELEM && nfull > 0 && V <= TILE_V;  // whole row through the VGPR tile

  // ------------------------------------------------ loads
  // Issue order matters: the per-row parameters (scalar loads) first, so they
  // do not queue behind 256 KB of row data; then the history ids (prefetched
  // by row stride); then the row, branch-free with clamped addresses, so that
  // waiting for the ids never waits for the row and all loads are in flight
  // together.  The temperature array, always present, stands in for absent
  // arrays so that every load is an unconditional global load.
  const int32_t* dummy = reinterpret_cast<const int32_t*>(a.temperature);
  const bool select = (a.flags & FL_FLAG_NO_SELECT) == 0;
  const float T = a.temperature[b];
  const int K = a.top_k[b];
  const float TP = a.top_p[b];
  const float MP = a.min_p[b];
  const float RP = a.rep_penalty[b];
  const int64_t ub = a.uniform_div > 1 ? b / a.uniform_div : b;  // rows sharing a draw
  const float U_in = (select ? a.uniforms : a.temperature)[select ? ub : b];
  const int H_in = (a.hist_ids ? a.hist_len : dummy)[b];
  __builtin_amdgcn_sched_barrier(0);
  const bool hist_rows = a.hist_ids != nullptr && a.hist_ld > 0;   // one id list per row
  const int32_t* hid = a.hist_ids ? a.hist_ids + b * a.hist_ld : dummy;
  const int32_t* hpre_src = hist_rows ? hid : dummy;
  int32_t hpre[HPRE];
#pragma unroll
  for (int k = 0; k < HPRE; ++k) {
    const int i = tid + k * NT;
    hpre[k] = hpre_src[hist_rows ? min(i, static_cast<int>(a.hist_ld) - 1) : 0];
  }
  // The first EARLY_CHUNKS chunks of the row tile (the whole lookahead
  // window) are requested before the LDS clear, so that the row starts to
  // stream in during it; the rest as the count goes: a wave stalls in issuing
  // its loads until the memory system accepts them (at the HBM rate), so a
  // barrier placed after all of them would only open once most of the row
  // had arrived.  (Two chunks before the clear: 0.5 us slower per launch.)
  const __amdgpu_buffer_rsrc_t rrow = row_rsrc(row, fast_row ? 2u * static_cast<uint32_t>(V) : 0u);
  uint4 d[NCH];
#pragma unroll
  for (int j = 0; j < EARLY_CHUNKS; ++j) {
    d[j] = buf_load16_once(rrow, 16u * tid, 16u * NT * j);
    __builtin_amdgcn_sched_barrier(0);
  }
  // ------------------------------------------------ clear LDS
  // Straight-line stores: a loop here makes the compiler wait for
  // outstanding loads.
  FL_MARK(0);  // (after the parameter loads: a mark before them makes the tuning build spill)
  static_assert(HIST_WORDS == 8 * 4 * NT && HBITS_WORDS == 4 * NT && OWNER_WORDS <= 4 * NT, "LDS clear layout");
#pragma unroll
  for (int k = 0; k < 8; ++k) reinterpret_cast<uint4*>(sh.hist)[tid + k * NT] = make_uint4(0, 0, 0, 0);
  if (tid < WAVE) sh.hist[HIST_WORDS + tid] = 0;
  reinterpret_cast<uint4*>(sh.hbits)[tid] = make_uint4(0, 0, 0, 0);
  if (tid < OWNER_WORDS / 4) reinterpret_cast<uint4*>(sh.owner)[tid] = make_uint4(0, 0, 0, 0);
  static_assert(2 * NSLOT * NWAVE <= NT, "one member counter per thread to clear");
  if (tid < 2 * NSLOT * NWAVE) (&sh.wc[0][0][0])[tid] = 0;
  if (tid == 0) {
    sh.status = 0;
    sh.nh[0] = sh.nh[1] = 0;
    sh.n_heavy = 0;
    sh.result[0] = sh.result[1] = -1;
    sh.dec.L = 0;
    sh.dec.i0 = -1;
    sh.dec.c0 = 0;
    sh.dec.S = sh.dec.SK = 0.0;
    sh.dec.cut_lo = sh.dec.cut_hi = sh.dec.sel_lo = 0;
    sh.dec.sel_hi = -1;
    sh.dec.cut_kept = sh.dec.cut_total = sh.dec.n_kept = sh.dec.sel_rank = 0;
    sh.dec.o_lo[0] = sh.dec.o_lo[1] = sh.dec.o_hi[0] = sh.dec.o_hi[1] = 0;
    sh.dec.y_sel = 0.0f;
    sh.dec.y_cut = __builtin_inff();
  }
  lds_barrier();
  FL_MARK(1);

  // u outside [0, 1) (or NaN) is clamped into it
  const float U = select ? fminf(fmaxf(U_in, 0.0f), 0.99999994f) : 0.0f;
  const float CAP = a.softcap;
  const float RT = T > 0.0f ? recip_rt(T) : 0.0f;  // one IEEE division per row (temperature_val)
  // (H_in is only meaningful with a history: without one it was read from the stand-in array)
  const bool hist_too_long = a.hist_ids != nullptr && H_in > FL_MAX_HISTORY;
  const int H = (a.hist_ids != nullptr && RP != 1.0f && !hist_too_long) ? max(H_in, 0) : 0;
  const bool pen = H > 0;
  // Rows longer than the history bitmap (TILE_V values) de-duplicate their
  // history in two windows of TILE_V ids and keep the full bitmap in the
  // histogram's memory for the identification.
  const bool wide = V > TILE_V;
  const bool sc_entry = SC && (CAP > 0.0f) && !SC_ELEM;
  if (tid == 0 && hist_too_long) atomicOr(&sh.status, FL_ROW_LIMIT);

  // Value pattern of an element as the filters see it before penalty.
  auto elem_bits = [&](uint32_t raw) -> uint32_t {
    return SC_ELEM ? capped_bits<D>(raw, CAP) : raw;
  };

  // ------------------------------------------------ history: unique ids
  // Each id's first claimant owns it and fetches its logit now, so that the
  // load overlaps the counting pass below.
  uint32_t xh[HPRE];
  bool own[HPRE];
  // (window w of a wide row: ids w * TILE_V .. w * TILE_V + TILE_V - 1)
  auto claim = [&](int i, int id, int w) -> bool {
    if (id < 0 || id >= V) {
      if (w == 0) atomicOr(&sh.status, FL_ROW_BAD_HISTORY);
      return false;
    }
    const int bid = id - w * TILE_V;
    if (static_cast<uint32_t>(bid) >= static_cast<uint32_t>(TILE_V)) return false;  // the other window
    const uint32_t bit = 1u << (bid & 31);
    if (atomicOr(&sh.hbits[bid >> 5], bit) & bit) return false;  // a duplicate id
    atomicOr(&sh.owner[i >> 5], 1u << (i & 31));
    return true;
  };
#pragma unroll
  for (int k = 0; k < HPRE; ++k) {
    const int i = tid + k * NT;
    own[k] = !HEAVY && pen && hist_rows && i < H && !wide;
    if (own[k]) own[k] = claim(i, hpre[k], 0);
  }
#pragma unroll
  for (int k = 0; k < HPRE; ++k) xh[k] = row[own[k] ? hpre[k] : 0];

  // ------------------------------------------------ row loads (VGPR tile)
  // Issued after the history gathers: a wave's loads complete in issue order,
  // so the gathered logits arrive ahead of the row's chunks and the penalty
  // moves are made before the counting (moves and counts commute).
  // (unconditional: behind a branch, the compiler's wait for the history ids
  // would also wait for the row on the path that loaded it; a row the fast
  // path does not take gets an empty range, so its loads return zeros)
  // (issued in chunk order, pinned by scheduling barriers: the count pass
  // takes the chunks in that order, and counting a chunk whose load was issued
  // late would hold back the counting of all chunks after it)
#pragma unroll
  for (int j = EARLY_CHUNKS; j < LOOKAHEAD; ++j) {
    d[j] = buf_load16_once(rrow, 16u * tid, 16u * NT * j);
    __builtin_amdgcn_sched_barrier(0);
  }

  // ------------------------------------------------ count patterns
  // Raw -inf values (a masked vocabulary) stay out of the pattern counts,
  // where more than 65535 of them would wrap a 16-bit counter, and go to a
  // 32-bit counter of this lane past the patterns.  Without a soft-cap they
  // are never kept, selected or weighted.  With one they are the value -cap:
  // after the counting they join their pattern's count, the part beyond 16
  // bits kept apart (inf_extra).
  constexpr uint32_t NEG_INF_RAW = 0x8000u | D::INF_BITS;
  const uint32_t inf_word = HIST_WORDS + (tid & (WAVE - 1));
  auto count = [&](uint32_t raw) {
    if constexpr (SC) {
      const uint32_t bits = elem_bits(raw);
      const bool ni = raw == NEG_INF_RAW;
      atomicAdd(&sh.hist[ni ? inf_word : bits >> 1], ni ? 1u : 1u + (bits & 1u) * 0xFFFFu);
    } else {
      // (the -inf pattern is even, so its increment is 1)
      atomicAdd(&sh.hist[raw == NEG_INF_RAW ? inf_word : raw >> 1], 1u + (raw & 1u) * 0xFFFFu);
    }
  };
  // The count of the two patterns of a word w (no -inf or negative NaN among
  // them): pattern p's counter is half p & 1 of word p >> 1, so the byte
  // address is (p << 1) & 0x1FFFC and the increment 1 + (p & 1) * 0xFFFF.
  // Written as instructions (4 VALU per value; the compiler's compare-and-
  // select form takes 7 with the -inf test).
  const uint32_t ffff = 0xFFFFu;
  auto count_pair = [&](uint32_t w) {
    uint32_t a0, a1, i0, i1;
    asm volatile(
        "v_lshlrev_b32 %0, 1, %4\n\t"
        "v_and_b32 %0, 0x1fffc, %0\n\t"
        "v_lshrrev_b32 %1, 15, %4\n\t"
        "v_and_b32 %1, 0x1fffc, %1\n\t"
        "v_and_b32 %2, 1, %4\n\t"
        "v_mad_u32_u24 %2, %2, %5, 1\n\t"
        "v_bfe_u32 %3, %4, 16, 1\n\t"
        "v_mad_u32_u24 %3, %3, %5, 1"
        : "=&v"(a0), "=&v"(a1), "=&v"(i0), "=&v"(i1)
        : "v"(w), "s"(ffff));
    atomicAdd(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(sh.hist) + a0), i0);
    atomicAdd(reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(sh.hist) + a1), i1);
  };
  // a chunk holding -inf or a negative NaN (raw patterns >= the -inf
  // pattern) takes the per-value count: one packed maximum per word
  auto chunk_has_top_patterns = [&](const uint32_t (&w4)[4]) -> bool {
    u16x2 m = __builtin_bit_cast(u16x2, w4[0]);
#pragma unroll
    for (int k = 1; k < 4; ++k) m = __builtin_elementwise_max(m, __builtin_bit_cast(u16x2, w4[k]));
    return max(static_cast<uint32_t>(m.x), static_cast<uint32_t>(m.y)) >= NEG_INF_RAW;
  };
  static_assert(HIST_WORDS * 4 == 0x20000, "pattern byte addresses are 17 bits");
  // ------------------------------------------------ repetition penalty
  // each unique id moves one count from its pattern to its penalised pattern
  auto move = [&](uint32_t raw, uint32_t z, uint32_t zp) {
    if (zp != z) {
      // (a soft-capped raw -inf was counted in this lane's -inf counter)
      if (SC && raw == NEG_INF_RAW) atomicAdd(&sh.hist[inf_word], 0xFFFFFFFFu);
      else atomicAdd(&sh.hist[z >> 1], (z & 1u) ? 0xFFFF0000u : 0xFFFFFFFFu);
      atomicAdd(&sh.hist[zp >> 1], (zp & 1u) ? 0x10000u : 1u);
    }
  };
  auto penalise = [&](uint32_t raw) {
    const uint32_t z = elem_bits(raw);
    move(raw, z, penalised_bits<D>(z, RP));
  };
  // the patterns of the owned prefetched ids, kept for the identification
  // (16 bits each, in one VGPR); their moves are made before the counting
  // (the packed counters add modulo 2^32, so a count taken below zero for a
  // while borrows from its neighbour and repays it: the order of the adds
  // does not matter)
  static_assert(HPRE == 2, "two patterns per word");
  uint32_t hz = 0;
#pragma unroll
  for (int k = 0; k < HPRE; ++k) {
    if (own[k]) {
      const uint32_t z = elem_bits(xh[k]);
      hz |= z << (16 * k);
      move(xh[k], z, penalised_bits<D>(z, RP));
    }
  }
  if constexpr (!HEAVY) {  // (the recounting body counts in heavy_recount)
  if (fast_row) {
    // Software-pipelined: chunk j + LOOKAHEAD is requested as chunk j is
    // counted, so each wave keeps a few chunks in flight and every wave's
    // data arrives spread over the whole stream.  (Requested all at once, the
    // oldest waves' loads are served first and the youngest waves receive
    // their whole tile, and count it, only at the end of the stream.)
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j + LOOKAHEAD < NCH) d[j + LOOKAHEAD] = buf_load16_once(rrow, 16u * tid, 16u * NT * (j + LOOKAHEAD));
      __builtin_amdgcn_sched_barrier(0);
      if (j * NT + tid < nfull) {
        const uint32_t w4[4] = {d[j].x, d[j].y, d[j].z, d[j].w};
        if (SC || chunk_has_top_patterns(w4)) {
#pragma unroll
          for (int e = 0; e < 8; ++e) count((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) count_pair(w4[k]);
        }
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  } else {
#pragma unroll
    for (int j = LOOKAHEAD; j < NCH; ++j) d[j] = make_uint4(0, 0, 0, 0);
    for (int c = tid; c < nfull; c += NT) {
      const uint4 q = load_chunk16(row, c, V, ALIGNED);
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) count((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
    }
  }
  if (tid == 0)
    for (int i = nfull * 8; i < V; ++i) count(row[i]);
  }

  FL_MARK(12);
  // ids past the prefetched ones (and every id of a row past the tile)
  if (!wide) {
    for (int i = tid + ((hist_rows && !HEAVY) ? HPRE * NT : 0); i < H; i += NT) {
      const int id = hid[i];
      if (claim(i, id, 0) && !HEAVY) penalise(row[id]);
    }
  } else if (pen) {
    for (int w = 0; w < 2; ++w) {
      if (w == 1) {  // the second window's ids through a cleared bitmap
        __syncthreads();
        reinterpret_cast<uint4*>(sh.hbits)[tid] = make_uint4(0, 0, 0, 0);
        __syncthreads();
      }
      for (int i = tid; i < H; i += NT) {
        const int id = hid[i];
        if (claim(i, id, w) && !HEAVY) penalise(row[id]);
      }
    }
  }
  __syncthreads();
  // soft-capped rows: the -inf values join the count of their pattern (that of
  // -cap), as far as its 16 bits hold (not at all where -cap is a pattern of
  // more than 65535 values, whose count is exact and includes them)
  uint32_t inf_extra = 0, inf_order = 0xFFFFFFFFu;
  auto merge_neg_inf = [&]() {
    if constexpr (SC) {
      if (tid < WAVE) {
        const uint32_t nin = wave_reduce(sh.hist[HIST_WORDS + tid], OpAdd{});
        if (tid == 0) {
          const uint32_t P = elem_bits(NEG_INF_RAW);
          bool heavy = false;
          for (uint32_t k = 0; k < sh.n_heavy; ++k) heavy |= sh.hv_order[k] == order16(P);
          uint32_t add = 0;
          if (nin != 0u && !heavy) {
            const uint32_t w = sh.hist[P >> 1];
            const uint32_t cur = (P & 1u) ? (w >> 16) : (w & 0xFFFFu);
            add = min(nin, 0xFFFFu - cur);
            sh.hist[P >> 1] = w + ((P & 1u) ? (add << 16) : add);
          }
          sh.inf_extra = heavy ? 0u : nin - add;
        }
      }
      __syncthreads();
      inf_extra = sh.inf_extra;
      inf_order = order16(elem_bits(NEG_INF_RAW));
    }
  };
  // (the recounting body: every count, exact, the penalty's moves included)
  if constexpr (HEAVY) heavy_recount<D>(sh, row, V, nfull, ALIGNED != 0, SC_ELEM, CAP, hid, H, pen, RP);
  merge_neg_inf();

  FL_MARK(2);

  const bool fast = fast_row;
  // ------------------------------------------------ compact to entries
  // Order o = 0 is the largest value.  Step s covers orders 128s .. 128s+127
  // (64 histogram words); wave w takes steps w, w + 16, ..., w + 496, so the
  // few dozen consecutive steps that real logits populate are spread over all
  // waves.  In a step, lane l reads the word of orders 128s + 2l and + 1: the
  // 64 reads hit 64 consecutive words (no bank conflicts).  Entry counts per
  // step go through LDS; each wave scans the 512 counts itself to place its
  // steps' entries.
  int N;
  {
    const int wave = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int lane = tid & (WAVE - 1);
    uint32_t x[SPW];
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      const int s = wave + NWAVE * k;
      if (k < SPW / 2) {
        // positive values (s < 256): the word holds order o + 1 in its low
        // half and o in its high half; swap so the low half is order o
        const uint32_t w = sh.hist[0x3FFF - 64 * s - lane];
        x[k] = __builtin_amdgcn_alignbit(w, w, 16);
      } else {
        x[k] = sh.hist[64 * s + lane];
      }
    }
    // NaN patterns occupy the two ends of the order: the first NAN_STEPS
    // steps (k = 0 of the first waves) and the last (k = SPW - 1 of the last
    // waves).  Drop them and flag the row.
    constexpr int NAN_STEPS = (0x8000 - static_cast<int>(D::INF_BITS) + 127) / 128;
    static_assert(NAN_STEPS <= NWAVE, "NaN steps fit one step per wave");
    bool nan = false;
    if (wave < NAN_STEPS) {
      const uint32_t o = 128u * wave + 2u * lane;
      uint32_t keep = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) keep |= (o + h < 0x7FFFu - D::INF_BITS) ? 0u : (h ? 0xFFFF0000u : 0x0000FFFFu);
      nan |= (x[0] & ~keep) != 0u;
      x[0] &= keep;
    }
    if (wave >= NWAVE - NAN_STEPS) {
      const uint32_t o = 128u * (wave + NWAVE * (SPW - 1)) + 2u * lane;
      uint32_t keep = 0;
#pragma unroll
      for (int h = 0; h < 2; ++h) keep |= (o + h > 0x8000u + D::INF_BITS) ? 0u : (h ? 0xFFFF0000u : 0x0000FFFFu);
      nan |= (x[SPW - 1] & ~keep) != 0u;
      x[SPW - 1] &= keep;
    }
    if (nan) atomicOr(&sh.status, FL_ROW_NAN);
    // entries of step wave + 16k, held by lane k; bit k of `busy` marks a
    // step with entries (wave-uniform)
    uint32_t cv = 0, busy = 0;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      if (__ballot(x[k] != 0u) != 0) {
        const uint32_t c = static_cast<uint32_t>(__popcll(__ballot((x[k] & 0xFFFFu) != 0u)) +
                                                 __popcll(__ballot((x[k] >> 16) != 0u)));
        cv = (lane == k) ? c : cv;
        busy |= 1u << k;
      }
    }
    if (lane < SPW) sh.stepc[wave + NWAVE * lane] = cv;
    __syncthreads();
    // lane l: the counts of steps 8l .. 8l+7.  This wave's steps sit at
    // position wave % 8 of lanes 2k + wave / 8.
    const uint4 s0 = reinterpret_cast<const uint4*>(sh.stepc)[2 * lane];
    const uint4 s1 = reinterpret_cast<const uint4*>(sh.stepc)[2 * lane + 1];
    const uint32_t sc8[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
    const int jw = wave & 7;
    uint32_t lsum = 0, pre = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      pre += (j < jw) ? sc8[j] : 0u;
      lsum += sc8[j];
    }
    const uint32_t linc = wave_incl_scan(lsum);
    const uint32_t start = linc - lsum + pre;  // entries before step 8 * lane + wave % 8
    const uint32_t tot = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(linc), WAVE - 1));
    // branch-free within a step: an empty half writes to this lane's spare
    // slot past the entry area instead of being skipped
    const uint32_t spare = ENT_MAX + 2u * lane;
#pragma unroll
    for (int k = 0; k < SPW; ++k) {
      if (((busy >> k) & 1u) == 0) continue;
      const uint32_t a1 = x[k] & 0xFFFFu, a2 = x[k] >> 16;
      const uint64_t m1 = __ballot(a1 != 0u), m2 = __ballot(a2 != 0u);
      const uint32_t base =
          static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(start), 2 * k + (wave >> 3)));
      const uint32_t below =
          __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m1 >> 32),
                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m1), 0)) +
          __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m2 >> 32),
                                    __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m2), 0));
      const uint32_t o = 128u * static_cast<uint32_t>(wave + NWAVE * k) + 2u * lane;
      const uint32_t p1 = base + below;
      const uint32_t p2 = p1 + (a1 ? 1u : 0u);
      sh.hist[(a1 && p1 < static_cast<uint32_t>(ENT_MAX)) ? p1 : spare] = (o << 16) | a1;
      sh.hist[(a2 && p2 < static_cast<uint32_t>(ENT_MAX)) ? p2 : spare + 1u] = ((o + 1u) << 16) | a2;
    }
    N = static_cast<int>(min(tot, static_cast<uint32_t>(ENT_MAX)));
    if (tid == 0 && tot > static_cast<uint32_t>(ENT_MAX)) atomicOr(&sh.status, FL_ROW_LIMIT);
  }
  __syncthreads();
  FL_MARK(3);

  // ------------------------------------------------ entry values
  // Entry i: order ent[i] >> 16, count ent[i] & 0xFFFF, value Y(i) after
  // soft-cap and temperature, E(i) = exp(Y(i) - M).  Thread t owns the
  // contiguous slice [t*per, t*per + per).  When the row has at most
  // CACHE_MAX entries, Y, E and the exclusive prefix counts and fixed-point
  // masses are kept per entry (any prefix is one read); otherwise values are
  // recomputed and prefixes are a slice-table read plus fewer than `per`
  // terms.
  uint32_t* ent = sh.hist;
  // an entry's count: its 16 bits, and for the -cap entry of a soft-capped
  // row the -inf values beyond them
  const uint32_t n_heavy = sh.n_heavy;
  auto entry_count = [&](uint32_t en) -> uint32_t {
    uint32_t c = en & 0xFFFFu;
    if constexpr (SC) c += (en >> 16) == inf_order ? inf_extra : 0u;
    if constexpr (HEAVY)  // counts beyond 16 bits of the patterns with more than 65535 values
      for (uint32_t k = 0; k < n_heavy; ++k) c += (en >> 16) == sh.hv_order[k] ? sh.hv_extra[k] : 0u;
    return c;
  };
  const bool cached = N <= CACHE_MAX;
  float* Yc = reinterpret_cast<float*>(sh.hist + N);
  float* Ec = reinterpret_cast<float*>(sh.hist + 2 * N);
  uint32_t* Cc = sh.hist + 3 * N;                                         // N + 1 counts
  uint64_t* Cm = reinterpret_cast<uint64_t*>(sh.hist + 4 * N + 2);        // N + 1 masses
  uint32_t* SliceCnt = sh.hist + SLICE_BASE;
  uint64_t* SliceM = reinterpret_cast<uint64_t*>(sh.hist + SLICE_BASE + NT);
  const int per = max(1, (N + NT - 1) / NT);
  const int lo = min(N, tid * per), hi = min(N, lo + per);

  auto cnt_of = [&](int i) -> uint32_t { return entry_count(ent[i]); };
  auto y_raw = [&](int i) -> float { return y_of_order<D, SC>(ent[i] >> 16, CAP, T, RT, sc_entry); };
  const float M = N > 0 ? y_raw(0) : 0.0f;
  // -inf values of the row (read where a total is off or nothing is left)
  auto neg_inf_count = [&]() -> uint32_t {
    uint32_t n = 0;
    for (int l = 0; l < WAVE; ++l) n += sh.hist[HIST_WORDS + l];
    return n;
  };
  if (tid == 0) {
    if (N == 0) sh.status |= neg_inf_count() == static_cast<uint32_t>(V) ? FL_ROW_ALL_MASKED : FL_ROW_NAN;
    else if (isnan(M)) sh.status |= FL_ROW_NAN;
    else if (isinf(M)) sh.status |= (M > 0.0f) ? FL_ROW_INF : FL_ROW_ALL_MASKED;
  }
  auto Y = [&](int i) -> float { return cached ? Yc[i] : y_raw(i); };
  auto E = [&](int i) -> float { return cached ? Ec[i] : exp_of_order<D, SC>(ent[i] >> 16, CAP, T, RT, sc_entry, M); };
  {
    uint32_t lc = 0;
    uint64_t lm = 0;
    for (int i = lo; i < hi; ++i) {
      const uint32_t en = ent[i];
      const float y = y_of_order<D, SC>(en >> 16, CAP, T, RT, sc_entry);
      const float e = expf(y - M);
      if (cached) {
        Yc[i] = y;
        Ec[i] = e;
        Cc[i] = lc;  // prefix within the slice; the slice base is added below
        Cm[i] = lm;
      }
      const uint32_t c = entry_count(en);
      lc += c;
      lm += c * to_fx(e);
    }
    uint32_t ec, tc;
    uint64_t em, tm;
    // (no trailing barrier: sh.redu / sh.redq are next written after the
    // decisions' barriers)
    block_excl_scan2<NWAVE, false>(lc, lm, sh.redu, sh.redq, ec, em, tc, tm);
    SliceCnt[tid] = ec;
    SliceM[tid] = em;
    if (cached) {
      for (int i = lo; i < hi; ++i) {
        Cc[i] += ec;
        Cm[i] += em;
      }
      if (tid == 0) {
        Cc[N] = tc;
        Cm[N] = tm;
      }
    }
    // a total other than V less the -inf values means a 16-bit counter
    // wrapped (> 65535 equal values)
    // (more than 65535 equal values: FL_ROW_LIMIT, sampled by the exact-count kernel)
    if (tid == 0 && tc != static_cast<uint32_t>(V) && tc + neg_inf_count() != static_cast<uint32_t>(V))
      atomicOr(&sh.status, FL_ROW_LIMIT);
  }
  __syncthreads();
  int32_t status = sh.status;
  FL_MARK(4);

  auto count_before = [&](int L) -> uint32_t {  // L in [0, N]
    if (cached) return Cc[L];
    const int s = min(L / per, NT - 1);
    uint32_t c = SliceCnt[s];
    for (int i = s * per; i < L; ++i) c += cnt_of(i);
    return c;
  };
  auto mass_before = [&](int L) -> uint64_t {
    if (cached) return Cm[L];
    const int s = min(L / per, NT - 1);
    uint64_t m = SliceM[s];
    for (int i = s * per; i < L; ++i) m += cnt_of(i) * to_fx(E(i));
    return m;
  };
  const int lane = tid & (WAVE - 1);
  // Entries of equal value Y form a group (several patterns can round to one
  // value).  Y is non-increasing along the entries, so a group is a run; the
  // window of 64 entries next to i settles its bound in one probe unless the
  // run is longer than that.
  auto group_lo = [&](int i, float y) -> int {  // first entry j <= i with Y(j) <= y
    const int w0 = max(0, i - (WAVE - 1));
    const int j = w0 + lane;
    const uint64_t m = __ballot(j <= i && Y(j) <= y);
    if (w0 == 0 || (m & 1ull) == 0) return w0 + __ffsll(static_cast<unsigned long long>(m)) - 1;
    return wave_first(0, w0 + 1, [&](int q) { return Y(q) <= y; });
  };
  auto group_hi = [&](int i, float y) -> int {  // last entry j >= i with Y(j) >= y
    const int j = i + 1 + lane;
    const uint64_t m = __ballot(j < N && Y(j) < y);
    if (m) return i + __ffsll(static_cast<unsigned long long>(m)) - 1;
    if (i + 1 + WAVE >= N) return N - 1;
    return wave_first(i + 1 + WAVE, N, [&](int q) { return Y(q) < y; }) - 1;
  };
  // The serial searches run in wave 0 alone while the other waves wait at a
  // barrier (running them in every wave would starve the younger waves,
  // which the SIMDs schedule after the older ones); their results go through
  // sh.dec.  The scans over many entries use the whole block.
  const bool w0 = tid < WAVE;

  // ---------------- top-k (sampling.py:36-38) and min-p (:40-43): value cuts
  if (status == 0) {
    if (w0) {
      int L = N;
      if (K > 0 && K < V) {
        // first entry whose inclusive count reaches K; every equal value stays
        // (every entry counts at least one value, so the K-th value lies in
        // the first K entries: one probe round for K <= 64)
        const int ik = wave_first(0, min(N, K), [&](int i) { return count_before(i + 1) >= static_cast<uint32_t>(K); });
        // (k beyond the finite values: the k-th largest is -inf, every
        // finite value stays)
        if (ik < N) L = group_hi(ik, Y(ik)) + 1;
      }
      double S = from_fx(mass_before(L));
      if (MP > 0.0f) {
        const float r = 1.0f / static_cast<float>(S);
        const float thr = D::rn(D::rn(r) * MP);
        const int Lm = wave_first(0, L, [&](int i) { return D::rn(E(i) * r) < thr; });
        if (Lm < L) {
          L = Lm;
          S = from_fx(mass_before(L));
        }
      }
      if (tid == 0) {
        sh.dec.L = L;
        sh.dec.S = S;
      }
    }
    __syncthreads();
  }
  const int L = sh.dec.L;
  if (status == 0 && L <= 0) status |= FL_ROW_ALL_MASKED;
  FL_MARK(5);

  // ---------------- top-p (sampling.py:45-51)
  // Position j (descending order) is removed when
  //   round(round_f32(C_j) - p_j) >= round(top_p)
  // with C_j the inclusive cumulative of the rounded probabilities.  The
  // predicate is monotone along the order, so the kept set is a prefix: a
  // block scan finds the first removed entry (tested on its first member),
  // then wave 0 counts the kept members of the entry before it.
  if (status == 0) {
    const double S = sh.dec.S;
    int i0 = L - 1;
    uint32_t c0 = cnt_of(L - 1);
    const float r1 = 1.0f / static_cast<float>(S);
    const float t = D::rn(TP);
    auto pf = [&](int i) -> uint64_t { return to_fx(D::rn(E(i) * r1)); };
    auto removed = [&](uint64_t c_incl, float p) {
      return D::rn(D::rn(static_cast<float>(from_fx(c_incl))) - p) >= t;
    };
    const bool top_p = TP > 0.0f && TP < 1.0f;
    ScanHit h = {L, 0ull, 0ull};
    if (top_p)
      h = scan_first(sh, L, false, 0ull, [&](int i) { return cnt_of(i) * pf(i); },
                     [&](int i, uint64_t ex, uint64_t) { return removed(ex + pf(i), D::rn(E(i) * r1)); });
    FL_MARK(15);
    if (w0) {
      if (top_p && h.idx == 0) {
        i0 = -1;
      } else if (top_p) {
        // the entry before the first removed one (the last entry when none
        // is removed) may lose its later members
        i0 = h.idx - 1;
        const float p = D::rn(E(i0) * r1);
        const uint64_t pfi = to_fx(p);
        const uint64_t c = h.excl - cnt_of(i0) * pfi;  // p-mass before entry i0 (h.excl: before entry idx)
        // member j of entry i0 is removed iff removed(c + (j+1) pf, p); member
        // 0 survives (entry i0 is not removed)
        c0 = static_cast<uint32_t>(wave_first(1, static_cast<int>(cnt_of(i0)), [&](int j) {
          return removed(c + static_cast<uint64_t>(j + 1) * pfi, p);
        }));
      }
      // the group of the cut value, the kept count and the kept mass (:58)
      if (i0 >= 0) {
        const float ycut = Y(i0);
        const int cut_lo = group_lo(i0, ycut);
        const int cut_hi = group_hi(i0, ycut);
        const uint32_t n_before_i0 = count_before(i0);
        const uint32_t n_before_lo = count_before(cut_lo);
        const double SK = from_fx(mass_before(i0) + c0 * to_fx(E(i0)));
        const uint32_t cut_total = count_before(cut_hi + 1) - n_before_lo;
        if (tid == 0) {
          sh.dec.cut_total = cut_total;
          sh.dec.cut_kept = n_before_i0 - n_before_lo + c0;
          sh.dec.cut_lo = cut_lo;
          sh.dec.cut_hi = cut_hi;
          sh.dec.n_kept = n_before_i0 + c0;
          sh.dec.SK = SK;
          sh.dec.y_cut = ycut;
          sh.dec.o_lo[1] = ent[cut_lo] >> 16;
          sh.dec.o_hi[1] = ent[cut_hi] >> 16;
        }
      }
      if (tid == 0) {
        sh.dec.i0 = i0;
        sh.dec.c0 = c0;
      }
    }
    FL_MARK(16);
    __syncthreads();
  }
  const int i0 = sh.dec.i0;
  const uint32_t c0 = sh.dec.c0;
  if (status == 0 && i0 < 0) status |= FL_ROW_ALL_MASKED;
  const double SK = sh.dec.SK;
  const float rK = 1.0f / static_cast<float>(SK);
  const uint32_t n_kept = sh.dec.n_kept;
  const uint32_t cut_kept = sh.dec.cut_kept, cut_total = sh.dec.cut_total;
  const float y_cut = status == 0 ? sh.dec.y_cut : __builtin_inff();

  // ---------------- selection (:59-61)
  auto kc = [&](int i) -> uint32_t { return i < i0 ? cnt_of(i) : (i == i0 ? c0 : 0u); };
  auto kept_before = [&](int Lb) -> uint32_t { return Lb <= i0 ? count_before(Lb) : n_kept; };
  const bool want_sel = select && status == 0;
  if (want_sel) {
    if (T <= 0.0f) {
      // greedy (sampling.py:59-60): first index among the maximal probabilities
      if (w0) {
        const float qmax = D::rn(E(0) * rK);
        const int last = wave_first(1, i0 + 1, [&](int i) { return D::rn(E(i) * rK) != qmax; }) - 1;
        const int sh_hi = group_hi(last, Y(last));
        if (tid == 0) {
          sh.dec.sel_rank = 0;
          sh.dec.y_sel = Y(0);
          sh.dec.o_lo[0] = ent[0] >> 16;
          sh.dec.o_hi[0] = ent[sh_hi] >> 16;
        }
      }
    } else {
      // inverse CDF (CONVENTION replacing torch.multinomial, sampling.py:61):
      // first member whose inclusive cumulative probability exceeds u * total,
      // cumulative sums in exact 2^-45 fixed point
      auto qf = [&](int i) -> uint64_t { return to_fx(D::rn(E(i) * rK)); };
      const int n = i0 + 1;
      uint64_t Q = 0;
      if (n > NT) {  // several scan rounds: the total first
        uint64_t local = 0;
        for (int i = tid; i < n; i += NT) local += kc(i) * qf(i);
        Q = block_reduce(local, OpAdd(), sh.redq);
      }
      auto target_of = [&](uint64_t q) { return __double2ull_rd(static_cast<double>(U) * static_cast<double>(q)); };
      const ScanHit h = scan_first(sh, n, n > NT, Q, [&](int i) { return kc(i) * qf(i); },
                                   [&](int i, uint64_t ex, uint64_t tq) { return ex + kc(i) * qf(i) > target_of(tq); });
      FL_MARK(17);
      if (w0) {
        const uint64_t target = target_of(h.total);
        int is = h.idx;
        uint64_t ex = h.excl;
        if (is > i0) {  // no positive mass at all (every kept probability rounds to zero)
          is = 0;
          ex = 0;
        }
        const float ys = Y(is);
        const int s_lo = group_lo(is, ys), s_hi = group_hi(is, ys);
        // q-mass before the group: the scan's prefix at `is` less the group's
        // entries before it
        uint64_t inner = 0;
        for (int j = s_lo + lane; j < is; j += WAVE) inner += kc(j) * qf(j);
        const uint64_t cg = ex - readlane64(wave_incl_scan(inner), WAVE - 1);
        const uint64_t q = qf(is);
        const uint32_t kept_g = kept_before(s_hi + 1) - kept_before(s_lo);
        // member r of the group covers [cg + r q, cg + (r+1) q): r is the
        // floor of (target - cg) / q, both below 2^53 (exact as doubles); the
        // rounded quotient is at most one above the floor
        uint64_t r = 0;
        if (q > 0 && target >= cg) {
          const uint64_t num = target - cg;
          r = static_cast<uint64_t>(static_cast<double>(num) / static_cast<double>(q));
          if (r * q > num) --r;
        }
        if (tid == 0) {
          sh.dec.sel_rank = static_cast<uint32_t>(min(r, static_cast<uint64_t>(kept_g > 0 ? kept_g - 1 : 0)));
          sh.dec.y_sel = ys;
          sh.dec.o_lo[0] = ent[s_lo] >> 16;
          sh.dec.o_hi[0] = ent[s_hi] >> 16;
        }
      }
    }
  }
  FL_MARK(6);

  // ------------------------------------------------ identification
  // Targets: 0 = selected token (group sel, rank sel_rank); 1 = last kept
  // member of a partially kept group (for the descriptor's idx_cut).
  const bool want_cut = (a.out_desc != nullptr) && status == 0 && cut_kept < cut_total;
  float y_sel = 0.0f;
  if (want_sel || want_cut) {
    // The row tile: the first read, still in VGPRs, or (soft-cap kernel,
    // whose calls keep it from staying there) the row read again.  A re-read
    // is issued here, not during the decisions: a wave stalls issuing loads
    // while the memory system is backed up, which would stall the search wave.
    uint4 r[NCH];
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if constexpr (SC) r[j] = fast ? buf_load16(rrow, 16u * tid, 16u * NT * j) : make_uint4(0, 0, 0, 0);
      else if constexpr (!HEAVY) r[j] = d[j];
      else r[j] = make_uint4(0, 0, 0, 0);
    }
    lds_barrier();  // the decisions are in sh.dec; the entries may be overwritten
    FL_MARK(13);
    y_sel = sh.dec.y_sel;
    // (wave-uniform values: kept in SGPRs, the VGPRs hold the tile)
    auto uni = [](uint32_t v) { return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(static_cast<int>(v))); };
    const uint32_t o_lo[2] = {uni(sh.dec.o_lo[0]), uni(sh.dec.o_lo[1])};
    const uint32_t o_hi[2] = {uni(sh.dec.o_hi[0]), uni(sh.dec.o_hi[1])};
    const uint32_t rank[2] = {uni(sh.dec.sel_rank), uni(cut_kept - 1)};
    const bool active[2] = {want_sel, want_cut};
    // Members of a target, in the order of the convention (ascending
    // vocabulary index), which is also the order of the tile: element e of
    // chunk j * NT + tid has index (j * NT + tid) * 8 + e, so indices go by
    // (j, tid, e).  History ids are members by their penalised value (their
    // owners test them and list them); other elements by their pattern.
    // Every chunk's members are counted (branch-free, packed), giving the
    // members of each slot j (chunks j * NT .. j * NT + NT - 1); only in the
    // slot of rank r do the threads form their members, and a block scan
    // picks the one of rank r.
    uint32_t* hlist[2] = {sh.hist, sh.hist + HLIST_CAP};
    // The history bitmap: sh.hbits, or for a row past TILE_V (whose
    // de-duplication used two windows of it) every id's bit, set here in the
    // histogram's memory past the two member lists.
    uint32_t* hb = sh.hbits;
    if (pen && wide) {
      hb = sh.hist + 2 * HLIST_CAP;
      static_assert(2 * HLIST_CAP + FL_MAX_VOCAB_16 / 32 <= HIST_WORDS, "the full history bitmap fits");
      for (int i = tid; i < FL_MAX_VOCAB_16 / 32; i += NT) hb[i] = 0u;
      __syncthreads();
      for (int i = tid; i < H; i += NT) {
        const int id = hid[i];
        if (id >= 0 && id < V) atomicOr(&hb[id >> 5], 1u << (id & 31));
      }
      __syncthreads();
    }
    auto in_range = [&](int t, uint32_t bits) { return order16(bits) - o_lo[t] <= o_hi[t] - o_lo[t]; };
    auto is_hist = [&](int idx) { return pen && ((hb[idx >> 5] >> (idx & 31)) & 1u); };
    auto push = [&](int t, int idx) {
      const uint32_t s = atomicAdd(&sh.nh[t], 1u);
      if (s < static_cast<uint32_t>(HLIST_CAP)) hlist[t][s] = idx;
    };
    // non-history members of chunk c (8 patterns in q): bit e for element e
    auto chunk_mask = [&](int t, int c, const uint4 q) -> uint32_t {
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
      uint32_t m = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) m |= in_range(t, elem_bits((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu)) ? (1u << e) : 0u;
      const int nv = V - c * 8;
      uint32_t valid = nv >= 8 ? 0xFFu : (nv > 0 ? (1u << nv) - 1u : 0u);
      if (pen) valid &= ~(hb[c >> 2] >> ((c & 3) * 8));
      return m & valid;
    };
    const int nchunks = (V + 7) >> 3;
    // Raw patterns of the targets as at most four ranges (a range across zero
    // splits into its positive and negative parts); slots 2t, 2t+1 belong to
    // target t (fixed slots keep the arrays in registers).  Range r covers
    // patterns rlo[r] .. rlo[r] + rw[r].
    uint32_t rlo[4] = {0, 0, 0, 0}, rw[4] = {0, 0, 0, 0};
    bool ren[4] = {false, false, false, false};
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (!active[t]) continue;
      if (o_hi[t] < 0x8000u) {
        rlo[2 * t] = 0x7FFFu - o_hi[t], rw[2 * t] = o_hi[t] - o_lo[t], ren[2 * t] = true;
      } else if (o_lo[t] >= 0x8000u) {
        rlo[2 * t] = o_lo[t], rw[2 * t] = o_hi[t] - o_lo[t], ren[2 * t] = true;
      } else {
        rlo[2 * t] = 0u, rw[2 * t] = 0x7FFFu - o_lo[t], ren[2 * t] = true;
        rlo[2 * t + 1] = 0x8000u, rw[2 * t + 1] = o_hi[t] - 0x8000u, ren[2 * t + 1] = true;
      }
    }
    // Members per slot j and wave w (chunks j * NT + 64 w .. + 63).  For a
    // word of two patterns, e = max(w - lo - width, 0) per half (wrapping
    // subtraction, then a clamped one) is zero exactly for a member; the
    // minimum over the chunk's words and both ranges flags a chunk holding
    // any.  Chunks rarely hold one, so the exact count (min(e, 1) summed over
    // the halves counts the non-members) runs only where a lane of the wave
    // has a flagged chunk.  (Written as instructions: the compiler would turn
    // the packed arithmetic back into compares.)
    const int wv = __builtin_amdgcn_readfirstlane(tid / WAVE);
    const int lane_id = tid & (WAVE - 1);
    // the partial chunk (V not a multiple of 8): its zero padding reads as
    // the pattern of +0.0
    const int pad = (nfull < nchunks) ? 8 - (V - nfull * 8) : 0;
    const uint32_t ones2 = 0x00010001u;
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (!active[t]) continue;
      const int zero_in = __builtin_amdgcn_readfirstlane(in_range(t, 0u) ? 1 : 0);
      if (fast) {
#pragma unroll
        for (int j = 0; j < NCH; ++j) {
          const uint32_t w4[4] = {r[j].x, r[j].y, r[j].z, r[j].w};
          uint32_t m[4];
          {
            const uint32_t lo2 = rlo[2 * t] * 0x10001u, wd2 = rw[2 * t] * 0x10001u;
#pragma unroll
            for (int k = 0; k < 4; ++k)
              asm("v_pk_sub_u16 %0, %1, %2\n\t"
                  "v_pk_sub_u16 %0, %0, %3 clamp"
                  : "=&v"(m[k])
                  : "v"(w4[k]), "s"(lo2), "s"(wd2));
          }
          if (ren[2 * t + 1]) {  // wave-uniform: a range across zero has a second part
            const uint32_t lo2 = rlo[2 * t + 1] * 0x10001u, wd2 = rw[2 * t + 1] * 0x10001u;
#pragma unroll
            for (int k = 0; k < 4; ++k) {
              uint32_t e;
              asm("v_pk_sub_u16 %0, %1, %2\n\t"
                  "v_pk_sub_u16 %0, %0, %3 clamp\n\t"
                  "v_pk_min_u16 %0, %0, %4"
                  : "=&v"(e)
                  : "v"(w4[k]), "s"(lo2), "s"(wd2), "v"(m[k]));
              m[k] = e;
            }
          }
          uint32_t mm, m23;
          asm("v_pk_min_u16 %0, %1, %2" : "=v"(mm) : "v"(m[0]), "v"(m[1]));
          asm("v_pk_min_u16 %0, %1, %2" : "=v"(m23) : "v"(m[2]), "v"(m[3]));
          asm("v_pk_min_u16 %0, %0, %1" : "+v"(mm) : "v"(m23));
          // (lanes past the row hold zeros: flagged only if +0.0 is a target)
          if (__ballot(static_cast<uint16_t>(mm) == 0u || mm < 0x10000u) != 0ull) {  // wave-uniform
            uint32_t f0, f1, f2, f3;
            asm("v_pk_min_u16 %0, %1, %2" : "=v"(f0) : "v"(m[0]), "s"(ones2));
            asm("v_pk_min_u16 %0, %1, %2" : "=v"(f1) : "v"(m[1]), "s"(ones2));
            asm("v_pk_min_u16 %0, %1, %2" : "=v"(f2) : "v"(m[2]), "s"(ones2));
            asm("v_pk_min_u16 %0, %1, %2" : "=v"(f3) : "v"(m[3]), "s"(ones2));
            const uint32_t nm = f0 + f1 + f2 + f3;  // halves at most 4: no carry between them
            const uint32_t cj = 8u - ((nm & 0xFFFFu) + (nm >> 16));
            if (cj) atomicAdd(&sh.wc[t][j][wv], cj);
          }
        }
        // +0.0 a target: take back the zeros of the padding and of the lanes
        // past the row
        if (zero_in && lane_id == 0) {
#pragma unroll
          for (int j = 0; j < NCH; ++j) {
            const int c0 = j * NT + wv * WAVE;
            uint32_t extra = 8u * static_cast<uint32_t>(min(WAVE, max(0, c0 + WAVE - nchunks)));
            if (pad > 0 && nfull >= c0 && nfull < c0 + WAVE) extra += static_cast<uint32_t>(pad);
            if (extra) atomicAdd(&sh.wc[t][j][wv], 0u - extra);
          }
        }
      } else {
        for (int j = 0; j < NSLOT; ++j) {
          const int c = j * NT + tid;
          if (c >= nchunks) break;
          const uint32_t cj = static_cast<uint32_t>(__popc(chunk_mask(t, c, load_chunk16(row, c, V, ALIGNED))));
          if (cj) atomicAdd(&sh.wc[t][j][wv], cj);
        }
      }
    }
    FL_MARK(14);
    // history elements whose penalised value lies in a target group
    if (pen) {
      auto hist_candidate = [&](int id, uint32_t z, uint32_t zp) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (!active[t]) continue;
          const bool mem = in_range(t, zp);
          // the packed count of the fast path took the id by its raw pattern
          const int corr = (mem ? 1 : 0) - ((fast && in_range(t, z)) ? 1 : 0);
          if (corr != 0) atomicAdd(&sh.wc[t][(id >> 3) / NT][((id >> 3) % NT) / WAVE], static_cast<uint32_t>(corr));
          if (mem) push(t, id);
        }
      };
#pragma unroll
      for (int k = 0; k < HPRE; ++k)
        if (own[k]) {
          const uint32_t z = (hz >> (16 * k)) & 0xFFFFu;
          hist_candidate(hpre[k], z, penalised_bits<D>(z, RP));
        }
      // (wide rows claimed every id in the windowed pass: none was prefetched)
      for (int i = tid + ((hist_rows && !wide && !HEAVY) ? HPRE * NT : 0); i < H; i += NT) {
        if (!((sh.owner[i >> 5] >> (i & 31)) & 1u)) continue;
        const int id = hid[i];
        const uint32_t z = elem_bits(row[id]);
        hist_candidate(id, z, penalised_bits<D>(z, RP));
      }
    }
    FL_MARK(10);
    __syncthreads();
    FL_MARK(7);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (!active[t]) continue;
      const uint32_t n = sh.nh[t];
      if (n <= static_cast<uint32_t>(HLIST_CAP)) {
        // The (slot, wave) holding rank r, found by every wave alike: lane l
        // reads the counts of slot l / 4, waves 4 (l % 4) .. + 3 (16 slots a
        // round, the second round only for rows past TILE_V), which puts the
        // lanes in index order; an inclusive scan over the lanes finds the
        // lane, four compares the wave.  That wave alone then forms its
        // lanes' members in the slot (the chunk's non-history members and the
        // listed history members in the chunk) and scans them.
        static_assert(NCH * NWAVE == 4 * WAVE && NSLOT % NCH == 0, "four counters per lane, NCH slots a round");
        int ws = -1, js = 0;
        uint32_t rr = rank[t];
        for (int j0 = 0; j0 < NSLOT && ws < 0 && j0 * NT * 8 < V; j0 += NCH) {
          const uint4 q4 = reinterpret_cast<const uint4*>(&sh.wc[t][j0][0])[lane_id];
          const uint32_t s4 = q4.x + q4.y + q4.z + q4.w;
          const uint32_t inc = wave_incl_scan(s4);
          const uint64_t hit = __ballot(inc > rr);
          if (hit == 0ull) {  // the same in every wave
            rr -= static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(inc), WAVE - 1));
            continue;
          }
          const int L = __ffsll(static_cast<unsigned long long>(hit)) - 1;
          rr -= static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(inc - s4), L));
          const uint32_t qc[4] = {static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(q4.x), L)),
                                  static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(q4.y), L)),
                                  static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(q4.z), L)),
                                  static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(q4.w), L))};
          int kq = 0;
          while (kq < 3 && rr >= qc[kq]) rr -= qc[kq++];
          ws = 4 * (L & 3) + kq;
          js = j0 + (L >> 2);
        }
        {
          if (wv == ws) {
            const int c = js * NT + tid;
            uint32_t b = 0;
            if (c < nchunks) {
              uint4 q = make_uint4(0, 0, 0, 0);
              if (fast) {
#pragma unroll
                for (int j = 0; j < NCH; ++j)
                  if (j == js) q = r[j];  // js is wave-uniform
              } else {
                q = load_chunk16(row, c, V, ALIGNED);
              }
              b = chunk_mask(t, c, q);
            }
            for (uint32_t k = 0; k < n; ++k) {
              const int id = static_cast<int>(hlist[t][k]);
              if ((id >> 3) == c) b |= 1u << (id & 7);
            }
            const uint32_t cb = static_cast<uint32_t>(__popc(b));
            const uint32_t ex = wave_incl_scan(cb) - cb;
            if (ex <= rr && rr < ex + cb) {
              uint32_t m = b;
              for (uint32_t q = ex; q < rr; ++q) m &= m - 1u;  // drop the lower members
              sh.result[t] = c * 8 + (__ffs(m) - 1);
            }
          }
        }
      } else {
        // the history member list overflowed: count members round by round
        // in index order (re-reads the row from memory; a rare path)
        uint32_t base = 0;
        for (int j = 0; j < NSLOT && j * NT * 8 < V; ++j) {
          const int e0 = (j * NT + tid) * 8;
          uint32_t m = 0;
          for (int e = 0; e < 8; ++e) {
            const int idx = e0 + e;
            if (idx >= V) continue;
            uint32_t bits = elem_bits(row[idx]);
            if (is_hist(idx)) bits = penalised_bits<D>(bits, RP);
            m |= static_cast<uint32_t>(in_range(t, bits)) << e;
          }
          uint32_t tot;
          const uint32_t ex = block_excl_scan<uint32_t>(static_cast<uint32_t>(__popc(m)), sh.redu, &tot);
          if (base + ex <= rank[t] && rank[t] < base + ex + __popc(m)) {
            uint32_t need = rank[t] - base - ex;
            for (int e = 0; e < 8; ++e) {
              if ((m >> e) & 1u) {
                if (need == 0) { sh.result[t] = e0 + e; break; }
                --need;
              }
            }
          }
          base += tot;
          if (base > rank[t]) break;
        }
      }
      __syncthreads();
    }
  }
  FL_MARK(8);

  // ------------------------------------------------ outputs
  FL_MARK(9);
  if (tid == 0) {
    int64_t tok = -1;
    if (want_sel) {
      tok = sh.result[0];
      if (tok < 0) status |= FL_ROW_LIMIT;
    }
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
      // log_softmax(filtered)[tok] as torch evaluates it on a 16-bit tensor
      // (sampling.py:97-98): the kept mass and its log each rounded to the
      // dtype, then y - max - log, rounded
      if (tok >= 0) lp = D::rn((y_sel - M) - D::rn(logf(D::rn(static_cast<float>(SK)))));
      a.out_logprob[b] = lp;
    }
    if ((a.flags & FL_FLAG_APPEND_HISTORY) && hist_rows && tok >= 0 && !was_finished && H_in >= 0 &&
        H_in < a.hist_ld) {
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
        dsc.y_cut = y_cut;
        dsc.idx_cut = (cut_kept < cut_total) ? sh.result[1] : 0x7FFFFFFF;
        dsc.n_kept = static_cast<int32_t>(n_kept);
      } else {
        dsc.y_cut = __builtin_inff();
        dsc.idx_cut = -1;
        dsc.n_kept = 0;
      }
      a.out_desc[b] = dsc;
    }
  }
  return true;
}

// The row sampler.  A row with more than 65535 equal values (a wrapped
// 16-bit counter, seen by the entry pass) reports FL_ROW_LIMIT; the
// exact-count kernel (FL_FLAG_EXACT_COUNTS) samples it.  (The exact body in
// this kernel, even never run, costs every row ~6 us: the register
// allocation of the common path gets worse.)
template <class D, bool SC>
__global__ __launch_bounds__(NT) void k_sample_rows16(const fl_sample_args a, const int ALIGNED, const int SC_ELEM_IN) {
  __shared__ Shared16 sh;
  FL_MARK(11);  // (kernel entry)
  row_body<D, SC, false>(a, ALIGNED, SC_ELEM_IN, sh);
}

template <class D, bool SC>
__global__ __launch_bounds__(NT) void k_sample_rows16_exact(const fl_sample_args a, const int ALIGNED,
                                                            const int SC_ELEM_IN) {
  __shared__ Shared16 sh;
  row_body<D, SC, true>(a, ALIGNED, SC_ELEM_IN, sh);
}

// ------------------------------------------------------------------ launch
hipError_t launch_sample_rows16(const fl_sample_args& a, hipStream_t s) {
  const int aligned = (reinterpret_cast<uintptr_t>(a.logits) % 16 == 0) && ((a.ld * 2) % 16 == 0);
  const bool has_pen = a.rep_penalty != nullptr && a.hist_ids != nullptr && a.hist_len != nullptr;
  const int sc_elem = (a.softcap > 0.0f && has_pen) ? 1 : 0;
  const dim3 grid(static_cast<unsigned>(a.batch)), block(NT);
  const bool sc = a.softcap > 0.0f;
  const bool exact = (a.flags & FL_FLAG_EXACT_COUNTS) != 0;
  if (a.dtype == FL_DTYPE_BF16) {
    if (exact) {
      if (sc) hipLaunchKernelGGL((k_sample_rows16_exact<BF16, true>), grid, block, 0, s, a, aligned, sc_elem);
      else hipLaunchKernelGGL((k_sample_rows16_exact<BF16, false>), grid, block, 0, s, a, aligned, sc_elem);
    } else {
      if (sc) hipLaunchKernelGGL((k_sample_rows16<BF16, true>), grid, block, 0, s, a, aligned, sc_elem);
      else hipLaunchKernelGGL((k_sample_rows16<BF16, false>), grid, block, 0, s, a, aligned, sc_elem);
    }
  } else {
    if (exact) {
      if (sc) hipLaunchKernelGGL((k_sample_rows16_exact<F16, true>), grid, block, 0, s, a, aligned, sc_elem);
      else hipLaunchKernelGGL((k_sample_rows16_exact<F16, false>), grid, block, 0, s, a, aligned, sc_elem);
    } else {
      if (sc) hipLaunchKernelGGL((k_sample_rows16<F16, true>), grid, block, 0, s, a, aligned, sc_elem);
      else hipLaunchKernelGGL((k_sample_rows16<F16, false>), grid, block, 0, s, a, aligned, sc_elem);
    }
  }
  return hipGetLastError();
}

}  // namespace fl

#ifdef FL_PHASE_TIMES
// Tuning builds only: copy the phase timestamps recorded by the last launch.
extern "C" int fl_debug_phase_ts(uint64_t* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(fl_phase_ts), sizeof(uint64_t) * FL_PHASE_SLOTS, 0,
                             hipMemcpyDeviceToHost) ==
                 hipSuccess ? 0 : -1;
}
#endif
