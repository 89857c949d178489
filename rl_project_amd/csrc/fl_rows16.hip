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
#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {

namespace {

constexpr int NCH = 16;                          // 16-byte chunks per thread
constexpr int HIST_WORDS = 32768;                // 65536 packed u16 counters
constexpr int HBITS_WORDS = FL_MAX_VOCAB_16 / 32;
constexpr int OWNER_WORDS = FL_MAX_HISTORY / 32;
constexpr int LIST_CAP = 3 * HIST_WORDS / 8;     // candidates per identification target
constexpr int HIT_CAP = HIST_WORDS / 4;          // queued chunks with a candidate (after the two lists)
constexpr int ENTRY_CACHE_MAX = HIST_WORDS / 3;  // entries whose y and e fit beside the list
constexpr int RANK_SELECT_MAX = 2048;            // candidates ranked by all-pairs counting
constexpr int HPRE = 2;                          // history ids per thread loaded ahead of the row

static_assert(NCH * NT * 8 == FL_MAX_VOCAB_16, "one VGPR tile holds the largest 16-bit row");

struct Shared16 {
  uint32_t hist[HIST_WORDS];
  uint32_t hbits[HBITS_WORDS];
  uint32_t owner[OWNER_WORDS];
  double redd[NWAVE];
  uint64_t redq[NWAVE];
  uint32_t redu[NWAVE];
  uint32_t redi_u[NWAVE];
  int32_t redi[NWAVE];
  int32_t status;
  int32_t n_entries;
  int32_t ik, lk;
  int32_t i0;
  uint32_t c0;
  int32_t sel_entry;
  uint64_t sel_cexcl;
  int32_t result[2];
  uint32_t nlist[2];
  uint32_t nhit;
};

typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));

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

}  // namespace

template <class D>
__global__ __launch_bounds__(NT) void k_sample_rows16(const fl_sample_args a, const int ALIGNED, const int SC_ELEM) {
  __shared__ Shared16 sh;
  FL_MARK(0);
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int V = static_cast<int>(a.vocab);
  const uint16_t* row = static_cast<const uint16_t*>(a.logits) + b * a.ld;
  const int nfull = V >> 3;                               // chunks holding 8 valid elements
  const bool fast = ALIGNED && !SC_ELEM && nfull > 0;     // whole row through the VGPR tile

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
  const float U_in = (select ? a.uniforms : a.temperature)[b];
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
  // ------------------------------------------------ clear LDS
  // Before the row loads: a wave stalls in issuing its loads until the memory
  // system accepts them (at the HBM rate), so a barrier placed after them
  // would only open once the whole row had arrived.  Straight-line stores: a
  // loop here makes the compiler wait for outstanding loads.
  FL_MARK(10);
  static_assert(HIST_WORDS == 8 * 4 * NT && HBITS_WORDS == 4 * NT && OWNER_WORDS <= 4 * NT, "LDS clear layout");
#pragma unroll
  for (int k = 0; k < 8; ++k) reinterpret_cast<uint4*>(sh.hist)[tid + k * NT] = make_uint4(0, 0, 0, 0);
  reinterpret_cast<uint4*>(sh.hbits)[tid] = make_uint4(0, 0, 0, 0);
  if (tid < OWNER_WORDS / 4) reinterpret_cast<uint4*>(sh.owner)[tid] = make_uint4(0, 0, 0, 0);
  if (tid == 0) {
    sh.status = 0;
    sh.nlist[0] = sh.nlist[1] = 0;
    sh.nhit = 0;
    sh.result[0] = sh.result[1] = -1;
    sh.ik = 0;
    sh.lk = 0;
  }
  lds_barrier();
  FL_MARK(1);

  // ------------------------------------------------ row loads (VGPR tile)
  // (unconditional: behind a branch, the compiler's wait for the history ids
  // would also wait for the row on the path that loaded it; a row the fast
  // path does not take gets an empty range, so its loads return zeros)
  const __amdgpu_buffer_rsrc_t rrow = row_rsrc(row, fast ? 2u * static_cast<uint32_t>(V) : 0u);
  uint4 d[NCH];
#pragma unroll
  for (int j = 0; j < NCH; ++j) d[j] = buf_load16(rrow, 16u * tid, 16u * NT * j);

  // u outside [0, 1) (or NaN) is clamped into it
  const float U = select ? fminf(fmaxf(U_in, 0.0f), 0.99999994f) : 0.0f;
  const float CAP = a.softcap;
  const bool hist_too_long = H_in > FL_MAX_HISTORY;
  const int H = (a.hist_ids != nullptr && RP != 1.0f && !hist_too_long) ? max(H_in, 0) : 0;
  const bool pen = H > 0;
  const bool sc_entry = (CAP > 0.0f) && !SC_ELEM;
  if (tid == 0 && hist_too_long) atomicOr(&sh.status, FL_ROW_LIMIT);

  // Value pattern of an element as the filters see it before penalty.
  auto elem_bits = [&](uint32_t raw) -> uint32_t {
    return SC_ELEM ? D::from_f32(softcap_val<D>(D::to_f32(raw), CAP)) : raw;
  };

  // ------------------------------------------------ history: unique ids
  // Each id's first claimant owns it and fetches its logit now, so that the
  // load overlaps the counting pass below.
  uint32_t xh[HPRE];
  bool own[HPRE];
  auto claim = [&](int i, int id) -> bool {
    if (id < 0 || id >= V) {
      atomicOr(&sh.status, FL_ROW_BAD_HISTORY);
      return false;
    }
    const uint32_t bit = 1u << (id & 31);
    if (atomicOr(&sh.hbits[id >> 5], bit) & bit) return false;  // a duplicate id
    atomicOr(&sh.owner[i >> 5], 1u << (i & 31));
    return true;
  };
#pragma unroll
  for (int k = 0; k < HPRE; ++k) {
    const int i = tid + k * NT;
    own[k] = pen && hist_rows && i < H;
    if (own[k]) own[k] = claim(i, hpre[k]);
  }
#pragma unroll
  for (int k = 0; k < HPRE; ++k) xh[k] = row[own[k] ? hpre[k] : 0];

  // ------------------------------------------------ count patterns
  auto count = [&](uint32_t bits) { atomicAdd(&sh.hist[bits >> 1], (bits & 1u) ? 0x10000u : 1u); };
  if (fast) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      if (j * NT + tid < nfull) {
        const uint32_t w4[4] = {d[j].x, d[j].y, d[j].z, d[j].w};
#pragma unroll
        for (int e = 0; e < 8; ++e) count((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
      }
    }
  } else {
    for (int c = tid; c < nfull; c += NT) {
      const uint4 q = load_chunk16(row, c, V, ALIGNED);
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) count(elem_bits((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu));
    }
  }
  if (tid == 0)
    for (int i = nfull * 8; i < V; ++i) count(elem_bits(row[i]));

  FL_MARK(12);
  // ------------------------------------------------ repetition penalty
  // each unique id moves one count from its pattern to its penalised pattern
  auto penalise = [&](uint32_t raw) {
    const uint32_t z = elem_bits(raw);
    const uint32_t zp = D::from_f32(penalty_val<D>(D::to_f32(z), RP));
    if (zp != z) {
      atomicAdd(&sh.hist[z >> 1], (z & 1u) ? 0xFFFF0000u : 0xFFFFFFFFu);
      atomicAdd(&sh.hist[zp >> 1], (zp & 1u) ? 0x10000u : 1u);
    }
  };
#pragma unroll
  for (int k = 0; k < HPRE; ++k)
    if (own[k]) penalise(xh[k]);
  for (int i = tid + (hist_rows ? HPRE * NT : 0); i < H; i += NT) {
    const int id = hid[i];
    if (claim(i, id)) penalise(row[id]);
  }
  __syncthreads();
  FL_MARK(2);

  // ------------------------------------------------ compact to entries
  // Wave w owns order indices [4096w, 4096w+4096): waves 0-7 the positive
  // patterns (descending bits), 8-15 the negative ones (ascending bits).  Lane
  // l reads word 64i+l of its wave's range in step i, so the 64 lanes of a
  // read hit consecutive LDS words (no bank conflicts); a word's two
  // counters are two consecutive order indices.  Positions come from ballots:
  // entries are written in ascending order index.
  {
    const int wave = tid / WAVE;
    const int lane = tid & (WAVE - 1);
    const bool pos = wave < NWAVE / 2;  // wave-uniform
    uint32_t x[32];
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const int W = pos ? (0x3FFF - 2048 * wave - (64 * i + lane)) : (2048 * wave + 64 * i + lane);
      x[i] = sh.hist[W];
    }
    uint32_t any = 0;
#pragma unroll
    for (int i = 0; i < 32; ++i) any |= x[i];
    const bool populated = __ballot(any != 0) != 0;  // wave-uniform
    // halves in ascending order index: positive words hi then lo, negative lo then hi
    auto first = [&](uint32_t w) { return pos ? (w >> 16) : (w & 0xFFFFu); };
    auto second = [&](uint32_t w) { return pos ? (w & 0xFFFFu) : (w >> 16); };
    auto word_of = [&](int i) { return pos ? (0x3FFF - 2048 * wave - (64 * i + lane)) : (2048 * wave + 64 * i + lane); };
    // bits of the first / second half of word W
    auto bits1 = [&](int W) { return pos ? 2u * W + 1 : 2u * W; };
    auto bits2 = [&](int W) { return pos ? 2u * W : 2u * W + 1; };
    const bool nan_range = wave == 0 || wave == NWAVE - 1;  // all NaN patterns live here
    auto valid = [&](uint32_t cnt, uint32_t bits) {
      return cnt != 0 && (!nan_range || (bits & 0x7FFFu) <= D::INF_BITS);
    };
    uint32_t wtot = 0, lsum = 0;
    bool nan = false;
    if (populated && !nan_range) {
      // SWAR: bit 15 / bit 31 set iff the low / high counter is non-zero
      uint32_t lcnt = 0;
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        lcnt += __popc((((x[i] & 0x7FFF7FFFu) + 0x7FFF7FFFu) | x[i]) & 0x80008000u);
        lsum += (x[i] & 0xFFFFu) + (x[i] >> 16);
      }
      wtot = wave_reduce(lcnt, OpAdd());
    } else if (populated) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        const int W = word_of(i);
        const uint32_t a1 = first(x[i]), a2 = second(x[i]);
        const bool v1 = valid(a1, bits1(W)), v2 = valid(a2, bits2(W));
        nan |= (a1 != 0 && !v1) || (a2 != 0 && !v2);
        wtot += __popcll(__ballot(v1)) + __popcll(__ballot(v2));
        lsum += a1 + a2;
      }
    }
    if (nan) atomicOr(&sh.status, FL_ROW_NAN);
    if (lane == 0) sh.redu[wave] = wtot;
    const uint32_t total_cnt = block_reduce<uint32_t>(lsum, OpAdd(), sh.redi_u);  // includes a barrier
    uint32_t base = 0, n_total = 0;
#pragma unroll
    for (int i = 0; i < NWAVE; ++i) {
      const uint32_t t = sh.redu[i];
      if (i < wave) base += t;
      n_total += t;
    }
    if (wtot) {
#pragma unroll
      for (int i = 0; i < 32; ++i) {
        if (__ballot(x[i] != 0) == 0) continue;  // 64 empty words (wave-uniform)
        const int W = word_of(i);
        const uint32_t a1 = first(x[i]), a2 = second(x[i]);
        const bool v1 = valid(a1, bits1(W)), v2 = valid(a2, bits2(W));
        const uint64_t m1 = __ballot(v1), m2 = __ballot(v2);
        const uint32_t below = __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m1 >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m1), 0)) +
                               __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(m2 >> 32),
                                                         __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(m2), 0));
        const uint32_t p1 = base + below;
        if (v1 && p1 < static_cast<uint32_t>(HIST_WORDS)) sh.hist[p1] = (order16(bits1(W)) << 16) | a1;
        const uint32_t p2 = p1 + (v1 ? 1u : 0u);
        if (v2 && p2 < static_cast<uint32_t>(HIST_WORDS)) sh.hist[p2] = (order16(bits2(W)) << 16) | a2;
        base += __popcll(m1) + __popcll(m2);
      }
    }
    if (tid == 0) {
      sh.n_entries = static_cast<int32_t>(min(n_total, static_cast<uint32_t>(HIST_WORDS)));
      // a total other than V means a 16-bit counter wrapped (> 65535 equal values)
      if (total_cnt != static_cast<uint32_t>(V) || n_total > static_cast<uint32_t>(HIST_WORDS))
        sh.status |= FL_ROW_LIMIT;
    }
  }
  __syncthreads();
  FL_MARK(3);

  const int N = sh.n_entries;
  uint32_t* ent = sh.hist;
  const bool cached = N <= ENTRY_CACHE_MAX;
  float* Yc = reinterpret_cast<float*>(sh.hist + N);
  float* Ec = reinterpret_cast<float*>(sh.hist + 2 * N);

  auto ent_cnt = [&](int i) -> uint32_t { return ent[i] & 0xFFFFu; };
  auto ent_y = [&](int i) -> float {
    float z = D::to_f32(bits_of_order16(ent[i] >> 16));
    if (sc_entry) z = softcap_val<D>(z, CAP);
    return temperature_val<D>(z, T);
  };

  float M = 0.0f;
  if (sh.status == 0 && N > 0) {
    M = ent_y(0);
    if (tid == 0) {
      if (isnan(M)) sh.status |= FL_ROW_NAN;
      else if (isinf(M)) sh.status |= (M > 0.0f) ? FL_ROW_INF : FL_ROW_ALL_MASKED;
    }
  }
  __syncthreads();
  int32_t status = sh.status;

  int lo, hi;
  thread_slice(N, lo, hi);
  if (status == 0 && cached) {
    for (int i = lo; i < hi; ++i) {
      const float y = ent_y(i);
      Yc[i] = y;
      Ec[i] = expf(y - M);
    }
  }
  __syncthreads();
  FL_MARK(4);
  auto Y = [&](int i) -> float { return cached ? Yc[i] : ent_y(i); };
  auto E = [&](int i) -> float { return cached ? Ec[i] : expf(ent_y(i) - M); };

  // Decision results (block-uniform once computed)
  int i0 = N - 1;            // last entry that holds kept members
  uint32_t c0 = 0;           // kept members of entry i0
  double SK = 0.0;           // sum of e over kept members
  uint32_t n_kept = 0;       // number of kept members
  float rK = 0.0f;           // float32 reciprocal of SK (softmax scale)
  int cut_lo = 0, cut_hi = 0;            // entries of i0's value group
  uint32_t cut_kept = 0, cut_total = 0;  // kept / all members of that group
  int sel_lo = 0, sel_hi = -1;           // entries of the selected value group
  uint32_t sel_rank = 0;                 // rank by index within that group

  if (status == 0) {
    // ---------------- top-k (sampling.py:36-38): k-th largest value, ties kept
    int L = N;
    if (K > 0 && K < V) {
      uint32_t local = 0;
      for (int i = lo; i < hi; ++i) local += ent_cnt(i);
      uint32_t tot;
      uint32_t acc = block_excl_scan<uint32_t>(local, sh.redu, &tot);
      if (acc < static_cast<uint32_t>(K) && acc + local >= static_cast<uint32_t>(K)) {
        for (int i = lo; i < hi; ++i) {
          acc += ent_cnt(i);
          if (acc >= static_cast<uint32_t>(K)) { sh.ik = i; break; }
        }
      }
      if (tid == 0) sh.lk = N;
      __syncthreads();
      const float tau = Y(sh.ik);
      for (int i = max(lo, 1); i < hi; ++i)
        if (Y(i) < tau && Y(i - 1) >= tau) sh.lk = i;
      __syncthreads();
      L = sh.lk;
    }

    // ---------------- min-p (sampling.py:40-43) over the top-k survivors
    auto mass_upto = [&](int n) -> double {
      double s = 0.0;
      for (int i = lo; i < min(hi, n); ++i) s += static_cast<double>(ent_cnt(i)) * E(i);
      return block_reduce<double>(s, OpAdd(), sh.redd);
    };
    double S = mass_upto(L);
    if (MP > 0.0f) {
      const float r = 1.0f / static_cast<float>(S);
      const float thr = D::rn(D::rn(r) * MP);
      int first_out = L;
      for (int i = lo; i < min(hi, L); ++i)
        if (D::rn(E(i) * r) < thr) { first_out = i; break; }
      const int Lm = block_reduce<int32_t>(first_out, OpMin(), sh.redi);
      if (Lm < L) {
        L = Lm;
        S = mass_upto(L);
      }
    }
    if (L <= 0) status |= FL_ROW_ALL_MASKED;

    // ---------------- top-p (sampling.py:45-51)
    // Position j (descending order) is removed when
    //   round(round_f32(C_j) - p_j) >= round(top_p)
    // with C_j the inclusive cumulative of the rounded probabilities.  The
    // predicate is monotone along the order, so the kept set is a prefix.
    i0 = L - 1;
    if (status == 0) c0 = ent_cnt(i0);
    if (status == 0 && TP > 0.0f && TP < 1.0f) {
      // cumulative sums in 2^-46 fixed point: exact, so every thread's slice
      // boundaries agree with the block scan
      const float r1 = 1.0f / static_cast<float>(S);
      const float t = D::rn(TP);
      auto removed = [&](uint64_t c_incl, float p) {
        return D::rn(D::rn(static_cast<float>(from_fx(c_incl))) - p) >= t;
      };
      uint64_t local = 0;
      for (int i = lo; i < min(hi, L); ++i) local += ent_cnt(i) * to_fx(D::rn(E(i) * r1));
      uint64_t tot;
      const uint64_t base = block_excl_scan<uint64_t>(local, sh.redq, &tot);
      int first = L;
      {
        uint64_t c = base;
        for (int i = lo; i < min(hi, L); ++i) {
          const float p = D::rn(E(i) * r1);
          const uint64_t pf = to_fx(p);
          if (removed(c + pf, p)) { first = i; break; }
          c += ent_cnt(i) * pf;
        }
      }
      const int i1 = block_reduce<int32_t>(first, OpMin(), sh.redi);
      if (i1 == 0) {
        status |= FL_ROW_ALL_MASKED;
      } else if (i1 < L) {
        i0 = i1 - 1;
        if (i0 >= lo && i0 < hi) {
          uint64_t c = base;
          for (int i = lo; i < i0; ++i) c += ent_cnt(i) * to_fx(D::rn(E(i) * r1));
          const float p = D::rn(E(i0) * r1);
          const uint64_t pf = to_fx(p);
          const uint32_t n = ent_cnt(i0);
          // members [0, kept) survive; member 0 is known to survive
          uint32_t klo = 1, khi = n;  // answer in [klo, khi]
          while (klo < khi) {
            const uint32_t mid = (klo + khi + 1) >> 1;   // does member mid-1 survive?
            if (!removed(c + static_cast<uint64_t>(mid) * pf, p)) klo = mid;
            else khi = mid - 1;
          }
          sh.c0 = klo;
        }
        __syncthreads();
        c0 = sh.c0;
      }
    }
  }

  if (status == 0) {
    // ---------------- group of the last kept entry
    const float ycut = Y(i0);
    cut_lo = i0;
    while (cut_lo > 0 && Y(cut_lo - 1) == ycut) --cut_lo;
    cut_hi = i0;
    while (cut_hi + 1 < N && Y(cut_hi + 1) == ycut) ++cut_hi;
    for (int i = cut_lo; i <= cut_hi; ++i) {
      cut_total += ent_cnt(i);
      if (i < i0) cut_kept += ent_cnt(i);
    }
    cut_kept += c0;

    auto kc = [&](int i) -> uint32_t { return i < i0 ? ent_cnt(i) : (i == i0 ? c0 : 0u); };

    // ---------------- softmax of the filtered row (sampling.py:58)
    {
      double s = 0.0;
      uint32_t n = 0;
      for (int i = lo; i < min(hi, i0 + 1); ++i) {
        s += static_cast<double>(kc(i)) * E(i);
        n += kc(i);
      }
      SK = block_reduce<double>(s, OpAdd(), sh.redd);
      n_kept = block_reduce<uint32_t>(n, OpAdd(), sh.redu);
    }
    rK = 1.0f / static_cast<float>(SK);

    if (select) {
      if (T <= 0.0f) {
        // greedy (sampling.py:59-60): first index among the maximal probabilities
        const float qmax = D::rn(E(0) * rK);
        int last = 0;
        for (int i = lo; i < min(hi, i0 + 1); ++i)
          if (D::rn(E(i) * rK) == qmax) last = i;
        last = block_reduce<int32_t>(last, OpMax(), sh.redi);
        sel_lo = 0;
        sel_hi = last;
        const float yl = Y(last);
        while (sel_hi + 1 < N && Y(sel_hi + 1) == yl) ++sel_hi;
        sel_rank = 0;
      } else {
        // inverse CDF (CONVENTION replacing torch.multinomial, sampling.py:61):
        // first member whose inclusive cumulative probability exceeds u * total,
        // cumulative sums in exact 2^-46 fixed point
        uint64_t local = 0;
        for (int i = lo; i < min(hi, i0 + 1); ++i) local += kc(i) * to_fx(D::rn(E(i) * rK));
        uint64_t Q;
        const uint64_t base = block_excl_scan<uint64_t>(local, sh.redq, &Q);
        const uint64_t target = __double2ull_rd(static_cast<double>(U) * static_cast<double>(Q));
        if (tid == 0) {
          sh.sel_entry = -1;
          sh.sel_cexcl = 0;
        }
        __syncthreads();
        {
          uint64_t c = base;
          for (int i = lo; i < min(hi, i0 + 1); ++i) {
            const uint64_t m = kc(i) * to_fx(D::rn(E(i) * rK));
            if (m > 0 && c <= target && target < c + m) sh.sel_entry = i;
            c += m;
          }
        }
        __syncthreads();
        int is = sh.sel_entry;
        if (is < 0) {
          // no positive mass at all (every kept probability rounds to zero)
          is = 0;
        }
        const float ys = Y(is);
        sel_lo = is;
        while (sel_lo > 0 && Y(sel_lo - 1) == ys) --sel_lo;
        sel_hi = is;
        while (sel_hi + 1 < N && Y(sel_hi + 1) == ys) ++sel_hi;
        // cumulative mass before the selected value group
        {
          uint64_t c = base;
          for (int i = lo; i < min(hi, i0 + 1); ++i) {
            if (i == sel_lo) sh.sel_cexcl = c;
            c += kc(i) * to_fx(D::rn(E(i) * rK));
          }
        }
        __syncthreads();
        const uint64_t cg = sh.sel_cexcl;
        const uint64_t q = to_fx(D::rn(E(is) * rK));
        uint32_t kept_g = 0;
        for (int i = sel_lo; i <= sel_hi; ++i) kept_g += kc(i);
        // member r of the group covers [cg + r q, cg + (r+1) q)
        uint64_t r = (q > 0 && target >= cg) ? (target - cg) / q : 0;
        sel_rank = static_cast<uint32_t>(min(r, static_cast<uint64_t>(kept_g - 1)));
      }
    }
  }
  // values the output stage needs, read before the entry list is overwritten
  const float y_sel = (status == 0 && select) ? Y(sel_lo) : 0.0f;
  const float y_cut = (status == 0) ? Y(i0) : __builtin_inff();
  __syncthreads();
  FL_MARK(6);

  // ------------------------------------------------ identification
  // Targets: 0 = selected token (group sel, rank sel_rank); 1 = last kept
  // member of a partially kept group (for the descriptor's idx_cut).
  const bool want_cut = (a.out_desc != nullptr) && status == 0 && cut_kept < cut_total;
  const bool want_sel = select && status == 0;
  uint32_t o_lo[2] = {0, 0}, o_hi[2] = {0, 0}, rank[2] = {0, 0};
  bool active[2] = {want_sel, want_cut};
  if (want_sel) { o_lo[0] = ent[sel_lo] >> 16; o_hi[0] = ent[sel_hi] >> 16; rank[0] = sel_rank; }
  if (want_cut) { o_lo[1] = ent[cut_lo] >> 16; o_hi[1] = ent[cut_hi] >> 16; rank[1] = cut_kept - 1; }
  __syncthreads();  // entries are overwritten by the candidate lists below

  if (active[0] || active[1]) {
    uint32_t* list[2] = {sh.hist, sh.hist + LIST_CAP};
    uint32_t* hitq = sh.hist + 2 * LIST_CAP;
    auto in_range = [&](int t, uint32_t bits) { return order16(bits) - o_lo[t] <= o_hi[t] - o_lo[t]; };
    auto is_hist = [&](int idx) { return pen && ((sh.hbits[idx >> 5] >> (idx & 31)) & 1u); };
    // The targets' order ranges as at most four ranges of raw bit patterns
    // (a range across zero splits into its positive and negative parts).
    // (slots 2t, 2t+1 belong to target t; fixed slots keep the arrays in VGPRs)
    // Range r covers patterns rlo[r] .. rlo[r] + rw[r].
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
    // Packed 16-bit range test of both halves of a word: a wrapping subtract
    // of the range start, then a saturating subtract of the width, leaves 0
    // exactly in the halves inside the range.
    auto range_test = [&](uint32_t w, int r) -> uint32_t {
      const u16x2 d = __builtin_bit_cast(u16x2, w) - u16x2{static_cast<unsigned short>(rlo[r]),
                                                            static_cast<unsigned short>(rlo[r])};
      return __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(
                                              d, u16x2{static_cast<unsigned short>(rw[r]),
                                                       static_cast<unsigned short>(rw[r])}));
    };
    // non-zero iff a half of e is zero (may also flag a half above a zero
    // one; the exact test on the hit path sorts that out)
    auto zero_halves = [](uint32_t e) { return (e - 0x00010001u) & ~e & 0x80008000u; };
    auto candidate = [&](int idx, int t) {
      if (idx < V && !is_hist(idx)) {
        const uint32_t s = atomicAdd(&sh.nlist[t], 1u);
        if (s < static_cast<uint32_t>(LIST_CAP)) list[t][s] = idx;
      }
    };
    // Element work for one chunk (patterns recomputed one by one).
    auto chunk_candidates = [&](int c, const uint4 q) {
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t bits = elem_bits((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
#pragma unroll
        for (int t = 0; t < 2; ++t)
          if (active[t] && in_range(t, bits)) candidate(c * 8 + e, t);
      }
    };
    const int nchunks = (V + 7) >> 3;
    if (fast) {
      // Non-history elements whose value lies in a target group.  The row is
      // read again, all chunks in flight at once (mostly a cache hit); each
      // chunk gets a branch-free packed test, and the rare hit chunks are
      // queued in LDS and examined element by element afterwards, which keeps
      // this loop small enough to stay unrolled with the tile in VGPRs.
      uint4 r[NCH];
#pragma unroll
      for (int j = 0; j < NCH; ++j) r[j] = buf_load16(rrow, 16u * tid, 16u * NT * j);
      FL_MARK(13);
#pragma unroll
      for (int j = 0; j < NCH; ++j) {
        uint32_t any = 0;
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          if (!ren[rr]) continue;  // wave-uniform
          any |= zero_halves(range_test(r[j].x, rr)) | zero_halves(range_test(r[j].y, rr)) |
                 zero_halves(range_test(r[j].z, rr)) | zero_halves(range_test(r[j].w, rr));
        }
        const int c = j * NT + tid;
        if (any != 0 && c < nchunks) {
          const uint32_t s = atomicAdd(&sh.nhit, 1u);
          if (s < static_cast<uint32_t>(HIT_CAP)) hitq[s] = c;
        }
      }
      FL_MARK(14);
      __syncthreads();
      const uint32_t nhit = sh.nhit;
      if (nhit <= static_cast<uint32_t>(HIT_CAP)) {
        for (int i = tid; i < static_cast<int>(nhit); i += NT) {
          const int c = hitq[i];
          chunk_candidates(c, buf_load16(rrow, 16u * c, 0u));
        }
      } else {
        for (int c = tid; c < nchunks; c += NT) chunk_candidates(c, buf_load16(rrow, 16u * c, 0u));
      }
    } else {
      for (int c = tid; c < nchunks; c += NT) chunk_candidates(c, load_chunk16(row, c, V, ALIGNED));
    }
    // history elements whose penalised value lies in a target group (the
    // first HPRE ids of each thread and their logits are still in registers)
    if (pen) {
      auto hist_candidate = [&](int id, uint32_t raw) {
        const uint32_t z = elem_bits(raw);
        const uint32_t zp = D::from_f32(penalty_val<D>(D::to_f32(z), RP));
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (active[t] && in_range(t, zp)) {
            const uint32_t s = atomicAdd(&sh.nlist[t], 1u);
            if (s < static_cast<uint32_t>(LIST_CAP)) list[t][s] = id;
          }
        }
      };
#pragma unroll
      for (int k = 0; k < HPRE; ++k)
        if (own[k]) hist_candidate(hpre[k], xh[k]);
      for (int i = tid + (hist_rows ? HPRE * NT : 0); i < H; i += NT) {
        if (!((sh.owner[i >> 5] >> (i & 31)) & 1u)) continue;
        const int id = hid[i];
        hist_candidate(id, row[id]);
      }
    }
    __syncthreads();
    FL_MARK(7);
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      if (!active[t]) continue;
      const int n = static_cast<int>(sh.nlist[t]);
      if (n <= RANK_SELECT_MAX) {
        // rank by all-pairs counting over the (distinct) candidate indices
        for (int i = tid; i < n; i += NT) {
          const uint32_t v = list[t][i];
          uint32_t below = 0;
          for (int k2 = 0; k2 < n; ++k2) below += list[t][k2] < v;
          if (below == rank[t]) sh.result[t] = static_cast<int32_t>(v);
        }
      } else {
        // too many candidates: count matches round by round in index order
        // (re-reads the row from memory; a rare path kept out of the VGPR tile)
        uint32_t base = 0;
        for (int j = 0; j < NCH; ++j) {
          const int e0 = (j * NT + tid) * 8;
          uint32_t m = 0;
          for (int e = 0; e < 8; ++e) {
            const int idx = e0 + e;
            if (idx >= V) continue;
            uint32_t bits = elem_bits(row[idx]);
            if (is_hist(idx)) bits = D::from_f32(penalty_val<D>(D::to_f32(bits), RP));
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
  __syncthreads();
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
    if (a.out_token) a.out_token[b] = tok;
    if (a.out_status) a.out_status[b] = status;
    if (a.out_finished) {
      const bool fin = (a.finished_in != nullptr && a.finished_in[b] != 0) ||
                       (tok >= 0 && is_stop(a.stop_ids, a.stop_ld, a.n_stop, b, tok));
      a.out_finished[b] = fin ? 1 : 0;
    }
    if (a.out_logprob) {
      float lp = __builtin_nanf("");
      if (tok >= 0) lp = D::rn((y_sel - M) - logf(static_cast<float>(SK)));
      a.out_logprob[b] = lp;
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
}

// ------------------------------------------------------------------ launch
hipError_t launch_sample_rows16(const fl_sample_args& a, hipStream_t s) {
  const int aligned = (reinterpret_cast<uintptr_t>(a.logits) % 16 == 0) && ((a.ld * 2) % 16 == 0);
  const bool has_pen = a.rep_penalty != nullptr && a.hist_ids != nullptr && a.hist_len != nullptr;
  const int sc_elem = (a.softcap > 0.0f && has_pen) ? 1 : 0;
  const dim3 grid(static_cast<unsigned>(a.batch)), block(NT);
  if (a.dtype == FL_DTYPE_BF16) hipLaunchKernelGGL(k_sample_rows16<BF16>, grid, block, 0, s, a, aligned, sc_elem);
  else hipLaunchKernelGGL(k_sample_rows16<F16>, grid, block, 0, s, a, aligned, sc_elem);
  return hipGetLastError();
}

}  // namespace fl

#ifdef FL_PHASE_TIMES
// Tuning builds only: copy the phase timestamps recorded by the last launch.
extern "C" int fl_debug_phase_ts(uint64_t* out) {
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(fl_phase_ts), sizeof(uint64_t) * 192, 0, hipMemcpyDeviceToHost) ==
                 hipSuccess ? 0 : -1;
}
#endif
