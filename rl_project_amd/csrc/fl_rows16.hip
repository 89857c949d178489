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
constexpr int LIST_CAP = HIST_WORDS / 2;         // candidates per identification target
constexpr int ENTRY_CACHE_MAX = HIST_WORDS / 3;  // entries whose y and e fit beside the list
constexpr int RANK_SELECT_MAX = 2048;            // candidates ranked by all-pairs counting

static_assert(NCH * NT * 8 == FL_MAX_VOCAB_16, "one VGPR tile holds the largest 16-bit row");

struct Shared16 {
  uint32_t hist[HIST_WORDS];
  uint32_t hbits[HBITS_WORDS];
  uint32_t owner[OWNER_WORDS];
  double redd[NWAVE];
  uint64_t redq[NWAVE];
  uint32_t redu[NWAVE];
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
};

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
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int V = static_cast<int>(a.vocab);
  const uint16_t* row = static_cast<const uint16_t*>(a.logits) + b * a.ld;

  const float T = a.temperature ? a.temperature[b] : 1.0f;
  const int K = a.top_k ? a.top_k[b] : 0;
  const float TP = a.top_p ? a.top_p[b] : 1.0f;
  const float MP = a.min_p ? a.min_p[b] : 0.0f;
  const float RP = a.rep_penalty ? a.rep_penalty[b] : 1.0f;
  // u outside [0, 1) (or NaN) is clamped into it
  const float U = fminf(fmaxf(a.uniforms ? a.uniforms[b] : 0.0f, 0.0f), 0.99999994f);
  const float CAP = a.softcap;
  const int H_in = (a.hist_ids != nullptr && a.hist_len != nullptr && RP != 1.0f) ? a.hist_len[b] : 0;
  const bool hist_too_long = H_in > FL_MAX_HISTORY;
  const int H = hist_too_long ? 0 : H_in;
  const bool pen = H > 0;
  const bool sc_entry = (CAP > 0.0f) && !SC_ELEM;
  const bool select = (a.flags & FL_FLAG_NO_SELECT) == 0;

  // Value pattern of an element as the filters see it before penalty.
  auto elem_bits = [&](uint32_t raw) -> uint32_t {
    return SC_ELEM ? D::from_f32(softcap_val<D>(D::to_f32(raw), CAP)) : raw;
  };
  const int nfull = V >> 3;                 // chunks holding 8 valid elements
  const bool fast = ALIGNED && !SC_ELEM;    // whole row through the VGPR tile

  // ------------------------------------------------ load the row (VGPRs)
  uint4 d[NCH];
  if (fast) {
#pragma unroll
    for (int j = 0; j < NCH; ++j) {
      const int c = j * NT + tid;
      d[j] = (c < nfull) ? reinterpret_cast<const uint4*>(row)[c] : make_uint4(0, 0, 0, 0);
    }
  }

  // ------------------------------------------------ clear LDS
  for (int i = tid; i < HIST_WORDS / 4; i += NT) reinterpret_cast<uint4*>(sh.hist)[i] = make_uint4(0, 0, 0, 0);
  if (pen) {
    for (int i = tid; i < (V + 31) / 32; i += NT) sh.hbits[i] = 0;
    for (int i = tid; i < (H + 31) / 32; i += NT) sh.owner[i] = 0;
  }
  if (tid == 0) {
    sh.status = hist_too_long ? FL_ROW_LIMIT : 0;
    sh.nlist[0] = sh.nlist[1] = 0;
    sh.result[0] = sh.result[1] = -1;
    sh.ik = 0;
    sh.lk = 0;
  }
  __syncthreads();

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

  // ------------------------------------------------ repetition penalty
  const int32_t* hid = pen ? a.hist_ids + b * a.hist_ld : nullptr;
  if (pen) {
    for (int i = tid; i < H; i += NT) {
      const int id = hid[i];
      if (id < 0 || id >= V) {
        atomicOr(&sh.status, FL_ROW_BAD_HISTORY);
        continue;
      }
      const uint32_t bit = 1u << (id & 31);
      if (atomicOr(&sh.hbits[id >> 5], bit) & bit) continue;  // a duplicate id
      atomicOr(&sh.owner[i >> 5], 1u << (i & 31));
      const uint32_t z = elem_bits(row[id]);
      const uint32_t zp = D::from_f32(penalty_val<D>(D::to_f32(z), RP));
      if (zp != z) {
        atomicAdd(&sh.hist[z >> 1], (z & 1u) ? 0xFFFF0000u : 0xFFFFFFFFu);
        atomicAdd(&sh.hist[zp >> 1], (zp & 1u) ? 0x10000u : 1u);
      }
    }
  }
  __syncthreads();

  // ------------------------------------------------ compact to entries
  // Thread t owns order indices [64t, 64t+64): threads < 512 the positive
  // patterns (descending bits), the rest the negative ones (ascending bits).
  {
    uint32_t w[32];
    const bool pos = tid < NT / 2;
    const int base_w = pos ? (0x3FE0 - 32 * tid) : (32 * tid);
#pragma unroll
    for (int i = 0; i < 32; ++i) w[i] = sh.hist[base_w + i];
    auto cnt_at = [&](int q) -> uint32_t {
      const uint32_t word = pos ? w[31 - (q >> 1)] : w[q >> 1];
      return pos ? ((q & 1) ? (word & 0xFFFFu) : (word >> 16)) : ((q & 1) ? (word >> 16) : (word & 0xFFFFu));
    };
    uint32_t n_local = 0, sum_local = 0;
    int32_t flags = 0;
#pragma unroll
    for (int q = 0; q < 64; ++q) {
      const uint32_t cnt = cnt_at(q);
      const uint32_t bits = bits_of_order16(64 * tid + q);
      sum_local += cnt;
      if (cnt) {
        if ((bits & 0x7FFFu) > D::INF_BITS) flags |= FL_ROW_NAN;
        else ++n_local;
      }
    }
    if (flags) atomicOr(&sh.status, flags);
    uint32_t n_total;
    uint32_t p = block_excl_scan<uint32_t>(n_local, sh.redu, &n_total);
    const uint32_t total_cnt = block_reduce<uint32_t>(sum_local, OpAdd(), sh.redu);
#pragma unroll
    for (int q = 0; q < 64; ++q) {
      const uint32_t cnt = cnt_at(q);
      const uint32_t bits = bits_of_order16(64 * tid + q);
      if (cnt && (bits & 0x7FFFu) <= D::INF_BITS) {
        if (p < static_cast<uint32_t>(HIST_WORDS)) sh.hist[p] = (static_cast<uint32_t>(64 * tid + q) << 16) | cnt;
        ++p;
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
    auto in_range = [&](int t, uint32_t bits) { return order16(bits) - o_lo[t] <= o_hi[t] - o_lo[t]; };
    auto is_hist = [&](int idx) { return pen && ((sh.hbits[idx >> 5] >> (idx & 31)) & 1u); };
    // non-history elements whose value lies in a target group (re-reads the row)
    for (int c = tid; c < (V + 7) / 8; c += NT) {
      const uint4 q = load_chunk16(row, c, V, ALIGNED);
      const uint32_t w4[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int idx = c * 8 + e;
        if (idx < V) {
          const uint32_t bits = elem_bits((w4[e >> 1] >> ((e & 1) * 16)) & 0xFFFFu);
#pragma unroll
          for (int t = 0; t < 2; ++t) {
            if (active[t] && in_range(t, bits) && !is_hist(idx)) {
              const uint32_t s = atomicAdd(&sh.nlist[t], 1u);
              if (s < static_cast<uint32_t>(LIST_CAP)) list[t][s] = idx;
            }
          }
        }
      }
    }
    // history elements whose penalised value lies in a target group
    if (pen) {
      for (int i = tid; i < H; i += NT) {
        if (!((sh.owner[i >> 5] >> (i & 31)) & 1u)) continue;
        const int id = hid[i];
        const uint32_t z = elem_bits(row[id]);
        const uint32_t zp = D::from_f32(penalty_val<D>(D::to_f32(z), RP));
#pragma unroll
        for (int t = 0; t < 2; ++t) {
          if (active[t] && in_range(t, zp)) {
            const uint32_t s = atomicAdd(&sh.nlist[t], 1u);
            if (s < static_cast<uint32_t>(LIST_CAP)) list[t][s] = id;
          }
        }
      }
    }
    __syncthreads();
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

  // ------------------------------------------------ outputs
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
