// Speculative-decoding verify: accept / residual resample / bonus for a batch
// of sequences, one work-group of 1024 threads per sequence (reference
// src/forgeline/models/generation/speculative.py:54-84).
//
// The filtered target and draft distributions come as row descriptors from
// the row samplers (the target rows' own samples are the bonus tokens), so this
// kernel reads logits only at the draft tokens and, at the first rejection, the
// two rows of that position:
//
//   accept   thread 0 walks the drafts: ratio = min(1, p(d) / (q(d) + 1e-10))
//            with p, q and the arithmetic in the logits' dtype (:63); the draft
//            is accepted iff u_accept < ratio (:65)
//   residual r = max(0, p - q) / (sum(r) + 1e-10) (:73-74), or p where r is all
//            zero; the token is the first index, in ascending order, whose
//            inclusive mass exceeds u_resample times the total (inverse CDF in
//            place of torch.multinomial, :75), with masses in exact 2^-45
//            fixed point and the order kept by thread-contiguous row slices
//   bonus    every draft accepted: the target sample of position K (:79-84)
#include <mutex>

#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {

namespace {

constexpr int FXB = 45;

__device__ __forceinline__ uint64_t fx45(float e) {
  const uint32_t u = __float_as_uint(e);
  const int ex = static_cast<int>(u >> 23);
  if (ex == 0) return 0;
  const uint64_t m = (u & 0x7FFFFFu) | 0x800000u;
  const int s = ex - 150 + FXB;
  if (s >= 0) return m << s;
  if (s < -24) return 0;
  return (m + (1ull << (-s - 1))) >> (-s);
}

// 16-byte chunks of a row in dtype D: N elements each.
template <class D>
struct Chunk;
template <>
struct Chunk<F32> {
  static constexpr int N = 4;
  __device__ static float elem(__amdgpu_buffer_rsrc_t r, int i) {
    return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(r, 4 * i, 0, 0));
  }
  __device__ static void unpack(const uint4 u, float (&x)[N]) {
    x[0] = __uint_as_float(u.x);
    x[1] = __uint_as_float(u.y);
    x[2] = __uint_as_float(u.z);
    x[3] = __uint_as_float(u.w);
  }
};
template <class H>
struct Chunk16 {
  static constexpr int N = 8;
  __device__ static float elem(__amdgpu_buffer_rsrc_t r, int i) {
    return H::to_f32(__builtin_amdgcn_raw_buffer_load_b16(r, 2 * i, 0, 0));
  }
  __device__ static void unpack(const uint4 u, float (&x)[N]) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = H::to_f32(w[k] & 0xFFFFu);
      x[2 * k + 1] = H::to_f32(w[k] >> 16);
    }
  }
};
template <>
struct Chunk<BF16> : Chunk16<BF16> {};
template <>
struct Chunk<F16> : Chunk16<F16> {};

// Filtered value of a logit as the row samplers compute it (no history on
// speculative rows).
template <class D>
__device__ __forceinline__ float filt_value(float x, float cap, float t) {
  float z = x;
  if (cap > 0.0f) z = softcap_val<D>(z, cap);
  return temperature_val<D>(z, t);
}

// Probability of element i under a row descriptor: softmax of the kept set,
// computed as the reference's softmax does, e * (1 / S), rounded to D.
template <class D>
__device__ __forceinline__ float prob_of(const fl_row_desc& ds, float y, int64_t i) {
  const bool kept = ds.status == 0 && y > -__builtin_inff() && (y > ds.y_cut || (y == ds.y_cut && i <= ds.idx_cut));
  return kept ? D::rn(expf(y - ds.shift) * ds.inv_mass) : 0.0f;
}

// Rows up to 262144 elements: at most 64 rounds of NT 16-byte chunks.
constexpr int MAX_ROUNDS = 64;
// Sliced residual: at most this many slices of a row pair per sequence, and
// this many threads per slice work-group.
constexpr int MAX_SLICES = WAVE;  // slices of a row pair (one per lane of a wave in the pick)
constexpr int NT_PART = 256;

struct SharedSpec {
  uint64_t redq[NWAVE];
  uint64_t seg[MAX_ROUNDS * NWAVE];  // weight sum of each (round, wave) segment
  int32_t n_acc;
  int32_t rejected;
  int32_t token;
};

// Accept walk of sequence b (one wave): ratio = min(1, p(d)/(q(d)+1e-10))
// in the logits' dtype (:63), accept iff u_accept < ratio (:65).  Writes the
// ratios and the accepted drafts when `write`; returns the accepted count,
// *rej = whether a draft was rejected.
template <class D>
__device__ int accept_walk(const fl_spec_args& a, int64_t b, bool* rej, bool write = true) {
  // Called by one whole wave: lane l evaluates positions l, l + 64, ... in
  // parallel (their loads in flight together); the first position whose
  // draw fails the ratio ends the walk, as the sequential rule has it.
  using C = Chunk<D>;
  const int lane = threadIdx.x & (WAVE - 1);
  const int64_t K = a.k;
  const int V = static_cast<int>(a.vocab);
  const float T = a.temperature[b];
  const size_t esz = D::id == FL_DTYPE_F32 ? 4 : 2;
  int64_t n = K;  // accepted drafts (the first rejected position, if any)
  for (int64_t i0 = 0; i0 < K && n == K; i0 += WAVE) {
    const int64_t i = i0 + lane;
    float ratio = 0.0f;
    int64_t d = -1;
    bool acc = false;
    if (i < K) {
      d = a.draft_ids[b * K + i];
      if (d >= 0 && d < V) {
        const fl_row_desc td = a.target_desc[b * (K + 1) + i];
        const fl_row_desc dd = a.draft_desc[b * K + i];
        const char* tp = static_cast<const char*>(a.target) + (b * (K + 1) + i) * a.ld * esz;
        const char* dp = static_cast<const char*>(a.draft) + (b * K + i) * a.ld * esz;
        const __amdgpu_buffer_rsrc_t rt = row_rsrc(tp, static_cast<uint32_t>(V * esz));
        const __amdgpu_buffer_rsrc_t rd = row_rsrc(dp, static_cast<uint32_t>(V * esz));
        const float p = prob_of<D>(td, filt_value<D>(C::elem(rt, static_cast<int>(d)), a.softcap, T), d);
        const float q = prob_of<D>(dd, filt_value<D>(C::elem(rd, static_cast<int>(d)), a.softcap, T), d);
        ratio = fminf(1.0f, D::rn(p / D::rn(q + 1e-10f)));
      }
      acc = a.u_accept[b * K + i] < ratio;
    }
    const uint64_t fail = __ballot(i < K && !acc);
    const int64_t f = fail ? i0 + __ffsll(static_cast<unsigned long long>(fail)) - 1 : K;
    if (write && i < K) {
      if (a.out_ratio) a.out_ratio[b * K + i] = i <= f ? ratio : __builtin_nanf("");
      if (i < f) a.out_tokens[b * (K + 1) + i] = d;
    }
    n = f;
  }
  // (positions of rounds after the rejecting one: no ratio)
  if (write && a.out_ratio && n < K)
    for (int64_t i = (n / WAVE + 1) * WAVE + lane; i < K; i += WAVE) a.out_ratio[b * K + i] = __builtin_nanf("");
  *rej = n < K;
  return static_cast<int>(n);
}

// The target and draft rows of one position and their filtered probabilities.
template <class D>
struct PairRows {
  using C = Chunk<D>;
  static constexpr int N = C::N;
  __amdgpu_buffer_rsrc_t rt, rd;
  fl_row_desc td, dd;
  bool aligned;
  int V, nch, nfull;
  float cap, T;
  __device__ PairRows(const fl_spec_args& a, int64_t b, int pos) {
    const int64_t K = a.k;
    const size_t esz = D::id == FL_DTYPE_F32 ? 4 : 2;
    V = static_cast<int>(a.vocab);
    T = a.temperature[b];
    cap = a.softcap;
    td = a.target_desc[b * (K + 1) + pos];
    dd = a.draft_desc[b * K + pos];
    const char* tp = static_cast<const char*>(a.target) + (b * (K + 1) + pos) * a.ld * esz;
    const char* dp = static_cast<const char*>(a.draft) + (b * K + pos) * a.ld * esz;
    rt = row_rsrc(tp, static_cast<uint32_t>(V * esz));
    rd = row_rsrc(dp, static_cast<uint32_t>(V * esz));
    aligned = ((reinterpret_cast<uintptr_t>(tp) | reinterpret_cast<uintptr_t>(dp)) & 15u) == 0;
    nch = (V + N - 1) / N;
    nfull = V / N;
  }
  // the raw logits of chunk c of both rows
  __device__ __forceinline__ void load(int c, float (&xt)[N], float (&xd)[N]) const {
    if (aligned && c < nfull) {
      C::unpack(buf_load16(rt, 16u * c, 0u), xt);
      C::unpack(buf_load16(rd, 16u * c, 0u), xd);
    } else {
#pragma unroll
      for (int e = 0; e < N; ++e) {
        xt[e] = C::elem(rt, N * c + e);
        xd[e] = C::elem(rd, N * c + e);
      }
    }
  }
  // f(e, i, p_i, q_i) for the N elements of chunk c (ascending index i = N c + e)
  template <class F>
  __device__ __forceinline__ void eval(int c, const float (&xt)[N], const float (&xd)[N], F&& f) const {
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const int i = N * c + e;
      if (i < V) f(e, i, prob_of<D>(td, filt_value<D>(xt[e], cap, T), i), prob_of<D>(dd, filt_value<D>(xd[e], cap, T), i));
    }
  }
  template <class F>
  __device__ __forceinline__ void chunk(int c, F&& f) const {
    float xt[N], xd[N];
    load(c, xt, xd);
    eval(c, xt, xd, f);
  }
};

template <class D>
__device__ __forceinline__ float resid_of(float p, float q) { return fmaxf(D::rn(p - q), 0.0f); }

// Residual weights (:73-74): r / (sum(r) + 1e-10) in the dtype, or p where r
// is all zero (the oracle's fallback).  rsum: sum(r) in 2^-45 fixed point.
template <class D>
struct Weight {
  bool use_p;
  float den;
  __device__ explicit Weight(uint64_t rsum) {
    use_p = rsum == 0;
    den = D::rn(D::rn(static_cast<float>(static_cast<double>(rsum) * (1.0 / 35184372088832.0))) + 1e-10f);
  }
  __device__ __forceinline__ float operator()(float p, float q) const { return use_p ? p : D::rn(resid_of<D>(p, q) / den); }
};

// Sum over chunks [c0, c1) of fx45(g(p, q)) by the calling thread, chunks
// interleaved over nthreads threads (coalesced loads), four chunks of both
// rows in flight per thread.
template <class D, class G>
__device__ __forceinline__ uint64_t range_sum(const PairRows<D>& R, int c0, int c1, int nthreads, G&& g) {
  constexpr int U = 4;
  uint64_t acc = 0;
  for (int cb = c0 + static_cast<int>(threadIdx.x); cb < c1; cb += U * nthreads) {
    float xt[U][PairRows<D>::N], xd[U][PairRows<D>::N];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cb + u * nthreads;
      if (c < c1) R.load(c, xt[u], xd[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cb + u * nthreads;
      if (c < c1) R.eval(c, xt[u], xd[u], [&](int, int, float p, float q) { acc += fx45(g(p, q)); });
    }
  }
  return acc;
}

// The residual cache: one row of max(0, p - q) per sequence (the rejected
// position's), written by the first slice pass so that the second pass and
// the pick read 4 bytes per element instead of recomputing both rows'
// filtered probabilities.  Row stride: the vocabulary rounded up to 8 floats,
// so that every chunk of a row (4 or 8 elements, 16-byte aligned) lies inside
// its row's buffer range whole; the padding holds zeros.
__host__ __device__ inline int64_t spec_cache_ld(int64_t vocab) { return (vocab + 7) & ~int64_t(7); }

template <class D>
struct CachedRow {
  static constexpr int N = Chunk<D>::N;  // elements per chunk, as in PairRows
  __amdgpu_buffer_rsrc_t rr;
  int V;
  __device__ CachedRow(float* cache, int64_t ld, int64_t b, int V_) : V(V_) {
    rr = row_rsrc(cache + b * ld, static_cast<uint32_t>(ld) * 4u);
  }
  // the cached residuals of chunk c (zeros past the row)
  __device__ __forceinline__ void load(int c, float (&r)[N]) const {
#pragma unroll
    for (int h = 0; h < N / 4; ++h) {
      const uint4 u = buf_load16(rr, 16u * static_cast<uint32_t>(N / 4 * c + h), 0u);
      r[4 * h] = __uint_as_float(u.x);
      r[4 * h + 1] = __uint_as_float(u.y);
      r[4 * h + 2] = __uint_as_float(u.z);
      r[4 * h + 3] = __uint_as_float(u.w);
    }
  }
  __device__ __forceinline__ void store(int c, const float (&r)[N]) const {
#pragma unroll
    for (int h = 0; h < N / 4; ++h) {
      __builtin_amdgcn_raw_buffer_store_b128(
          __builtin_bit_cast(__attribute__((ext_vector_type(4))) unsigned int,
                             make_uint4(__float_as_uint(r[4 * h]), __float_as_uint(r[4 * h + 1]),
                                        __float_as_uint(r[4 * h + 2]), __float_as_uint(r[4 * h + 3]))),
          rr, static_cast<int>(16u * static_cast<uint32_t>(N / 4 * c + h)), 0, 0);
    }
  }
  // g(e, i, w) with w = rn(r / den), the weight of Weight<D> for r > 0 sums
  template <class G>
  __device__ __forceinline__ void weights(int c, float den, G&& g) const {
    float r[N];
    load(c, r);
#pragma unroll
    for (int e = 0; e < N; ++e) {
      const int i = N * c + e;
      if (i < V) g(e, i, D::rn(r[e] / den));
    }
  }
};

// range_sum of the residual that also stores it in the cache
template <class D>
__device__ __forceinline__ uint64_t range_sum_store(const PairRows<D>& R, const CachedRow<D>& C, int c0, int c1,
                                                    int nthreads) {
  constexpr int U = 4, N = PairRows<D>::N;
  uint64_t acc = 0;
  for (int cb = c0 + static_cast<int>(threadIdx.x); cb < c1; cb += U * nthreads) {
    float xt[U][N], xd[U][N];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cb + u * nthreads;
      if (c < c1) R.load(c, xt[u], xd[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cb + u * nthreads;
      if (c < c1) {
        float r[N];
#pragma unroll
        for (int e = 0; e < N; ++e) r[e] = 0.0f;
        R.eval(c, xt[u], xd[u], [&](int e, int, float p, float q) {
          r[e] = resid_of<D>(p, q);
          acc += fx45(r[e]);
        });
        C.store(c, r);
      }
    }
  }
  return acc;
}

// range_sum of the weights read from the cache
template <class D>
__device__ __forceinline__ uint64_t range_sum_cached(const CachedRow<D>& C, float den, int c0, int c1, int nthreads) {
  constexpr int U = 4, N = CachedRow<D>::N;
  uint64_t acc = 0;
  for (int cb = c0 + static_cast<int>(threadIdx.x); cb < c1; cb += U * nthreads) {
    float r[U][N];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cb + u * nthreads;
      if (c < c1) C.load(c, r[u]);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = cb + u * nthreads;
#pragma unroll
      for (int e = 0; e < N; ++e)
        if (c < c1 && N * c + e < C.V) acc += fx45(D::rn(r[u][e] / den));
    }
  }
  return acc;
}

// Inverse CDF over chunks [c0, c1) with NT threads: the first index whose
// inclusive weight, added to `base`, exceeds `target`.  With `own_target`
// the target is floor(u * total) of the range itself and base is 0.  Records
// each (round, wave) segment's weight sum, then wave 0 finds the segment and
// scans its 64 chunks.  Returns the index or -1 (to every thread).
// (wchunk(c, g) calls g(e, i, w) with the weight w of each element i = N c + e
// of chunk c below the row's length)
template <int N, class WChunk>
__device__ int pick_in_range(SharedSpec& sh, WChunk&& wchunk, int c0, int c1, bool own_target, float u, uint64_t base,
                             uint64_t target) {
  const int tid = threadIdx.x;
  const int w = tid / WAVE, lane = tid & (WAVE - 1);
  const int nround = (c1 - c0 + NT - 1) / NT;
  for (int k = 0; k < nround; ++k) {
    const int c = c0 + k * NT + tid;
    uint64_t lw = 0;
    if (c < c1) wchunk(c, [&](int, int, float w) { lw += fx45(w); });
    lw = wave_reduce(lw, OpAdd());
    if (lane == 0) sh.seg[k * NWAVE + w] = lw;
  }
  if (tid == 0) sh.token = -1;
  __syncthreads();
  if (tid < WAVE) {
    const int nseg = nround * NWAVE;
    if (own_target) {
      uint64_t W = 0;
      for (int j = lane; j < nseg; j += WAVE) W += sh.seg[j];
      W = wave_reduce(W, OpAdd());
      target = static_cast<uint64_t>(floor(static_cast<double>(u) * static_cast<double>(W)));
      base = 0;
    }
    // first segment whose inclusive sum exceeds target
    int seg = -1;
    for (int j0 = 0; j0 < nseg && seg < 0; j0 += WAVE) {
      const uint64_t v = j0 + lane < nseg ? sh.seg[j0 + lane] : 0ull;
      const uint64_t inc = wave_incl_scan(v);
      const uint64_t m = __ballot(base + inc > target);
      if (m) {
        const int f = __ffsll(static_cast<unsigned long long>(m)) - 1;
        seg = j0 + f;
        base += __shfl(inc - v, f, WAVE);
      } else {
        base += __shfl(inc, WAVE - 1, WAVE);
      }
    }
    if (seg >= 0) {
      // the segment's chunks, one per lane, in ascending order
      const int c = c0 + (seg / NWAVE) * NT + (seg % NWAVE) * WAVE + lane;
      uint64_t wl[N];
      uint64_t lc = 0;
#pragma unroll
      for (int e = 0; e < N; ++e) wl[e] = 0;
      if (c < c1) {
        wchunk(c, [&](int e, int, float w) {
          wl[e] = fx45(w);
          lc += wl[e];
        });
      }
      const uint64_t inc = wave_incl_scan(lc);
      const uint64_t m = __ballot(base + inc > target);
      if (m) {
        const int f = __ffsll(static_cast<unsigned long long>(m)) - 1;
        if (lane == f) {
          uint64_t cc = base + inc - lc;
          int found = -1;
#pragma unroll
          for (int e = 0; e < N; ++e) {
            cc += wl[e];
            if (found < 0 && cc > target) found = N * c + e;
          }
          sh.token = found;
        }
      }
    }
  }
  __syncthreads();
  return sh.token;
}

__device__ __forceinline__ void write_tail(const fl_spec_args& a, int64_t b, int n_acc, int64_t tok) {
  const int64_t K = a.k;
  a.out_n_accepted[b] = n_acc;
  a.out_tokens[b * (K + 1) + n_acc] = tok;
  for (int64_t i = n_acc + 1; i <= K; ++i) a.out_tokens[b * (K + 1) + i] = -1;
}

// Slices of a row pair for the sliced residual path.
__host__ __device__ inline int spec_slices(int64_t batch) {
  int64_t s = batch > 0 ? 2048 / batch : 1;
  return static_cast<int>(s < 1 ? 1 : (s > MAX_SLICES ? MAX_SLICES : s));
}

// Workspace of the sliced path: int32 state[batch] (rejected position or -1),
// padded to 8 bytes, then uint64 part1[batch * S] and part2[batch * S].
// A workspace of at least spec_cache_bytes(batch, vocab) bytes also holds
// the residual cache (float[batch][spec_cache_ld(vocab)], 16-byte aligned).
struct SpecWs {
  int32_t* state;
  uint64_t* part1;
  uint64_t* part2;
  float* cache;  // or nullptr
  int64_t cache_ld;
  int S;
};
__host__ __device__ inline size_t spec_ws_bytes(int64_t batch) {
  const int S = spec_slices(batch);
  return ((static_cast<size_t>(batch) * 4 + 7) & ~static_cast<size_t>(7)) + 16u * static_cast<size_t>(batch) * S;
}
__host__ __device__ inline size_t spec_cache_bytes(int64_t batch, int64_t vocab) {
  return ((spec_ws_bytes(batch) + 15) & ~static_cast<size_t>(15)) +
         4u * static_cast<size_t>(batch) * static_cast<size_t>(spec_cache_ld(vocab));
}
__host__ __device__ inline SpecWs spec_ws(void* p, int64_t batch, size_t bytes, int64_t vocab) {
  SpecWs w;
  w.S = spec_slices(batch);
  w.state = static_cast<int32_t*>(p);
  char* q = static_cast<char*>(p) + ((static_cast<size_t>(batch) * 4 + 7) & ~static_cast<size_t>(7));
  w.part1 = reinterpret_cast<uint64_t*>(q);
  w.part2 = w.part1 + batch * w.S;
  const bool cached = bytes >= spec_cache_bytes(batch, vocab) && (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
  w.cache = cached ? reinterpret_cast<float*>(static_cast<char*>(p) + ((spec_ws_bytes(batch) + 15) & ~static_cast<size_t>(15)))
                   : nullptr;
  w.cache_ld = spec_cache_ld(vocab);
  return w;
}

}  // namespace

// ---------------------------------------------------------------- one work-group per sequence
template <class D>
__global__ __launch_bounds__(NT) void k_spec_verify(const fl_spec_args a) {
  __shared__ SharedSpec sh;
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  if (tid < WAVE) {
    bool rej;
    const int n = accept_walk<D>(a, b, &rej);
    if (tid == 0) {
      sh.n_acc = n;
      sh.rejected = rej ? 1 : 0;
    }
  }
  __syncthreads();
  const int n_acc = sh.n_acc;
  int64_t tok;
  if (!sh.rejected) {
    tok = a.bonus_token[b * (a.k + 1) + a.k];
  } else {
    // residual at position n_acc: pass 1 sums r, pass 2 draws
    const PairRows<D> R(a, b, n_acc);
    const uint64_t lr = range_sum(R, 0, R.nch, NT, [](float p, float q) { return resid_of<D>(p, q); });
    const uint64_t rsum = block_reduce<uint64_t>(lr, OpAdd(), sh.redq);
    const Weight<D> wt(rsum);
    const float U = fminf(fmaxf(a.u_resample[b], 0.0f), 0.99999994f);
    auto wchunk = [&](int c, auto&& g) { R.chunk(c, [&](int e, int i, float p, float q) { g(e, i, wt(p, q)); }); };
    const int t = pick_in_range<PairRows<D>::N>(sh, wchunk, 0, R.nch, true, U, 0, 0);
    tok = t < 0 ? R.V - 1 : t;
  }
  if (tid == 0) write_tail(a, b, n_acc, tok);
}

// ---------------------------------------------------------------- sliced path
// 1. per slice of the rejected position's row pair: sum(r) (PASS2 false), or
//    the sum of the weights (PASS2 true, after every slice's sum(r)).  The
//    first pass starts with the accept walk, in every slice's work-group (a
//    few gathers per sequence, served by L2 after the first): slice 0 writes
//    the walk's outputs, the sequence's state for the later launches and,
//    when every draft is accepted, its tokens; a separate launch for the walk
//    cost 5.5 us of the verify.
template <class D, bool PASS2>
__global__ __launch_bounds__(NT_PART) void k_spec_part(const fl_spec_args a, SpecWs ws) {
  __shared__ uint64_t red[NT_PART / WAVE];
  __shared__ int32_t pos_sh;
  const int64_t b = blockIdx.y;
  const int s = blockIdx.x;
  int pos;
  if constexpr (!PASS2) {
    if (threadIdx.x < WAVE) {
      bool rej;
      const int n = accept_walk<D>(a, b, &rej, s == 0);
      if (threadIdx.x == 0) {
        pos_sh = rej ? n : -1;
        if (s == 0) {
          ws.state[b] = rej ? n : -1;
          if (rej) a.out_n_accepted[b] = n;
          else write_tail(a, b, n, a.bonus_token[b * (a.k + 1) + a.k]);
        }
      }
    }
    __syncthreads();
    pos = pos_sh;
  } else {
    pos = ws.state[b];
  }
  if (pos < 0) return;
  const PairRows<D> R(a, b, pos);
  const int cps = (R.nch + ws.S - 1) / ws.S;
  const int c0 = min(R.nch, s * cps), c1 = min(R.nch, c0 + cps);
  uint64_t v;
  if constexpr (!PASS2) {
    if (ws.cache != nullptr)
      v = range_sum_store(R, CachedRow<D>(ws.cache, ws.cache_ld, b, R.V), c0, c1, NT_PART);
    else
      v = range_sum(R, c0, c1, NT_PART, [](float p, float q) { return resid_of<D>(p, q); });
  } else {
    // sum(r) over the slices: one slice per lane, in every wave
    const int lane = threadIdx.x & (WAVE - 1);
    const uint64_t rsum = wave_reduce(lane < ws.S ? ws.part1[b * ws.S + lane] : 0ull, OpAdd());
    const Weight<D> wt(rsum);
    // (all-zero residuals draw from p: the rows are read again)
    if (ws.cache != nullptr && !wt.use_p)
      v = range_sum_cached(CachedRow<D>(ws.cache, ws.cache_ld, b, R.V), wt.den, c0, c1, NT_PART);
    else
      v = range_sum(R, c0, c1, NT_PART, wt);
  }
  v = block_reduce<uint64_t, OpAdd, NT_PART / WAVE>(v, OpAdd(), red);
  if (threadIdx.x == 0) (PASS2 ? ws.part2 : ws.part1)[b * ws.S + s] = v;
}

// 2. the slice holding floor(u * W), then the member inside it
template <class D>
__global__ __launch_bounds__(NT) void k_spec_pick(const fl_spec_args a, SpecWs ws) {
  __shared__ SharedSpec sh;
  const int64_t b = blockIdx.x;
  const int pos = ws.state[b];
  if (pos < 0) return;
  const PairRows<D> R(a, b, pos);
  // one slice per lane, in every wave: the totals, then the first slice
  // whose inclusive weight exceeds the target (the last slice if none does)
  const int lane = threadIdx.x & (WAVE - 1);
  const uint64_t p1 = lane < ws.S ? ws.part1[b * ws.S + lane] : 0ull;
  const uint64_t p2 = lane < ws.S ? ws.part2[b * ws.S + lane] : 0ull;
  const uint64_t rsum = wave_reduce(p1, OpAdd());
  const uint64_t inc = wave_incl_scan(p2);
  const uint64_t W = readlane64(inc, WAVE - 1);
  const Weight<D> wt(rsum);
  const float U = fminf(fmaxf(a.u_resample[b], 0.0f), 0.99999994f);
  const uint64_t target = static_cast<uint64_t>(floor(static_cast<double>(U) * static_cast<double>(W)));
  const uint64_t hit = __ballot(lane < ws.S - 1 && inc > target);
  const int s = hit ? __ffsll(static_cast<unsigned long long>(hit)) - 1 : ws.S - 1;
  const uint64_t base = readlane64(inc - p2, s);
  const int cps = (R.nch + ws.S - 1) / ws.S;
  const int c0 = min(R.nch, s * cps), c1 = min(R.nch, c0 + cps);
  int t;
  if (ws.cache != nullptr && !wt.use_p) {
    const CachedRow<D> C(ws.cache, ws.cache_ld, b, R.V);
    auto wchunk = [&](int c, auto&& g) { C.weights(c, wt.den, g); };
    t = pick_in_range<PairRows<D>::N>(sh, wchunk, c0, c1, false, U, base, target);
  } else {
    auto wchunk = [&](int c, auto&& g) { R.chunk(c, [&](int e, int i, float p, float q) { g(e, i, wt(p, q)); }); };
    t = pick_in_range<PairRows<D>::N>(sh, wchunk, c0, c1, false, U, base, target);
  }
  if (threadIdx.x == 0) write_tail(a, b, pos, t < 0 ? R.V - 1 : t);
}

size_t spec_workspace_bytes(int64_t batch) { return spec_ws_bytes(batch); }
size_t spec_cache_workspace_bytes(int64_t batch, int64_t vocab) { return spec_cache_bytes(batch, vocab); }

// ---------------------------------------------------------------- scratch that needs no allocation
// The sliced path's workspace for up to FL_SPEC_STATIC_MAX_BATCH sequences
// (20 bytes a sequence at 4096 of them; at most 40 KiB below 2048), one copy on
// each GPU the library runs on, held until the process ends.  Every byte a
// call reads was written earlier in the same call (the first slice pass writes
// each sequence's state, the slice kernels each part they later read), so
// nothing is cleared between calls; calls that overlap on one GPU race.
constexpr size_t SPEC_STATIC_BYTES = 81920;
static __device__ __align__(256) unsigned char scratch[SPEC_STATIC_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES] = {};  // the device address of `scratch`, per device
}  // namespace

size_t spec_static_scratch_bytes() { return SPEC_STATIC_BYTES; }

// The device address of this GPU's `scratch` (the name itself is a host-side
// stand-in, never a device address), looked up once per device with that
// device current.
hipError_t spec_static_scratch(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= MAX_DEVICES) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    if (p == nullptr) return hipErrorInvalidSymbol;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return hipSuccess;
}

hipError_t launch_spec_verify(const fl_spec_args& a, hipStream_t s) {
  return launch_spec_verify_on(a, a.workspace, static_cast<size_t>(a.workspace_bytes), s);
}

hipError_t launch_spec_verify_static(const fl_spec_args& a, hipStream_t s) {
  if (spec_ws_bytes(a.batch) > SPEC_STATIC_BYTES) return hipErrorInvalidValue;  // (the caller checks first)
  void* p = nullptr;
  const hipError_t e = spec_static_scratch(&p);
  if (e != hipSuccess) return e;
  return launch_spec_verify_on(a, p, SPEC_STATIC_BYTES, s);
}

hipError_t launch_spec_verify_on(const fl_spec_args& a, void* workspace, size_t workspace_bytes, hipStream_t s) {
  const bool sliced = workspace != nullptr;
  const SpecWs ws = sliced ? spec_ws(workspace, a.batch, workspace_bytes, a.vocab) : SpecWs{};
  const dim3 grid(static_cast<unsigned>(a.batch));
  auto run = [&](auto tag) {
    using D = decltype(tag);
    if (!sliced) {
      hipLaunchKernelGGL(k_spec_verify<D>, grid, dim3(NT), 0, s, a);
      return;
    }
    const dim3 pgrid(static_cast<unsigned>(ws.S), static_cast<unsigned>(a.batch));
    hipLaunchKernelGGL((k_spec_part<D, false>), pgrid, dim3(NT_PART), 0, s, a, ws);
    hipLaunchKernelGGL((k_spec_part<D, true>), pgrid, dim3(NT_PART), 0, s, a, ws);
    hipLaunchKernelGGL(k_spec_pick<D>, grid, dim3(NT), 0, s, a, ws);
  };
  if (a.dtype == FL_DTYPE_F32) run(F32{});
  else if (a.dtype == FL_DTYPE_BF16) run(BF16{});
  else run(F16{});
  return hipGetLastError();
}

}  // namespace fl
