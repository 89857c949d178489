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

struct SharedSpec {
  uint64_t redq[NWAVE];
  uint64_t seg[MAX_ROUNDS * NWAVE];  // weight sum of each (round, wave) segment
  int32_t n_acc;
  int32_t rejected;
  int32_t token;
};

}  // namespace

template <class D>
__global__ __launch_bounds__(NT) void k_spec_verify(const fl_spec_args a) {
  __shared__ SharedSpec sh;
  using C = Chunk<D>;
  constexpr int N = C::N;
  const int tid = threadIdx.x;
  const int64_t b = blockIdx.x;
  const int64_t K = a.k;
  const int V = static_cast<int>(a.vocab);
  const float T = a.temperature[b];
  const float cap = a.softcap;
  const size_t esz = D::id == FL_DTYPE_F32 ? 4 : 2;
  const char* tgt_base = static_cast<const char*>(a.target);
  const char* drf_base = static_cast<const char*>(a.draft);
  auto trow = [&](int64_t i) { return tgt_base + (b * (K + 1) + i) * a.ld * esz; };
  auto drow = [&](int64_t i) { return drf_base + (b * K + i) * a.ld * esz; };

  // ------------------------------------------------ accept walk (thread 0)
  if (tid == 0) {
    int n = 0;
    bool rej = false;
    for (int64_t i = 0; i < K; ++i) {
      const int64_t d = a.draft_ids[b * K + i];
      float ratio = 0.0f;
      if (d >= 0 && d < V) {
        const fl_row_desc td = a.target_desc[b * (K + 1) + i];
        const fl_row_desc dd = a.draft_desc[b * K + i];
        const __amdgpu_buffer_rsrc_t rt = row_rsrc(trow(i), static_cast<uint32_t>(V * esz));
        const __amdgpu_buffer_rsrc_t rd = row_rsrc(drow(i), static_cast<uint32_t>(V * esz));
        const float p = prob_of<D>(td, filt_value<D>(C::elem(rt, static_cast<int>(d)), cap, T), d);
        const float q = prob_of<D>(dd, filt_value<D>(C::elem(rd, static_cast<int>(d)), cap, T), d);
        ratio = fminf(1.0f, D::rn(p / D::rn(q + 1e-10f)));
      }
      if (a.out_ratio) a.out_ratio[b * K + i] = ratio;
      if (a.u_accept[b * K + i] < ratio) {
        a.out_tokens[b * (K + 1) + i] = d;
        ++n;
      } else {
        rej = true;
        break;
      }
    }
    if (a.out_ratio)
      for (int64_t i = n + (rej ? 1 : 0); i < K; ++i) a.out_ratio[b * K + i] = __builtin_nanf("");
    sh.n_acc = n;
    sh.rejected = rej ? 1 : 0;
    sh.token = -1;
  }
  __syncthreads();
  const int n_acc = sh.n_acc;
  const bool rejected = sh.rejected != 0;

  int64_t tok;
  if (!rejected) {
    tok = a.bonus_token[b * (K + 1) + K];
  } else {
    // ---------------------------------------------- residual at position n_acc
    const fl_row_desc td = a.target_desc[b * (K + 1) + n_acc];
    const fl_row_desc dd = a.draft_desc[b * K + n_acc];
    const char* tp = trow(n_acc);
    const char* dp = drow(n_acc);
    const __amdgpu_buffer_rsrc_t rt = row_rsrc(tp, static_cast<uint32_t>(V * esz));
    const __amdgpu_buffer_rsrc_t rd = row_rsrc(dp, static_cast<uint32_t>(V * esz));
    const bool aligned = ((reinterpret_cast<uintptr_t>(tp) | reinterpret_cast<uintptr_t>(dp)) & 15u) == 0;
    const int nch = (V + N - 1) / N;
    const int nfull = V / N;
    const int nround = (nch + NT - 1) / NT;
    const int w = tid / WAVE, lane = tid & (WAVE - 1);

    // f(e, i, p_i, q_i) for the N elements of chunk c (ascending index i = N c + e)
    auto chunk = [&](int c, auto&& f) __attribute__((always_inline)) {
      float xt[N], xd[N];
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
#pragma unroll
      for (int e = 0; e < N; ++e) {
        const int i = N * c + e;
        if (i < V) f(e, i, prob_of<D>(td, filt_value<D>(xt[e], cap, T), i), prob_of<D>(dd, filt_value<D>(xd[e], cap, T), i));
      }
    };
    auto resid = [](float p, float q) { return fmaxf(D::rn(p - q), 0.0f); };

    // pass 1: sum(r) in the dtype (:74); chunk c of round k is read by thread
    // c - k * NT, so every wave load covers 64 consecutive chunks
    uint64_t lr = 0;
    for (int k = 0; k < nround; ++k) chunk(k * NT + tid, [&](int, int, float p, float q) { lr += fx45(resid(p, q)); });
    const uint64_t rsum = block_reduce<uint64_t>(lr, OpAdd(), sh.redq);
    const bool use_p = rsum == 0;  // p == q: the oracle's fallback to p
    const float den = D::rn(D::rn(static_cast<float>(static_cast<double>(rsum) * (1.0 / 35184372088832.0))) + 1e-10f);
    auto weight = [&](float p, float q) { return use_p ? p : D::rn(resid(p, q) / den); };

    // pass 2: weight sums per (round, wave) segment, in ascending index order
    for (int k = 0; k < nround; ++k) {
      uint64_t lw = 0;
      chunk(k * NT + tid, [&](int, int, float p, float q) { lw += fx45(weight(p, q)); });
      lw = wave_reduce(lw, OpAdd());
      if (lane == 0) sh.seg[k * NWAVE + w] = lw;
    }
    __syncthreads();
    // wave 0: segment holding the target, then its member by a wave scan
    if (tid < WAVE) {
      const int nseg = nround * NWAVE;
      uint64_t W = 0;
      for (int j = lane; j < nseg; j += WAVE) W += sh.seg[j];
      W = wave_reduce(W, OpAdd());
      const float U = fminf(fmaxf(a.u_resample[b], 0.0f), 0.99999994f);
      const uint64_t target = static_cast<uint64_t>(floor(static_cast<double>(U) * static_cast<double>(W)));
      // first segment whose inclusive sum exceeds target
      uint64_t base = 0;
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
      int found = -1;
      if (seg >= 0) {
        // the segment's chunks, one per lane, in ascending order
        const int c = (seg / NWAVE) * NT + (seg % NWAVE) * WAVE + lane;
        uint64_t wl[N];
        uint64_t lc = 0;
#pragma unroll
        for (int e = 0; e < N; ++e) wl[e] = 0;
        if (c < nch) {
          chunk(c, [&](int e, int, float p, float q) {
            wl[e] = fx45(weight(p, q));
            lc += wl[e];
          });
        }
        const uint64_t inc = wave_incl_scan(lc);
        const uint64_t m = __ballot(base + inc > target);
        if (m) {
          const int f = __ffsll(static_cast<unsigned long long>(m)) - 1;
          if (lane == f) {
            uint64_t cc = base + inc - lc;
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
    tok = sh.token < 0 ? V - 1 : sh.token;
  }

  // ------------------------------------------------ outputs
  if (tid == 0) {
    a.out_n_accepted[b] = n_acc;
    a.out_tokens[b * (K + 1) + n_acc] = tok;
    for (int64_t i = n_acc + 1; i <= K; ++i) a.out_tokens[b * (K + 1) + i] = -1;
  }
}

hipError_t launch_spec_verify(const fl_spec_args& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.batch)), block(NT);
  if (a.dtype == FL_DTYPE_F32) hipLaunchKernelGGL(k_spec_verify<F32>, grid, block, 0, s, a);
  else if (a.dtype == FL_DTYPE_BF16) hipLaunchKernelGGL(k_spec_verify<BF16>, grid, block, 0, s, a);
  else hipLaunchKernelGGL(k_spec_verify<F16>, grid, block, 0, s, a);
  return hipGetLastError();
}

}  // namespace fl
