// Full-distribution statistics of logits rows in one streaming pass:
//   token log-probability   -cross_entropy(x.float(), label)
//                           (src/forgeline/models/policy.py:47-50)
//   entropy                 -(softmax * log_softmax).sum(-1)
//                           (src/forgeline/training/common/logprobs.py:65-68)
//   KL(new || ref)          (p_new * (log p_new - log p_ref)).sum(-1)
//                           (src/forgeline/training/common/logprobs.py:58-62)
// all in float32 as the reference's .float() computes them.
//
// One work-group of 256 threads per row; the row streams through 16-byte
// chunks interleaved over the threads (coalesced), 4 chunks per thread in
// flight.  Each thread keeps, relative to its running maximum m of the row x,
//   s = sum exp(x - m),  u = sum exp(x - m) (x - m),
// and with a reference row y (running maximum m') also
//   s' = sum exp(y - m'),  w = sum exp(x - m) ((x - m) - (y - m')),
// in float64, rescaled when a maximum grows.  The partials merge in a fixed
// tree, so results are deterministic.  With M, S the row's maximum and sum:
//   log p(label) = x_label - M - log S
//   entropy      = log S - u / S
//   KL           = w / S - log S + log S'
// A -inf logit contributes exp(-inf) * (-inf) = NaN to u and w, as 0 * -inf
// does in the reference's expression.
#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {

namespace {

constexpr int NT_RS = 256;
constexpr int NW_RS = NT_RS / WAVE;
constexpr float LOG2E_F = 1.44269504088896340736f;
constexpr double LN2_D = 0.69314718055994530942;

template <class D>
struct RowChunk;
template <>
struct RowChunk<F32> {
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
struct RowChunk16 {
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
struct RowChunk<BF16> : RowChunk16<BF16> {};
template <>
struct RowChunk<F16> : RowChunk16<F16> {};

// Running state of one row for one thread (or a merged set of threads).
struct Acc {
  float m;    // running maximum of x (-inf: nothing yet)
  double s;   // sum exp(x - m)
  double u;   // sum exp(x - m) (x - m)
  float my;   // running maximum of y
  double sy;  // sum exp(y - my)
  double w;   // sum exp(x - m) ((x - m) - (y - my))
};

// Re-base a partial on a larger maximum M (m <= M).  A partial with no
// element yet (m == -inf) has zero sums and stays zero.
__device__ __forceinline__ void rebase_x(Acc& a, float M) {
  if (a.m == M || a.m == -__builtin_inff()) {
    a.m = M;
    return;
  }
  const double d = static_cast<double>(a.m) - static_cast<double>(M);
  const double f = exp(d);
  a.u = (a.u + a.s * d) * f;
  a.w = (a.w + a.s * d) * f;
  a.s *= f;
  a.m = M;
}
__device__ __forceinline__ void rebase_y(Acc& a, float M) {
  if (a.my == M || a.my == -__builtin_inff()) {
    a.my = M;
    return;
  }
  const double d = static_cast<double>(a.my) - static_cast<double>(M);
  // (x - m) - (y - M) = (x - m) - (y - my) - d
  a.w -= a.s * d;
  a.sy *= exp(d);
  a.my = M;
}

__device__ __forceinline__ void merge(Acc& a, Acc b, bool kl) {
  const float M = fmaxf(a.m, b.m);
  rebase_x(a, M);
  rebase_x(b, M);
  if (kl) {
    const float My = fmaxf(a.my, b.my);
    rebase_y(a, My);
    rebase_y(b, My);
    a.sy += b.sy;
    a.w += b.w;
  }
  a.s += b.s;
  a.u += b.u;
}

__device__ __forceinline__ Acc shfl_acc(const Acc& a, int src) {
  Acc r;
  r.m = __shfl(a.m, src, WAVE);
  r.s = __shfl(a.s, src, WAVE);
  r.u = __shfl(a.u, src, WAVE);
  r.my = __shfl(a.my, src, WAVE);
  r.sy = __shfl(a.sy, src, WAVE);
  r.w = __shfl(a.w, src, WAVE);
  return r;
}

}  // namespace

template <class D, bool KL>
__global__ __launch_bounds__(NT_RS) void k_row_stats(const fl_row_stats_args a) {
  using C = RowChunk<D>;
  constexpr int N = C::N;
  constexpr int U_RS = 4;  // chunks per thread in flight (8 lowers the occupancy and the bandwidth)
  __shared__ Acc part[NW_RS];
  const int tid = threadIdx.x;
  const int64_t r = blockIdx.x;
  const int V = static_cast<int>(a.vocab);
  const size_t esz = D::id == FL_DTYPE_F32 ? 4 : 2;
  const char* xp = static_cast<const char*>(a.logits) + r * a.ld * esz;
  const char* yp = KL ? static_cast<const char*>(a.ref_logits) + r * a.ref_ld * esz : xp;
  const __amdgpu_buffer_rsrc_t rx = row_rsrc(xp, static_cast<uint32_t>(V * esz));
  const __amdgpu_buffer_rsrc_t ry = row_rsrc(yp, static_cast<uint32_t>(V * esz));
  const bool aligned = ((reinterpret_cast<uintptr_t>(xp) | reinterpret_cast<uintptr_t>(yp)) & 15u) == 0;
  const int nch = (V + N - 1) / N;
  const int nfull = V / N;

  Acc acc = {-__builtin_inff(), 0.0, 0.0, -__builtin_inff(), 0.0, 0.0};
  auto load = [&](__amdgpu_buffer_rsrc_t rs, int c, float (&x)[N]) __attribute__((always_inline)) {
    if (aligned && c < nfull) {
      C::unpack(buf_load16_once(rs, 16u * c, 0u), x);  // (read once: 207 -> 201 us at 4096 x 128256 bf16)
    } else {
#pragma unroll
      for (int e = 0; e < N; ++e) x[e] = N * c + e < V ? C::elem(rs, N * c + e) : -__builtin_inff();
    }
  };
  for (int c0 = 0; c0 < nch; c0 += U_RS * NT_RS) {
    float xs[U_RS][N], ys[U_RS][N];
#pragma unroll
    for (int k = 0; k < U_RS; ++k) {
      const int c = c0 + k * NT_RS + tid;
      if (c < nch) {
        load(rx, c, xs[k]);
        if (KL) load(ry, c, ys[k]);
      } else {
#pragma unroll
        for (int e = 0; e < N; ++e) xs[k][e] = ys[k][e] = -__builtin_inff();
      }
    }
    // maxima of the iteration's chunks first: at most one re-base per
    // iteration (padding is -inf)
    float cm = xs[0][0], cmy = ys[0][0];
#pragma unroll
    for (int k = 0; k < U_RS; ++k)
#pragma unroll
      for (int e = 0; e < N; ++e) {
        cm = fmaxf(cm, xs[k][e]);
        if (KL) cmy = fmaxf(cmy, ys[k][e]);
      }
    if (cm > acc.m) rebase_x(acc, cm);
    if (KL && cmy > acc.my) rebase_y(acc, cmy);
    // exponents in base 2: d2 = (x - m) log2(e) in one rounding; the base-2
    // sums of the iteration (at most U_RS * N terms, each at most 1) are
    // scaled to natural units and added to the float64 partials once
    const float mb = acc.m * LOG2E_F, myb = acc.my * LOG2E_F;
    float fs = 0.0f, fu = 0.0f, fsy = 0.0f, fw = 0.0f;
    const bool finite_max = acc.m != -__builtin_inff() && (!KL || acc.my != -__builtin_inff());
    if (c0 + (U_RS - 1) * NT_RS + tid < nfull && finite_max) {
      // whole chunks under a finite maximum: -inf gives d2 = -inf, e = 0 and
      // e * d2 = NaN, the reference's 0 * -inf
#pragma unroll
      for (int k = 0; k < U_RS; ++k)
#pragma unroll
        for (int e = 0; e < N; ++e) {
          const float d2 = fmaf(xs[k][e], LOG2E_F, -mb);
          const float ex = __builtin_amdgcn_exp2f(d2);
          fs += ex;
          fu = fmaf(ex, d2, fu);
          if (KL) {
            const float dy2 = fmaf(ys[k][e], LOG2E_F, -myb);
            fsy += __builtin_amdgcn_exp2f(dy2);
            fw = fmaf(ex, d2 - dy2, fw);
          }
        }
    } else {
      // the row's last chunks (partial or past the row) and values before any
      // finite one (-inf below a maximum that is still -inf)
#pragma unroll
      for (int k = 0; k < U_RS; ++k) {
        const int c = c0 + k * NT_RS + tid;
#pragma unroll
        for (int e = 0; e < N; ++e) {
          if (N * c + e >= V) continue;
          const float d2 = xs[k][e] == -__builtin_inff() ? -__builtin_inff() : fmaf(xs[k][e], LOG2E_F, -mb);
          const float ex = __builtin_amdgcn_exp2f(d2);
          fs += ex;
          fu += ex * d2;
          if (KL) {
            const float dy2 = ys[k][e] == -__builtin_inff() ? -__builtin_inff() : fmaf(ys[k][e], LOG2E_F, -myb);
            fsy += __builtin_amdgcn_exp2f(dy2);
            fw += ex * (d2 - dy2);
          }
        }
      }
    }
    acc.s += fs;
    acc.u += static_cast<double>(fu) * LN2_D;
    if (KL) {
      acc.sy += fsy;
      acc.w += static_cast<double>(fw) * LN2_D;
    }
  }
  // merge: wave tree, then the waves in order
#pragma unroll
  for (int off = WAVE / 2; off > 0; off >>= 1) {
    const Acc o = shfl_acc(acc, (tid & (WAVE - 1)) ^ off);
    merge(acc, o, KL);
  }
  if ((tid & (WAVE - 1)) == 0) part[tid / WAVE] = acc;
  __syncthreads();
  if (tid != 0) return;
  Acc t = part[0];
#pragma unroll
  for (int i = 1; i < NW_RS; ++i) merge(t, part[i], KL);
  const double logS = log(t.s);
  if (a.out_entropy) a.out_entropy[r] = static_cast<float>(logS - t.u / t.s);
  if (a.out_lse) a.out_lse[r] = static_cast<float>(static_cast<double>(t.m) + logS);
  if (KL && a.out_kl) a.out_kl[r] = static_cast<float>(t.w / t.s - logS + log(t.sy));
  if (a.labels && a.out_logprob) {
    const int64_t lab = a.labels[r];
    float lp;
    if (lab == a.ignore_index) lp = -0.0f;  // -(cross_entropy = 0) for an ignored target
    else if (lab < 0 || lab >= V) lp = __builtin_nanf("");
    else lp = static_cast<float>(static_cast<double>(C::elem(rx, static_cast<int>(lab))) - static_cast<double>(t.m) - logS);
    a.out_logprob[r] = lp;
  }
}

hipError_t launch_row_stats(const fl_row_stats_args& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.rows)), block(NT_RS);
  const bool kl = a.ref_logits != nullptr;
  if (a.dtype == FL_DTYPE_F32) {
    if (kl) hipLaunchKernelGGL((k_row_stats<F32, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_row_stats<F32, false>), grid, block, 0, s, a);
  } else if (a.dtype == FL_DTYPE_BF16) {
    if (kl) hipLaunchKernelGGL((k_row_stats<BF16, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_row_stats<BF16, false>), grid, block, 0, s, a);
  } else {
    if (kl) hipLaunchKernelGGL((k_row_stats<F16, true>), grid, block, 0, s, a);
    else hipLaunchKernelGGL((k_row_stats<F16, false>), grid, block, 0, s, a);
  }
  return hipGetLastError();
}

}  // namespace fl
