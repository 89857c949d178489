// Element-wise materialisation of the filtered distribution from per-row
// descriptors: what apply_sampling_filters returns
// (src/forgeline/models/generation/sampling.py:16-53), its softmax, or a
// keep bit-mask.  Two launches: a streaming pass over every element with the
// un-penalised value, then a fix-up pass over each row's history ids (their
// penalised value decides; duplicate ids write identical results).
#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {

namespace {

constexpr int APPLY_NT = 256;

template <class D>
struct Load;
template <>
struct Load<F32> {
  __device__ static float at(const void* p, int64_t i) { return static_cast<const float*>(p)[i]; }
  __device__ static void store(void* p, int64_t i, float v) { static_cast<float*>(p)[i] = v; }
};
template <>
struct Load<BF16> {
  __device__ static float at(const void* p, int64_t i) { return BF16::to_f32(static_cast<const uint16_t*>(p)[i]); }
  __device__ static void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(BF16::from_f32(v));
  }
};
template <>
struct Load<F16> {
  __device__ static float at(const void* p, int64_t i) { return F16::to_f32(static_cast<const uint16_t*>(p)[i]); }
  __device__ static void store(void* p, int64_t i, float v) {
    static_cast<uint16_t*>(p)[i] = static_cast<uint16_t>(F16::from_f32(v));
  }
};

template <class D>
__device__ __forceinline__ float prob_of(const fl_row_desc& ds, float y) {
  if (D::id == FL_DTYPE_F32) return static_cast<float>(exp(static_cast<double>(y) - ds.shift) / ds.mass);
  return D::rn(expf(y - ds.shift) * ds.inv_mass);
}

__device__ __forceinline__ bool kept_of(const fl_row_desc& ds, float y, int64_t i) {
  // an element whose value is -inf is filtered whatever the cut
  return ds.status == 0 && y > -__builtin_inff() && (y > ds.y_cut || (y == ds.y_cut && i <= ds.idx_cut));
}

template <class D>
__global__ __launch_bounds__(APPLY_NT) void k_apply(const fl_sample_args a, const fl_row_desc* desc,
                                                    void* out_filtered, int64_t out_ld, float* out_probs,
                                                    uint32_t* out_mask) {
  const int64_t b = blockIdx.y;
  const int64_t i = static_cast<int64_t>(blockIdx.x) * APPLY_NT + threadIdx.x;
  const int64_t V = a.vocab;
  const fl_row_desc ds = desc[b];
  const float T = a.temperature ? a.temperature[b] : 1.0f;
  bool keep = false;
  float y = 0.0f;
  if (i < V) {
    float z = Load<D>::at(a.logits, b * a.ld + i);
    if (a.softcap > 0.0f) z = softcap_val<D>(z, a.softcap);
    y = temperature_val<D>(z, T);
    keep = kept_of(ds, y, i);
    if (out_filtered) Load<D>::store(out_filtered, b * out_ld + i, keep ? y : -__builtin_inff());
    if (out_probs) out_probs[b * V + i] = keep ? prob_of<D>(ds, y) : 0.0f;
  }
  if (out_mask) {
    const uint64_t m = __ballot(keep);
    const int lane = threadIdx.x & (WAVE - 1);
    const int64_t w0 = (static_cast<int64_t>(blockIdx.x) * APPLY_NT + (threadIdx.x & ~(WAVE - 1))) / 32;
    const int64_t nw = (V + 31) / 32;
    uint32_t* mrow = out_mask + b * nw;
    if (lane == 0 && w0 < nw) mrow[w0] = static_cast<uint32_t>(m);
    if (lane == 32 && w0 + 1 < nw) mrow[w0 + 1] = static_cast<uint32_t>(m >> 32);
  }
}

template <class D>
__global__ __launch_bounds__(APPLY_NT) void k_apply_history(const fl_sample_args a, const fl_row_desc* desc,
                                                            void* out_filtered, int64_t out_ld, float* out_probs,
                                                            uint32_t* out_mask) {
  const int64_t b = blockIdx.x;
  const float RP = a.rep_penalty ? a.rep_penalty[b] : 1.0f;
  if (RP == 1.0f || a.hist_ids == nullptr || a.hist_len == nullptr) return;
  const int H = min(a.hist_len[b], FL_MAX_HISTORY);
  const fl_row_desc ds = desc[b];
  const float T = a.temperature ? a.temperature[b] : 1.0f;
  const int64_t V = a.vocab;
  const int32_t* hid = a.hist_ids + b * a.hist_ld;
  for (int i = threadIdx.x; i < H; i += APPLY_NT) {
    const int64_t id = hid[i];
    if (id < 0 || id >= V) continue;
    float z = Load<D>::at(a.logits, b * a.ld + id);
    if (a.softcap > 0.0f) z = softcap_val<D>(z, a.softcap);
    const float y = temperature_val<D>(penalty_val<D>(z, RP), T);
    const bool keep = kept_of(ds, y, id);
    if (out_filtered) Load<D>::store(out_filtered, b * out_ld + id, keep ? y : -__builtin_inff());
    if (out_probs) out_probs[b * V + id] = keep ? prob_of<D>(ds, y) : 0.0f;
    if (out_mask) {
      uint32_t* w = out_mask + b * ((V + 31) / 32) + id / 32;
      const uint32_t bit = 1u << (id & 31);
      if (keep) atomicOr(w, bit);
      else atomicAnd(w, ~bit);
    }
  }
}

template <class D>
hipError_t launch_apply_t(const fl_sample_args& a, const fl_row_desc* desc, void* f, int64_t ld, float* p, uint32_t* m,
                          hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.vocab + APPLY_NT - 1) / APPLY_NT), static_cast<unsigned>(a.batch));
  hipLaunchKernelGGL(k_apply<D>, grid, dim3(APPLY_NT), 0, s, a, desc, f, ld, p, m);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(k_apply_history<D>, dim3(static_cast<unsigned>(a.batch)), dim3(APPLY_NT), 0, s, a, desc, f, ld, p,
                     m);
  return hipGetLastError();
}

}  // namespace

hipError_t launch_apply_filter(const fl_sample_args& a, const fl_row_desc* desc, void* out_filtered, int64_t out_ld,
                               float* out_probs, uint32_t* out_mask, hipStream_t s) {
  if (a.dtype == FL_DTYPE_F32) return launch_apply_t<F32>(a, desc, out_filtered, out_ld, out_probs, out_mask, s);
  if (a.dtype == FL_DTYPE_BF16) return launch_apply_t<BF16>(a, desc, out_filtered, out_ld, out_probs, out_mask, s);
  return launch_apply_t<F16>(a, desc, out_filtered, out_ld, out_probs, out_mask, s);
}

}  // namespace fl
