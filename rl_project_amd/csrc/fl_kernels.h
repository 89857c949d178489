// Host-side launchers of the sampling kernels (one translation unit each).
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/fl_sampler.h"

namespace fl {

// Row samplers: one work-group per row; a.dtype selects the kernel family.
hipError_t launch_sample_rows16(const fl_sample_args& a, hipStream_t s);
hipError_t launch_sample_rows32(const fl_sample_args& a, hipStream_t s);

// Element-wise materialisation of filtered logits / probabilities / masks.
hipError_t launch_apply_filter(const fl_sample_args& a, const fl_row_desc* desc, void* out_filtered, int64_t out_ld,
                               float* out_probs, uint32_t* out_mask, hipStream_t s);

// Speculative accept / residual resample, one work-group per sequence.
hipError_t launch_spec_verify(const fl_spec_args& a, hipStream_t s);
hipError_t launch_spec_verify_on(const fl_spec_args& a, void* workspace, size_t workspace_bytes, hipStream_t s);
size_t spec_workspace_bytes(int64_t batch);
size_t spec_cache_workspace_bytes(int64_t batch, int64_t vocab);
// The same with the library's static device scratch (no allocation).
hipError_t launch_spec_verify_static(const fl_spec_args& a, hipStream_t s);
size_t spec_static_scratch_bytes();
hipError_t launch_row_stats(const fl_row_stats_args& a, hipStream_t s);

// lm_head GEMM with the sampler in its epilogue (prep, gemm, pick).
hipError_t launch_lm_head(const fl_lm_head_args& a, hipStream_t s);
size_t lm_head_workspace_bytes(int64_t batch, int64_t vocab);

}  // namespace fl
