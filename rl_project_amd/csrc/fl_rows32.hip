// Fused per-row sampler for float32 logits (placeholder until the fp32 path lands).
#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {
hipError_t launch_sample_rows32(const fl_sample_args&, hipStream_t) { return hipErrorNotSupported; }
}  // namespace fl
