// Speculative verify (placeholder until the verify kernel lands).
#include "fl_device.h"
#include "fl_kernels.h"

namespace fl {
hipError_t launch_spec_verify(const fl_spec_args&, hipStream_t) { return hipErrorNotSupported; }
}  // namespace fl
