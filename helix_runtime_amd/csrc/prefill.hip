// Chunked-prefill attention (MFMA path); filled in by the prefill kernel.
#include "kernels.hpp"

namespace helix::hip {

hipError_t launch_prefill(const PrefillArgs&, hipStream_t) { return hipErrorNotSupported; }

}  // namespace helix::hip
