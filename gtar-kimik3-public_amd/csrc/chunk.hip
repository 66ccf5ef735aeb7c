// Chunkwise forward: placeholder until the fused kernel lands.
#include "gdr_common.h"
#include "gdr_internal.h"

namespace gdr {
hipError_t launch_chunk(const gdr_args&, hipStream_t) { return hipErrorNotSupported; }
}  // namespace gdr
