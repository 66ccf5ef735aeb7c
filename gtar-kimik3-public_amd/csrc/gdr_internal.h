// Host-side declarations shared between the C-ABI layer (gdr_api.hip) and the kernel translation units.
#pragma once

#include <hip/hip_runtime.h>

#include "../../include/gdr.h"

namespace gdr {

// Enqueue the recurrent forward; `a` has been validated.
hipError_t launch_recurrent(const gdr_args& a, hipStream_t stream);

// Enqueue the chunkwise forward; `a` has been validated (q, k, v share one dtype).
hipError_t launch_chunk(const gdr_args& a, hipStream_t stream);

// Chunkwise forward as a chunk-parallel preparation launch plus a state-scan launch over a workspace of
// chunk_workspace_bytes(a) bytes at a.workspace.
int64_t chunk_workspace_bytes(const gdr_args& a);
hipError_t launch_chunk_split(const gdr_args& a, hipStream_t stream);

}  // namespace gdr
