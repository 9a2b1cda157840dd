// Device scratch that kernels of this library share between the workgroups of
// one launch (split-k partial tiles and arrival counters, reduction
// statistics).  Each (device, stream) pair gets its own allocation, so calls
// enqueued on different streams never share one; calls on one stream run in
// stream order.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace s2 {

enum ScratchKind {
    kScratchSplitK = 0,   // SharedLinear split-k slots and counters
    kScratchCfg = 1,      // guidance statistics of the CFG rescale
    kScratchKinds = 2
};

// *out = the zero-initialised allocation of `bytes` for (current device,
// stream, kind), made on the first request and kept until the process ends.
// Every request of one kind must ask for the same size.
hipError_t stream_scratch(ScratchKind kind, hipStream_t stream, size_t bytes, void** out);

}  // namespace s2
