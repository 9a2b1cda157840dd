// Device scratch that kernels of this library share between the workgroups of
// one launch (split-k partial tiles and arrival counters, reduction
// statistics).  Each (device, stream) pair gets its own allocation, so calls
// enqueued on different streams never share one; calls on one stream run in
// stream order.  The ownership rules are scratch_registry.h's: owners of a
// stream acquire its scratch when they are created (stream_scratch_acquire),
// forward calls only look it up (stream_scratch), and the last owner's
// release frees it.
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
// stream, kind).  When no owner has acquired it, it is made here, zeroed on
// `stream` without a host wait, and kept until the process ends.  Every
// request of one kind must ask for the same size.
hipError_t stream_scratch(ScratchKind kind, hipStream_t stream, size_t bytes, void** out);

// One owner reference to every kind of scratch of (current device, stream),
// made and zeroed on the stream now if it does not exist yet; released by
// stream_scratch_release, whose last call waits for the stream and frees it.
hipError_t stream_scratch_acquire(hipStream_t stream);
hipError_t stream_scratch_release(hipStream_t stream);

// Sizes of the kinds on the current device.
hipError_t splitk_scratch_bytes(size_t* bytes);
size_t cfg_scratch_bytes();

}  // namespace s2
