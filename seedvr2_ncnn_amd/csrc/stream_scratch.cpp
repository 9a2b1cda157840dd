// Per-(device, stream) scratch allocations (stream_scratch.h) over the HIP
// runtime, with the ownership rules of scratch_registry.h.
#include "stream_scratch.h"

#include "scratch_registry.h"

namespace s2 {

namespace {

int hip_device(int* dev) { return (int)hipGetDevice(dev); }
int hip_allocate(void** p, size_t bytes) { return (int)hipMalloc(p, bytes); }
int hip_zero(void* p, size_t bytes, void* stream) {
    return (int)hipMemsetAsync(p, 0, bytes, (hipStream_t)stream);
}
int hip_sync(void* stream) { return (int)hipStreamSynchronize((hipStream_t)stream); }
int hip_release(void* p) { return (int)hipFree(p); }

ScratchRegistry& registry() {
    static const ScratchOps ops = {hip_device, hip_allocate, hip_zero, hip_sync, hip_release};
    static ScratchRegistry r(ops);
    return r;
}

hipError_t as_hip(int ret) {
    return ret == ScratchRegistry::kMisuse ? hipErrorInvalidValue : (hipError_t)ret;
}

hipError_t kind_bytes(int kind, size_t* bytes) {
    if (kind == kScratchSplitK) return splitk_scratch_bytes(bytes);
    *bytes = cfg_scratch_bytes();
    return hipSuccess;
}

}  // namespace

hipError_t stream_scratch(ScratchKind kind, hipStream_t stream, size_t bytes, void** out) {
    if ((int)kind < 0 || (int)kind >= kScratchKinds) return hipErrorInvalidValue;
    return as_hip(registry().get((int)kind, stream, bytes, out));
}

hipError_t stream_scratch_acquire(hipStream_t stream) {
    for (int kind = 0; kind < kScratchKinds; kind++) {
        size_t bytes = 0;
        hipError_t e = kind_bytes(kind, &bytes);
        if (e == hipSuccess) e = as_hip(registry().acquire(kind, stream, bytes));
        if (e != hipSuccess) {
            // undo the kinds already taken
            for (int k = 0; k < kind; k++) (void)registry().release(k, stream);
            return e;
        }
    }
    return hipSuccess;
}

hipError_t stream_scratch_release(hipStream_t stream) {
    hipError_t first = hipSuccess;
    for (int kind = 0; kind < kScratchKinds; kind++) {
        const hipError_t e = as_hip(registry().release(kind, stream));
        if (first == hipSuccess) first = e;
    }
    return first;
}

}  // namespace s2
