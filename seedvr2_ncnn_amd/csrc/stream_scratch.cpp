// Per-(device, stream) scratch allocations (stream_scratch.h).
#include "stream_scratch.h"

#include <map>
#include <mutex>
#include <tuple>

namespace s2 {

namespace {

struct Entry {
    void* ptr = nullptr;
    size_t bytes = 0;
};

std::mutex g_mutex;
std::map<std::tuple<int, int, hipStream_t>, Entry> g_scratch;

}  // namespace

hipError_t stream_scratch(ScratchKind kind, hipStream_t stream, size_t bytes, void** out) {
    int dev = 0;
    hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return e;
    if ((int)kind < 0 || (int)kind >= kScratchKinds) return hipErrorInvalidValue;
    std::lock_guard<std::mutex> lock(g_mutex);
    Entry& en = g_scratch[std::make_tuple(dev, (int)kind, stream)];
    if (!en.ptr) {
        void* p = nullptr;
        e = hipMalloc(&p, bytes);
        if (e != hipSuccess) return e;
        // zeroed before any kernel of this stream can use it
        e = hipMemset(p, 0, bytes);
        if (e == hipSuccess) e = hipDeviceSynchronize();
        if (e != hipSuccess) {
            (void)hipFree(p);
            return e;
        }
        en.ptr = p;
        en.bytes = bytes;
    } else if (en.bytes < bytes) {
        return hipErrorInvalidValue;
    }
    *out = en.ptr;
    return hipSuccess;
}

}  // namespace s2
