// Device-resident blobs for the MI355X layers.
//
// A device blob is an ncnn::Mat over external HIP device memory whose
// `allocator` member points at a HipDeviceAllocator; the layers see that tag
// and run zero-copy on the device, on the allocator's stream.  Blobs made by
// create_blob() are owned by the allocator until clear() or its destruction
// (ncnn::Mat itself never frees external data).  Host Mats (any other
// allocator) take the staged path: upload, compute, download, synchronise.
//
// Never pass a HipDeviceAllocator to ncnn::Mat::create: upstream ncnn keeps
// the reference count at the end of the data block and would write it from
// the host into device memory.  fastMalloc therefore refuses (returns 0).
#ifndef SEEDVR2_HIP_ALLOCATOR_H
#define SEEDVR2_HIP_ALLOCATOR_H

#include <mutex>
#include <vector>

#include <allocator.h>
#include <mat.h>
#include <option.h>

#include "seedvr2_hip.h"

namespace seedvr2 {

// One owner reference to a stream's kernel scratch (split-k partial tiles,
// guidance statistics; s2_stream_scratch_acquire): taken by take() when a
// gfx950 device is present (a no-op without one), dropped by drop() or the
// destructor.  Owners: every HipDeviceAllocator for its stream, and each
// layer whose host-blob path runs on the default stream, from
// create_pipeline to destroy_pipeline.  So the scratch is allocated and
// zeroed when an owner is made, never inside a forward.
class StreamScratchRef {
public:
    StreamScratchRef() : stream_(0), held_(false) {}
    ~StreamScratchRef() { drop(); }
    int take(void* stream);   // S2_OK, or the acquire's error code
    void drop();
    bool held() const { return held_; }

private:
    StreamScratchRef(const StreamScratchRef&);
    StreamScratchRef& operator=(const StreamScratchRef&);
    void* stream_;
    bool held_;
};

class HipDeviceAllocator : public ncnn::Allocator {
public:
    // stream: a hipStream_t (as void*), 0 = the default stream.  Takes the
    // stream's kernel scratch (StreamScratchRef) for as long as it lives.
    explicit HipDeviceAllocator(void* stream = 0);
    virtual ~HipDeviceAllocator();

    virtual void* fastMalloc(size_t size);
    virtual void fastFree(void* ptr);

    // Device Mat (dims 2: w x h, elemsize 4 = fp32, 2 = bf16 or fp16, see
    // device_blob_dtype) owned by this allocator.  Empty on allocation failure.
    ncnn::Mat create_blob(int w, int h, size_t elemsize);
    // 4-D device Mat (w, h, d, c) with ncnn's channel stride (each channel
    // rounded up to 16 bytes), owned by this allocator.
    ncnn::Mat create_blob(int w, int h, int d, int c, size_t elemsize);
    // Wraps caller-owned device memory as a device blob (not owned).
    ncnn::Mat wrap_blob(int w, int h, void* device_data, size_t elemsize);
    ncnn::Mat wrap_blob(int w, int h, int d, int c, void* device_data, size_t elemsize);
    // Returns a blob this allocator created to its pool of free blocks (a
    // no-op for other pointers).  The next create_blob of the same byte size
    // reuses the block without synchronising: safe when every kernel that
    // touches this allocator's blobs runs on its stream, in order, as the
    // graph executor's layers do.
    void release_blob(void* ptr);
    // Frees every blob this allocator created, pooled blocks included.
    void clear();

    void* stream() const { return stream_; }
    // Blocks this allocator holds, in use or pooled (for tests).
    size_t owned_count() const {
        std::lock_guard<std::mutex> lock(mutex_);
        return owned_.size();
    }

private:
    void* alloc_bytes(size_t bytes);

    void* stream_;
    StreamScratchRef scratch_;
    mutable std::mutex mutex_;
    std::vector<void*> owned_;
    std::vector<size_t> owned_bytes_;
    std::vector<std::pair<size_t, void*> > pool_;   // (bytes, block) free for reuse
};

// True when m is a device blob (its allocator is a HipDeviceAllocator).
HipDeviceAllocator* device_allocator_of(const ncnn::Mat& m);

// Element type of a device blob: elemsize 4 is fp32; elemsize 2 follows
// ncnn's 16-bit storage options, as the reference Vulkan path's blobs of
// elembits 16 do (adaptive_window_attention.cpp:1082-1087): fp16 when only
// use_fp16_storage is set, bf16 otherwise (use_bf16_storage, or neither).
inline s2_dtype device_blob_dtype(size_t elemsize, const ncnn::Option& opt)
{
    if (elemsize == 4)
        return S2_DTYPE_F32;
    return opt.use_fp16_storage && !opt.use_bf16_storage ? S2_DTYPE_F16 : S2_DTYPE_BF16;
}

// Return code of a layer entry point.  The reference layers return 0, -1
// (invalid configuration, shape or arity), -2 (plan inconsistency) or -100
// (allocation or weight-load failure); ncnn callers handle only those.  A
// HIP runtime failure or a missing gfx950 device (S2_ERR_DEVICE at the
// C-ABI) is therefore reported as -100, and s2_last_error() keeps the detail.
inline int layer_status(int ret)
{
    return (ret == S2_OK || ret == S2_ERR_INVALID || ret == S2_ERR_PLAN) ? ret : S2_ERR_ALLOC;
}

// Device buffer that only grows; used for layer workspaces and staging.
class DeviceBuffer {
public:
    DeviceBuffer() : ptr_(0), bytes_(0) {}
    ~DeviceBuffer();
    int reserve(size_t bytes);   // S2_OK or S2_ERR_ALLOC / S2_ERR_DEVICE
    void release();
    void* get() const { return ptr_; }
    size_t size() const { return bytes_; }

private:
    DeviceBuffer(const DeviceBuffer&);
    DeviceBuffer& operator=(const DeviceBuffer&);
    void* ptr_;
    size_t bytes_;
};

}  // namespace seedvr2

#endif  // SEEDVR2_HIP_ALLOCATOR_H
