#include "hip_allocator.h"

#include <algorithm>

#include "seedvr2_hip.h"

namespace seedvr2 {

int StreamScratchRef::take(void* stream) {
    if (held_) {
        if (stream == stream_) return S2_OK;
        drop();
    }
    int devices = 0;
    if (s2_device_count(&devices) != S2_OK || devices == 0) return S2_OK;
    const int ret = s2_stream_scratch_acquire(stream);
    if (ret != S2_OK) return ret;
    stream_ = stream;
    held_ = true;
    return S2_OK;
}

void StreamScratchRef::drop() {
    if (!held_) return;
    held_ = false;
    (void)s2_stream_scratch_release(stream_);
}

// (a failed acquire leaves the scratch to the first forward that needs it)
HipDeviceAllocator::HipDeviceAllocator(void* stream) : stream_(stream) { (void)scratch_.take(stream); }

HipDeviceAllocator::~HipDeviceAllocator() {
    clear();
    scratch_.drop();
}

void* HipDeviceAllocator::fastMalloc(size_t) { return 0; }

void HipDeviceAllocator::fastFree(void* ptr) {
    std::lock_guard<std::mutex> lock(mutex_);
    std::vector<void*>::iterator it = std::find(owned_.begin(), owned_.end(), ptr);
    if (it != owned_.end()) {
        for (size_t i = 0; i < pool_.size(); i++)
            if (pool_[i].second == ptr) {
                pool_.erase(pool_.begin() + i);
                break;
            }
        s2_free(ptr);
        owned_bytes_.erase(owned_bytes_.begin() + (it - owned_.begin()));
        owned_.erase(it);
    }
}

// A pooled block of exactly `bytes`, or a new allocation.
void* HipDeviceAllocator::alloc_bytes(size_t bytes) {
    {
        std::lock_guard<std::mutex> lock(mutex_);
        for (size_t i = 0; i < pool_.size(); i++)
            if (pool_[i].first == bytes) {
                void* p = pool_[i].second;
                pool_.erase(pool_.begin() + i);
                return p;
            }
    }
    void* p = 0;
    if (s2_malloc(&p, bytes) != S2_OK || !p) return 0;
    std::lock_guard<std::mutex> lock(mutex_);
    owned_.push_back(p);
    owned_bytes_.push_back(bytes);
    return p;
}

void HipDeviceAllocator::release_blob(void* ptr) {
    std::lock_guard<std::mutex> lock(mutex_);
    std::vector<void*>::iterator it = std::find(owned_.begin(), owned_.end(), ptr);
    if (it == owned_.end()) return;
    for (size_t i = 0; i < pool_.size(); i++)
        if (pool_[i].second == ptr) return;
    pool_.push_back(std::make_pair(owned_bytes_[it - owned_.begin()], ptr));
}

ncnn::Mat HipDeviceAllocator::create_blob(int w, int h, size_t elemsize) {
    if (w <= 0 || h <= 0 || (elemsize != 2 && elemsize != 4)) return ncnn::Mat();
    void* p = alloc_bytes((size_t)w * h * elemsize);
    if (!p) return ncnn::Mat();
    return ncnn::Mat(w, h, p, elemsize, this);
}

ncnn::Mat HipDeviceAllocator::wrap_blob(int w, int h, void* device_data, size_t elemsize) {
    return ncnn::Mat(w, h, device_data, elemsize, this);
}

ncnn::Mat HipDeviceAllocator::create_blob(int w, int h, int d, int c, size_t elemsize) {
    if (w <= 0 || h <= 0 || d <= 0 || c <= 0 || (elemsize != 2 && elemsize != 4)) return ncnn::Mat();
    ncnn::Mat shape(w, h, d, c, (void*)0, elemsize, this);
    void* p = alloc_bytes(shape.cstep * c * elemsize);
    if (!p) return ncnn::Mat();
    return ncnn::Mat(w, h, d, c, p, elemsize, this);
}

ncnn::Mat HipDeviceAllocator::wrap_blob(int w, int h, int d, int c, void* device_data,
                                        size_t elemsize) {
    return ncnn::Mat(w, h, d, c, device_data, elemsize, this);
}

void HipDeviceAllocator::clear() {
    std::lock_guard<std::mutex> lock(mutex_);
    if (!owned_.empty()) s2_stream_synchronize(stream_);
    for (size_t i = 0; i < owned_.size(); i++) s2_free(owned_[i]);
    owned_.clear();
    owned_bytes_.clear();
    pool_.clear();
}

HipDeviceAllocator* device_allocator_of(const ncnn::Mat& m) {
    return dynamic_cast<HipDeviceAllocator*>(m.allocator);
}

DeviceBuffer::~DeviceBuffer() { release(); }

int DeviceBuffer::reserve(size_t bytes) {
    if (bytes <= bytes_) return S2_OK;
    release();
    void* p = 0;
    const int ret = s2_malloc(&p, bytes);
    if (ret != S2_OK) return ret;
    ptr_ = p;
    bytes_ = bytes;
    return S2_OK;
}

void DeviceBuffer::release() {
    if (ptr_) s2_free(ptr_);
    ptr_ = 0;
    bytes_ = 0;
}

}  // namespace seedvr2
