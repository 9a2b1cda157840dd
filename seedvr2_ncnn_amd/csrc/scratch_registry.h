// Ownership rules of the per-(device, stream) scratch that kernels of this
// library share between the workgroups of one launch (split-k partial tiles
// and arrival counters, guidance statistics).  Plain C++: the runtime calls
// come in through ScratchOps, so the rules can be exercised without a GPU.
//
//   acquire  an owner of a stream (a device allocator, a layer's host path)
//            takes a reference when it is created: the first one allocates
//            the scratch and zeroes it, ordered on that stream.  Nothing
//            waits on the host.
//   get      the forward path: returns the entry.  A caller that acquired
//            nothing (a direct C-ABI user) gets one made the same way, kept
//            until the process ends.  Never synchronises.
//   release  drops an owner reference; the last one waits for that stream
//            (its kernels may still read the scratch) and frees the memory,
//            unless a forward made the entry before any owner existed.
//
// Calls on different streams never share scratch; calls on one stream run in
// stream order, so one entry per (device, stream, kind) is enough.
#pragma once

#include <stddef.h>

#include <map>
#include <mutex>
#include <tuple>

namespace s2 {

// Runtime operations; each returns 0 on success.
struct ScratchOps {
    int (*current_device)(int* device);
    int (*allocate)(void** ptr, size_t bytes);
    int (*zero)(void* ptr, size_t bytes, void* stream);   // ordered on stream, no host wait
    int (*synchronize)(void* stream);                      // that stream only
    int (*release)(void* ptr);
};

class ScratchRegistry {
public:
    // Returned when a kind is requested with a size other than its entry's,
    // or an entry without owners is released.
    static const int kMisuse = -1;

    explicit ScratchRegistry(const ScratchOps& ops) : ops_(ops) {}

    int acquire(int kind, void* stream, size_t bytes) {
        std::lock_guard<std::mutex> lock(mutex_);
        Entry* e = 0;
        int ret = find_or_make(kind, stream, bytes, &e);
        if (ret == 0) e->owners++;
        return ret;
    }

    int get(int kind, void* stream, size_t bytes, void** out) {
        std::lock_guard<std::mutex> lock(mutex_);
        Entry* e = 0;
        const bool existed = has(kind, stream);
        int ret = find_or_make(kind, stream, bytes, &e);
        if (ret != 0) return ret;
        if (!existed) e->kept = true;
        *out = e->ptr;
        return 0;
    }

    int release(int kind, void* stream) {
        std::lock_guard<std::mutex> lock(mutex_);
        int dev = 0;
        int ret = ops_.current_device(&dev);
        if (ret != 0) return ret;
        Map::iterator it = map_.find(Key(dev, kind, stream));
        if (it == map_.end() || it->second.owners <= 0) return kMisuse;
        if (--it->second.owners > 0 || it->second.kept) return 0;
        ret = ops_.synchronize(stream);
        if (ret != 0) return ret;
        ret = ops_.release(it->second.ptr);
        map_.erase(it);
        return ret;
    }

    // Introspection (tests): owners of an entry of the current device, or -1
    // when there is none; kept entries report owners + 1000.
    int owners(int kind, void* stream) {
        std::lock_guard<std::mutex> lock(mutex_);
        int dev = 0;
        if (ops_.current_device(&dev) != 0) return -1;
        Map::iterator it = map_.find(Key(dev, kind, stream));
        if (it == map_.end()) return -1;
        return it->second.owners + (it->second.kept ? 1000 : 0);
    }

private:
    struct Entry {
        Entry() : ptr(0), bytes(0), owners(0), kept(false) {}
        void* ptr;
        size_t bytes;
        int owners;
        bool kept;   // made by a forward before any owner: lives until exit
    };
    typedef std::tuple<int, int, void*> Key;
    typedef std::map<Key, Entry> Map;

    bool has(int kind, void* stream) {
        int dev = 0;
        if (ops_.current_device(&dev) != 0) return false;
        return map_.count(Key(dev, kind, stream)) != 0;
    }

    int find_or_make(int kind, void* stream, size_t bytes, Entry** out) {
        int dev = 0;
        int ret = ops_.current_device(&dev);
        if (ret != 0) return ret;
        Entry& e = map_[Key(dev, kind, stream)];
        if (e.ptr) {
            if (e.bytes != bytes) return kMisuse;
            *out = &e;
            return 0;
        }
        void* p = 0;
        ret = ops_.allocate(&p, bytes);
        if (ret == 0) {
            ret = ops_.zero(p, bytes, stream);
            if (ret != 0) ops_.release(p);
        }
        if (ret != 0) {
            map_.erase(Key(dev, kind, stream));
            return ret;
        }
        e.ptr = p;
        e.bytes = bytes;
        *out = &e;
        return 0;
    }

    ScratchOps ops_;
    std::mutex mutex_;
    Map map_;
};

}  // namespace s2
