// ncnn-compatible subset: Allocator.
//
// The layers in ../layers are written against the public API of Tencent ncnn
// (https://github.com/Tencent/ncnn, src/allocator.h, src/mat.h, src/layer.h,
// src/paramdict.h, src/modelbin.h, src/option.h).  ncnn is not available in
// this image, so this directory provides the subset of that API the layers
// and their tests use, with the same names, signatures and semantics.  Built
// against a real ncnn instead, the layer sources compile unchanged.
#ifndef NCNN_ALLOCATOR_H
#define NCNN_ALLOCATOR_H

#include <stddef.h>
#include <stdlib.h>

namespace ncnn {

#define NCNN_MALLOC_ALIGN 64
#define NCNN_MALLOC_OVERREAD 64

static inline size_t alignSize(size_t sz, int n) { return (sz + n - 1) & -n; }

static inline void* fastMalloc(size_t size) {
    void* ptr = 0;
    if (posix_memalign(&ptr, NCNN_MALLOC_ALIGN, size + NCNN_MALLOC_OVERREAD)) ptr = 0;
    return ptr;
}

static inline void fastFree(void* ptr) {
    if (ptr) free(ptr);
}

static inline int NCNN_XADD(int* addr, int delta) {
    return __atomic_fetch_add(addr, delta, __ATOMIC_ACQ_REL);
}

class Allocator {
public:
    virtual ~Allocator();
    virtual void* fastMalloc(size_t size) = 0;
    virtual void fastFree(void* ptr) = 0;
};

}  // namespace ncnn

#endif  // NCNN_ALLOCATOR_H
