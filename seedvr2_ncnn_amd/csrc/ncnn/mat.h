// ncnn-compatible subset: Mat (see allocator.h for the scope of this directory).
//
// Same members and semantics as ncnn::Mat for dims 1..4: w is the fastest
// dimension, a 2-D Mat is h contiguous rows of w elements, cstep is the
// channel stride in elements (16-byte aligned for dims >= 3), elemsize is
// the byte size of one element.  Mats are reference counted; a Mat built
// over external data does not own it.
#ifndef NCNN_MAT_H
#define NCNN_MAT_H

#include <string.h>

#include "allocator.h"

namespace ncnn {

class Mat {
public:
    Mat();
    explicit Mat(int w, size_t elemsize = 4u, Allocator* allocator = 0);
    Mat(int w, int h, size_t elemsize = 4u, Allocator* allocator = 0);
    Mat(int w, int h, int c, size_t elemsize = 4u, Allocator* allocator = 0);
    Mat(int w, int h, int d, int c, size_t elemsize = 4u, Allocator* allocator = 0);
    Mat(const Mat& m);
    // external data, not owned
    Mat(int w, void* data, size_t elemsize = 4u, Allocator* allocator = 0);
    Mat(int w, int h, void* data, size_t elemsize = 4u, Allocator* allocator = 0);
    Mat(int w, int h, int c, void* data, size_t elemsize = 4u, Allocator* allocator = 0);
    Mat(int w, int h, int d, int c, void* data, size_t elemsize = 4u, Allocator* allocator = 0);
    ~Mat();

    Mat& operator=(const Mat& m);

    void fill(float v);
    void fill(int v);
    Mat clone(Allocator* allocator = 0) const;
    Mat reshape(int w, Allocator* allocator = 0) const;
    Mat reshape(int w, int h, Allocator* allocator = 0) const;
    Mat reshape(int w, int h, int c, Allocator* allocator = 0) const;

    void create(int w, size_t elemsize = 4u, Allocator* allocator = 0);
    void create(int w, int h, size_t elemsize = 4u, Allocator* allocator = 0);
    void create(int w, int h, int c, size_t elemsize = 4u, Allocator* allocator = 0);
    void create(int w, int h, int d, int c, size_t elemsize = 4u, Allocator* allocator = 0);
    void create_like(const Mat& m, Allocator* allocator = 0);

    void addref();
    void release();

    bool empty() const { return data == 0 || total() == 0; }
    size_t total() const { return cstep * c; }
    int elembits() const { return elempack ? static_cast<int>(elemsize * 8) / elempack : 0; }

    Mat channel(int _c);
    const Mat channel(int _c) const;
    Mat row_range(int y, int rows);
    const Mat row_range(int y, int rows) const;

    float* row(int y) { return (float*)((unsigned char*)data + (size_t)w * y * elemsize); }
    const float* row(int y) const {
        return (const float*)((unsigned char*)data + (size_t)w * y * elemsize);
    }
    template <typename T>
    T* row(int y) {
        return (T*)((unsigned char*)data + (size_t)w * y * elemsize);
    }
    template <typename T>
    const T* row(int y) const {
        return (const T*)((unsigned char*)data + (size_t)w * y * elemsize);
    }

    template <typename T>
    operator T*() { return (T*)data; }
    template <typename T>
    operator const T*() const { return (const T*)data; }

    float& operator[](size_t i) { return ((float*)data)[i]; }
    const float& operator[](size_t i) const { return ((const float*)data)[i]; }

    void* data;
    int* refcount;
    size_t elemsize;
    int elempack;
    Allocator* allocator;
    int dims;
    int w;
    int h;
    int d;
    int c;
    size_t cstep;
};

}  // namespace ncnn

#endif  // NCNN_MAT_H
