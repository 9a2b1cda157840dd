// ncnn-compatible subset: Mat, Option, ParamDict and ModelBin implementations.
#include "mat.h"

#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

#include "modelbin.h"
#include "option.h"
#include "paramdict.h"

namespace ncnn {

Allocator::~Allocator() {}

// ---- Mat -------------------------------------------------------------------

Mat::Mat()
    : data(0), refcount(0), elemsize(0), elempack(0), allocator(0), dims(0), w(0), h(0), d(0),
      c(0), cstep(0) {}

Mat::Mat(int _w, size_t _elemsize, Allocator* _allocator) : Mat() {
    create(_w, _elemsize, _allocator);
}

Mat::Mat(int _w, int _h, size_t _elemsize, Allocator* _allocator) : Mat() {
    create(_w, _h, _elemsize, _allocator);
}

Mat::Mat(int _w, int _h, int _c, size_t _elemsize, Allocator* _allocator) : Mat() {
    create(_w, _h, _c, _elemsize, _allocator);
}

Mat::Mat(int _w, int _h, int _d, int _c, size_t _elemsize, Allocator* _allocator) : Mat() {
    create(_w, _h, _d, _c, _elemsize, _allocator);
}

Mat::Mat(const Mat& m)
    : data(m.data), refcount(m.refcount), elemsize(m.elemsize), elempack(m.elempack),
      allocator(m.allocator), dims(m.dims), w(m.w), h(m.h), d(m.d), c(m.c), cstep(m.cstep) {
    addref();
}

Mat::Mat(int _w, void* _data, size_t _elemsize, Allocator* _allocator)
    : data(_data), refcount(0), elemsize(_elemsize), elempack(1), allocator(_allocator), dims(1),
      w(_w), h(1), d(1), c(1), cstep(_w) {}

Mat::Mat(int _w, int _h, void* _data, size_t _elemsize, Allocator* _allocator)
    : data(_data), refcount(0), elemsize(_elemsize), elempack(1), allocator(_allocator), dims(2),
      w(_w), h(_h), d(1), c(1), cstep((size_t)_w * _h) {}

Mat::Mat(int _w, int _h, int _c, void* _data, size_t _elemsize, Allocator* _allocator)
    : data(_data), refcount(0), elemsize(_elemsize), elempack(1), allocator(_allocator), dims(3),
      w(_w), h(_h), d(1), c(_c) {
    cstep = alignSize((size_t)w * h * elemsize, 16) / elemsize;
}

Mat::Mat(int _w, int _h, int _d, int _c, void* _data, size_t _elemsize, Allocator* _allocator)
    : data(_data), refcount(0), elemsize(_elemsize), elempack(1), allocator(_allocator), dims(4),
      w(_w), h(_h), d(_d), c(_c) {
    cstep = alignSize((size_t)w * h * d * elemsize, 16) / elemsize;
}

Mat::~Mat() { release(); }

Mat& Mat::operator=(const Mat& m) {
    if (this == &m) return *this;
    if (m.refcount) NCNN_XADD(m.refcount, 1);
    release();
    data = m.data;
    refcount = m.refcount;
    elemsize = m.elemsize;
    elempack = m.elempack;
    allocator = m.allocator;
    dims = m.dims;
    w = m.w;
    h = m.h;
    d = m.d;
    c = m.c;
    cstep = m.cstep;
    return *this;
}

void Mat::addref() {
    if (refcount) NCNN_XADD(refcount, 1);
}

// The reference count lives in its own small host allocation, so a Mat whose
// allocator hands out device memory never has the host write into it.
void Mat::release() {
    if (refcount && NCNN_XADD(refcount, -1) == 1) {
        if (allocator)
            allocator->fastFree(data);
        else
            ncnn::fastFree(data);
        delete refcount;
    }
    data = 0;
    refcount = 0;
    elemsize = 0;
    elempack = 0;
    dims = 0;
    w = h = d = c = 0;
    cstep = 0;
}

static void mat_allocate(Mat& m, size_t bytes) {
    if (bytes == 0) return;
    void* p = m.allocator ? m.allocator->fastMalloc(bytes) : ncnn::fastMalloc(bytes);
    if (!p) {
        m.data = 0;
        return;
    }
    m.data = p;
    m.refcount = new int(1);
}

void Mat::create(int _w, size_t _elemsize, Allocator* _allocator) {
    if (dims == 1 && w == _w && elemsize == _elemsize && elempack == 1 && allocator == _allocator)
        return;
    release();
    elemsize = _elemsize;
    elempack = 1;
    allocator = _allocator;
    dims = 1;
    w = _w;
    h = d = c = 1;
    cstep = w;
    mat_allocate(*this, alignSize(total() * elemsize, 4));
}

void Mat::create(int _w, int _h, size_t _elemsize, Allocator* _allocator) {
    if (dims == 2 && w == _w && h == _h && elemsize == _elemsize && elempack == 1 &&
        allocator == _allocator)
        return;
    release();
    elemsize = _elemsize;
    elempack = 1;
    allocator = _allocator;
    dims = 2;
    w = _w;
    h = _h;
    d = c = 1;
    cstep = (size_t)w * h;
    mat_allocate(*this, alignSize(total() * elemsize, 4));
}

void Mat::create(int _w, int _h, int _c, size_t _elemsize, Allocator* _allocator) {
    if (dims == 3 && w == _w && h == _h && c == _c && elemsize == _elemsize && elempack == 1 &&
        allocator == _allocator)
        return;
    release();
    elemsize = _elemsize;
    elempack = 1;
    allocator = _allocator;
    dims = 3;
    w = _w;
    h = _h;
    d = 1;
    c = _c;
    cstep = alignSize((size_t)w * h * elemsize, 16) / elemsize;
    mat_allocate(*this, alignSize(total() * elemsize, 4));
}

void Mat::create(int _w, int _h, int _d, int _c, size_t _elemsize, Allocator* _allocator) {
    release();
    elemsize = _elemsize;
    elempack = 1;
    allocator = _allocator;
    dims = 4;
    w = _w;
    h = _h;
    d = _d;
    c = _c;
    cstep = alignSize((size_t)w * h * d * elemsize, 16) / elemsize;
    mat_allocate(*this, alignSize(total() * elemsize, 4));
}

void Mat::create_like(const Mat& m, Allocator* _allocator) {
    if (m.dims == 1) create(m.w, m.elemsize, _allocator);
    else if (m.dims == 2) create(m.w, m.h, m.elemsize, _allocator);
    else if (m.dims == 3) create(m.w, m.h, m.c, m.elemsize, _allocator);
    else if (m.dims == 4) create(m.w, m.h, m.d, m.c, m.elemsize, _allocator);
}

void Mat::fill(float v) {
    float* p = (float*)data;
    const size_t n = total();
    for (size_t i = 0; i < n; i++) p[i] = v;
}

void Mat::fill(int v) {
    int* p = (int*)data;
    const size_t n = total();
    for (size_t i = 0; i < n; i++) p[i] = v;
}

Mat Mat::clone(Allocator* _allocator) const {
    if (empty()) return Mat();
    Mat m;
    if (dims == 1) m.create(w, elemsize, _allocator);
    else if (dims == 2) m.create(w, h, elemsize, _allocator);
    else if (dims == 3) m.create(w, h, c, elemsize, _allocator);
    else m.create(w, h, d, c, elemsize, _allocator);
    if (!m.empty()) memcpy(m.data, data, total() * elemsize);
    return m;
}

Mat Mat::reshape(int _w, Allocator*) const {
    if ((size_t)w * h * d * c != (size_t)_w) return Mat();
    if (dims >= 3 && cstep != (size_t)w * h * d) return Mat();   // padded channels
    Mat m = *this;
    m.dims = 1;
    m.w = _w;
    m.h = m.d = m.c = 1;
    m.cstep = _w;
    return m;
}

Mat Mat::reshape(int _w, int _h, Allocator*) const {
    if ((size_t)w * h * d * c != (size_t)_w * _h) return Mat();
    if (dims >= 3 && cstep != (size_t)w * h * d) return Mat();
    Mat m = *this;
    m.dims = 2;
    m.w = _w;
    m.h = _h;
    m.d = m.c = 1;
    m.cstep = (size_t)_w * _h;
    return m;
}

Mat Mat::reshape(int _w, int _h, int _c, Allocator* _allocator) const {
    if ((size_t)w * h * d * c != (size_t)_w * _h * _c) return Mat();
    const size_t new_cstep = alignSize((size_t)_w * _h * elemsize, 16) / elemsize;
    if (new_cstep == (size_t)_w * _h && (dims < 3 || cstep == (size_t)w * h * d)) {
        Mat m = *this;
        m.dims = 3;
        m.w = _w;
        m.h = _h;
        m.d = 1;
        m.c = _c;
        m.cstep = new_cstep;
        return m;
    }
    Mat m(_w, _h, _c, elemsize, _allocator);
    if (m.empty()) return m;
    for (int i = 0; i < _c; i++)
        memcpy((unsigned char*)m.data + m.cstep * i * elemsize,
               (const unsigned char*)data + (size_t)_w * _h * i * elemsize,
               (size_t)_w * _h * elemsize);
    return m;
}

Mat Mat::channel(int _c) {
    Mat m(w, h, (unsigned char*)data + cstep * _c * elemsize, elemsize, allocator);
    m.dims = dims - 1;
    if (dims == 4) {
        m.dims = 3;
        m.c = d;
        m.cstep = (size_t)w * h;
    }
    return m;
}

const Mat Mat::channel(int _c) const {
    return const_cast<Mat*>(this)->channel(_c);
}

Mat Mat::row_range(int y, int rows) {
    Mat m(w, rows, (unsigned char*)data + (size_t)w * y * elemsize, elemsize, allocator);
    m.elempack = elempack;
    return m;
}

const Mat Mat::row_range(int y, int rows) const {
    return const_cast<Mat*>(this)->row_range(y, rows);
}

// ---- Option -----------------------------------------------------------------

Option::Option()
    : lightmode(true), num_threads(1), blob_allocator(0), workspace_allocator(0),
      use_vulkan_compute(false), use_fp16_packed(false), use_fp16_storage(false),
      use_fp16_arithmetic(false), use_bf16_packed(false), use_bf16_storage(false),
      use_packing_layout(false), use_cooperative_matrix(false), use_shader_local_memory(false),
      use_subgroup_ops(false) {}

// ---- ParamDict ----------------------------------------------------------------

ParamDict::ParamDict() { clear(); }

void ParamDict::clear() {
    for (int i = 0; i < NCNN_MAX_PARAM_COUNT; i++) {
        params[i].type = 0;
        params[i].i = 0;
        params[i].f = 0.f;
        params[i].v = Mat();
    }
}

int ParamDict::type(int id) const {
    return id >= 0 && id < NCNN_MAX_PARAM_COUNT ? params[id].type : 0;
}

int ParamDict::get(int id, int def) const {
    return type(id) ? params[id].i : def;
}

float ParamDict::get(int id, float def) const {
    return type(id) ? params[id].f : def;
}

Mat ParamDict::get(int id, const Mat& def) const {
    return type(id) == 4 ? params[id].v : def;
}

// As in ncnn, an int value also answers get(id, float) and vice versa.
void ParamDict::set(int id, int i) {
    if (id < 0 || id >= NCNN_MAX_PARAM_COUNT) return;
    params[id].type = 2;
    params[id].i = i;
    params[id].f = (float)i;
}

void ParamDict::set(int id, float f) {
    if (id < 0 || id >= NCNN_MAX_PARAM_COUNT) return;
    params[id].type = 3;
    params[id].f = f;
    params[id].i = (int)f;
}

void ParamDict::set(int id, const Mat& v) {
    if (id < 0 || id >= NCNN_MAX_PARAM_COUNT) return;
    params[id].type = 4;
    params[id].v = v;
}

static bool is_float_token(const char* s) {
    for (; *s && *s != ' ' && *s != ','; ++s)
        if (*s == '.' || *s == 'e' || *s == 'E') return true;
    return false;
}

int ParamDict::load_param_text(const char* p) {
    clear();
    while (*p) {
        while (*p == ' ' || *p == '\t' || *p == '\n' || *p == '\r') ++p;
        if (!*p) break;
        char* end = 0;
        long id = strtol(p, &end, 10);
        if (end == p || *end != '=') return -1;
        p = end + 1;
        const bool is_array = id <= -23300;
        if (is_array) id = -id - 23300;
        if (id < 0 || id >= NCNN_MAX_PARAM_COUNT) return -1;
        if (is_array) {
            long n = strtol(p, &end, 10);
            if (end == p || n < 0) return -1;
            p = end;
            const bool fl = is_float_token(p + (*p == ',' ? 1 : 0));
            Mat v((int)n);
            if (n && v.empty()) return -1;
            for (long i = 0; i < n; i++) {
                if (*p != ',') return -1;
                ++p;
                if (fl) ((float*)v.data)[i] = strtof(p, &end);
                else ((int*)v.data)[i] = (int)strtol(p, &end, 10);
                if (end == p) return -1;
                p = end;
            }
            set((int)id, v);
        } else if (is_float_token(p)) {
            float f = strtof(p, &end);
            if (end == p) return -1;
            set((int)id, f);
            p = end;
        } else {
            long i = strtol(p, &end, 10);
            if (end == p) return -1;
            set((int)id, (int)i);
            p = end;
        }
    }
    return 0;
}

// ---- ModelBin -----------------------------------------------------------------

ModelBin::ModelBin() {}
ModelBin::~ModelBin() {}

Mat ModelBin::load(int w, int h, int type) const {
    Mat m = load(w * h, type);
    return m.empty() ? m : m.reshape(w, h);
}

Mat ModelBin::load(int w, int h, int c, int type) const {
    Mat m = load(w * h * c, type);
    return m.empty() ? m : m.reshape(w, h, c);
}

ModelBinFromMatArray::ModelBinFromMatArray(const Mat* _weights) : weights(_weights) {}
ModelBinFromMatArray::~ModelBinFromMatArray() {}

Mat ModelBinFromMatArray::load(int, int) const {
    if (!weights) return Mat();
    Mat m = weights[0];
    weights++;
    return m;
}

ModelBinFromMemory::ModelBinFromMemory(const unsigned char* _data, size_t _size)
    : data(_data), size(_size), offset(0) {}
ModelBinFromMemory::~ModelBinFromMemory() {}

static float half_to_float(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    const uint32_t exp = (h >> 10) & 0x1f;
    const uint32_t mant = h & 0x3ff;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else {   // subnormal
            uint32_t m = mant;
            int e = -1;
            do {
                ++e;
                m <<= 1;
            } while (!(m & 0x400));
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | ((m & 0x3ff) << 13);
        }
    } else if (exp == 0x1f) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

Mat ModelBinFromMemory::load(int w, int type) const {
    if (w <= 0) return Mat();
    bool fp16 = false;
    if (type == 0) {
        if (offset + 4 > size) return Mat();
        uint32_t tag;
        memcpy(&tag, data + offset, 4);
        offset += 4;
        if (tag == 0x01306B47) fp16 = true;
        else if (tag != 0) return Mat();
    } else if (type != 1) {
        return Mat();
    }
    const size_t bytes = (size_t)w * (fp16 ? 2 : 4);
    if (offset + bytes > size) return Mat();
    Mat m(w);
    if (m.empty()) return m;
    if (fp16) {
        for (int i = 0; i < w; i++) {
            uint16_t h;
            memcpy(&h, data + offset + 2 * (size_t)i, 2);
            ((float*)m.data)[i] = half_to_float(h);
        }
    } else {
        memcpy(m.data, data + offset, bytes);
    }
    // ncnn aligns tagged fp16 payloads to 4 bytes
    offset += fp16 ? alignSize(bytes, 4) : bytes;
    return m;
}

}  // namespace ncnn
