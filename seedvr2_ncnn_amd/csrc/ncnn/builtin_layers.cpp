// ncnn-compatible subset: built-in layers of exported graphs (builtin_layers.h).
#include "builtin_layers.h"

#include <math.h>
#include <string.h>

#include <algorithm>
#include <mutex>
#include <vector>

#include "hip_allocator.h"
#include "seedvr2_hip.h"

namespace ncnn {

namespace {

using seedvr2::HipDeviceAllocator;
using seedvr2::device_allocator_of;
using seedvr2::device_blob_dtype;
using seedvr2::layer_status;

// A blob of dims 1 or 2 as rows x cols (dims 1: one row).
struct Shape {
    int dims, rows, cols;
};

bool shape_of(const Mat& m, Shape* s) {
    if (m.empty() || m.elempack != 1) return false;
    if (m.dims == 1) {
        s->dims = 1;
        s->rows = 1;
        s->cols = m.w;
        return true;
    }
    if (m.dims == 2) {
        s->dims = 2;
        s->rows = m.h;
        s->cols = m.w;
        return true;
    }
    return false;
}

HipDeviceAllocator* out_allocator(HipDeviceAllocator* dev, const Option& opt) {
    HipDeviceAllocator* out = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
    return out ? out : dev;
}

Allocator* host_allocator(const Option& opt) {
    return dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator) ? 0 : opt.blob_allocator;
}

// A new blob: on the device of `dev` in elemsize, or a host fp32 one.
Mat new_blob(HipDeviceAllocator* dev, int dims, int rows, int cols, size_t elemsize,
             const Option& opt) {
    if (dev) {
        Mat m = out_allocator(dev, opt)->create_blob(cols, rows, elemsize);
        if (!m.empty() && dims == 1) m.dims = 1;
        return m;
    }
    Mat m;
    if (dims == 1)
        m.create(cols, (size_t)4u, host_allocator(opt));
    else
        m.create(cols, rows, (size_t)4u, host_allocator(opt));
    return m;
}

s2_dtype dtype_of(const Mat& m, const Option& opt) { return device_blob_dtype(m.elemsize, opt); }

// Host blobs: fp32 only.
bool host_ok(const Mat& m) { return m.elemsize == 4; }

const float* fdata(const Mat& m) { return static_cast<const float*>(m.data); }
float* fdata(Mat& m) { return static_cast<float*>(m.data); }

// ---- host arithmetic (the same definitions as the device kernels) -------------

float binary_host(int op, float a, float b) {
    switch (op) {
        case 0: return a + b;
        case 1: return a - b;
        case 2: return a * b;
        case 3: return a / b;
        case 4: return std::max(a, b);
        case 5: return std::min(a, b);
        case 6: return powf(a, b);
        case 7: return b - a;
        case 8: return b / a;
        case 9: return powf(b, a);
        case 10: return atan2f(a, b);
        default: return atan2f(b, a);
    }
}

float unary_host(int op, float x) {
    switch (op) {
        case 0: return fabsf(x);
        case 1: return -x;
        case 2: return floorf(x);
        case 3: return ceilf(x);
        case 4: return x * x;
        case 5: return sqrtf(x);
        case 6: return 1.f / sqrtf(x);
        case 7: return expf(x);
        case 8: return logf(x);
        case 9: return sinf(x);
        case 10: return cosf(x);
        case 11: return tanf(x);
        case 12: return asinf(x);
        case 13: return acosf(x);
        case 14: return atanf(x);
        case 15: return 1.f / x;
        case 16: return tanhf(x);
        case 17: return log10f(x);
        case 18: return nearbyintf(x);
        case 19: return truncf(x);
        case 100: return 1.f / (1.f + expf(-x));
        default: return x / (1.f + expf(-x));
    }
}

// A device copy of host fp32 data, made once (create_pipeline, or the first
// forward on a device) and kept until destroy_pipeline.
class DeviceCopy {
public:
    DeviceCopy() : ptr_(0) {}
    ~DeviceCopy() { release(); }
    int ensure(const Mat& host) {
        if (ptr_ || host.empty()) return S2_OK;
        const size_t bytes = host.total() * host.elemsize;
        int ret = s2_malloc(&ptr_, bytes);
        if (ret == S2_OK) ret = s2_memcpy_h2d(ptr_, host.data, bytes, 0);
        if (ret == S2_OK) ret = s2_stream_synchronize(0);
        if (ret != S2_OK) release();
        return ret;
    }
    void release() {
        if (ptr_) s2_free(ptr_);
        ptr_ = 0;
    }
    void* get() const { return ptr_; }

private:
    DeviceCopy(const DeviceCopy&);
    DeviceCopy& operator=(const DeviceCopy&);
    void* ptr_;
};

bool have_device() {
    int n = 0;
    return s2_device_count(&n) == S2_OK && n > 0;
}

// ---- MemoryData ---------------------------------------------------------------

// Params 0 w, 1 h, 11 d, 2 c, 21 load_type (1: raw fp32); the data follows in
// the .bin as raw fp32.  Forward has no bottom: the data as a blob (device
// blobs alias the layer's device copy, which no consumer writes).
class MemoryDataLayer : public Layer {
public:
    MemoryDataLayer() : w(0), h(0) {
        one_blob_only = false;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        w = pd.get(0, 0);
        h = pd.get(1, 0);
        const int d = pd.get(11, 0), c = pd.get(2, 0), load_type = pd.get(21, 1);
        if (w < 0 || h < 0 || d != 0 || c != 0 || load_type != 1 || (h > 0 && w == 0)) return -1;
        return 0;
    }
    virtual int load_model(const ModelBin& mb) {
        std::lock_guard<std::mutex> lock(mutex);
        copy.release();
        if (h > 0)
            data = mb.load(w, h, 1);
        else if (w > 0)
            data = mb.load(w, 1);
        else {
            data.create(1);
            if (!data.empty()) data.fill(0.f);
        }
        return data.empty() ? -100 : 0;
    }
    virtual int create_pipeline(const Option&) {
        std::lock_guard<std::mutex> lock(mutex);
        return have_device() ? layer_status(copy.ensure(data)) : 0;
    }
    virtual int destroy_pipeline(const Option&) {
        std::lock_guard<std::mutex> lock(mutex);
        copy.release();
        return 0;
    }
    virtual int forward(const std::vector<Mat>&, std::vector<Mat>& tops, const Option& opt) const {
        if (tops.size() != 1) return -1;
        HipDeviceAllocator* out = dynamic_cast<HipDeviceAllocator*>(opt.blob_allocator);
        if (out) {
            std::lock_guard<std::mutex> lock(mutex);
            const int ret = copy.ensure(data);
            if (ret != S2_OK) return layer_status(ret);
            tops[0] = out->wrap_blob(data.w, data.dims == 2 ? data.h : 1, copy.get(), 4);
            if (data.dims == 1) tops[0].dims = 1;
            return 0;
        }
        tops[0] = data.clone(host_allocator(opt));
        return tops[0].empty() ? -100 : 0;
    }
    int w, h;
    Mat data;
    mutable std::mutex mutex;
    mutable DeviceCopy copy;
};

// ---- BinaryOp ---------------------------------------------------------------

// Params 0 op_type, 1 with_scalar, 2 b.  Two bottoms broadcast numpy-style
// (a 1-D blob is one row; an axis of size 1 spreads), or one bottom and the
// scalar b.
class BinaryOpLayer : public Layer {
public:
    BinaryOpLayer() : op_type(0), with_scalar(0), b(0.f) { support_inplace = false; }
    virtual int load_param(const ParamDict& pd) {
        op_type = pd.get(0, 0);
        with_scalar = pd.get(1, 0);
        b = pd.get(2, 0.f);
        one_blob_only = with_scalar != 0;
        return (op_type < 0 || op_type > 11) ? -1 : 0;
    }
    virtual int forward(const Mat& a, Mat& top, const Option& opt) const {
        Shape s;
        if (!shape_of(a, &s)) return -1;
        HipDeviceAllocator* dev = device_allocator_of(a);
        if (!dev && !host_ok(a)) return -1;
        top = new_blob(dev, s.dims, s.rows, s.cols, dev ? a.elemsize : 4, opt);
        if (top.empty()) return -100;
        if (dev) {
            const int ret = s2_binary_op(op_type, a.data, dtype_of(a, opt), s.rows, s.cols, s.cols, 0,
                                         S2_DTYPE_F32, 1, 1, 1, b, top.data, dtype_of(top, opt), s.rows,
                                         s.cols, s.cols, dev->stream());
            return layer_status(ret);
        }
        const size_t n = (size_t)s.rows * s.cols;
        for (size_t i = 0; i < n; i++) fdata(top)[i] = binary_host(op_type, fdata(a)[i], b);
        return 0;
    }
    virtual int forward(const std::vector<Mat>& bottoms, std::vector<Mat>& tops,
                        const Option& opt) const {
        if (bottoms.size() != 2 || tops.size() != 1) return -1;
        const Mat& a = bottoms[0];
        const Mat& bb = bottoms[1];
        Shape sa, sb;
        if (!shape_of(a, &sa) || !shape_of(bb, &sb)) return -1;
        const int rows = std::max(sa.rows, sb.rows), cols = std::max(sa.cols, sb.cols);
        if ((sa.rows != rows && sa.rows != 1) || (sb.rows != rows && sb.rows != 1) ||
            (sa.cols != cols && sa.cols != 1) || (sb.cols != cols && sb.cols != 1))
            return -1;
        const int dims = std::max(sa.dims, sb.dims);
        HipDeviceAllocator* da = device_allocator_of(a);
        HipDeviceAllocator* db = device_allocator_of(bb);
        if ((da != 0) != (db != 0)) return -1;
        if (da) {
            // the output takes the element type of an operand of its shape
            const bool a_full = sa.rows == rows && sa.cols == cols;
            const size_t es = a_full ? a.elemsize : (sb.rows == rows && sb.cols == cols ? bb.elemsize : a.elemsize);
            tops[0] = new_blob(da, dims, rows, cols, es, opt);
            if (tops[0].empty()) return -100;
            const int ret = s2_binary_op(op_type, a.data, dtype_of(a, opt), sa.rows, sa.cols, sa.cols,
                                         bb.data, dtype_of(bb, opt), sb.rows, sb.cols, sb.cols, 0.f,
                                         tops[0].data, dtype_of(tops[0], opt), rows, cols, cols,
                                         da->stream());
            return layer_status(ret);
        }
        if (!host_ok(a) || !host_ok(bb)) return -1;
        tops[0] = new_blob(0, dims, rows, cols, 4, opt);
        if (tops[0].empty()) return -100;
        float* y = fdata(tops[0]);
        for (int r = 0; r < rows; r++)
            for (int c = 0; c < cols; c++) {
                const float x0 = fdata(a)[(size_t)(sa.rows == 1 ? 0 : r) * sa.cols + (sa.cols == 1 ? 0 : c)];
                const float x1 = fdata(bb)[(size_t)(sb.rows == 1 ? 0 : r) * sb.cols + (sb.cols == 1 ? 0 : c)];
                y[(size_t)r * cols + c] = binary_host(op_type, x0, x1);
            }
        return 0;
    }
    int op_type, with_scalar;
    float b;
};

// ---- UnaryOp, Sigmoid, Swish -----------------------------------------------

class UnaryLayer : public Layer {
public:
    explicit UnaryLayer(int fixed_op) : op_type(fixed_op), fixed(fixed_op >= 0) {
        one_blob_only = true;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        if (fixed) return 0;
        op_type = pd.get(0, 0);
        return (op_type < 0 || op_type > 19) ? -1 : 0;
    }
    virtual int forward(const Mat& x, Mat& top, const Option& opt) const {
        Shape s;
        if (!shape_of(x, &s)) return -1;
        HipDeviceAllocator* dev = device_allocator_of(x);
        if (!dev && !host_ok(x)) return -1;
        top = new_blob(dev, s.dims, s.rows, s.cols, dev ? x.elemsize : 4, opt);
        if (top.empty()) return -100;
        const size_t n = (size_t)s.rows * s.cols;
        if (dev)
            return layer_status(s2_unary_op(op_type, x.data, dtype_of(x, opt), top.data,
                                            dtype_of(top, opt), n, dev->stream()));
        for (size_t i = 0; i < n; i++) fdata(top)[i] = unary_host(op_type, fdata(x)[i]);
        return 0;
    }
    int op_type;
    bool fixed;
};

// ---- Reduction ----------------------------------------------------------------

// Params 0 operation, 1 reduce_all (default 1), 2 coeff, 3 axes (array),
// 4 keepdims, 5 fixbug0 (1: numpy axis numbering, as pnnx writes).
class ReductionLayer : public Layer {
public:
    ReductionLayer() : operation(0), reduce_all(1), coeff(1.f), keepdims(0) {
        one_blob_only = true;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        operation = pd.get(0, 0);
        reduce_all = pd.get(1, 1);
        coeff = pd.get(2, 1.f);
        const Mat ax = pd.get(3, Mat());
        keepdims = pd.get(4, 0);
        const int fixbug0 = pd.get(5, 0);
        axes.clear();
        for (int i = 0; i < ax.w; i++) axes.push_back(static_cast<const int*>(ax.data)[i]);
        if (operation < 0 || operation > 10) return -1;
        if (!reduce_all && (axes.empty() || !fixbug0)) return -1;
        return 0;
    }
    // which axes of a blob of `dims` are reduced: rows and/or cols
    bool resolve(int dims, bool* rows, bool* cols) const {
        *rows = *cols = false;
        if (reduce_all) {
            *rows = *cols = true;
            return true;
        }
        for (size_t i = 0; i < axes.size(); i++) {
            int a = axes[i] < 0 ? axes[i] + dims : axes[i];
            if (a < 0 || a >= dims) return false;
            if (dims == 1 || a == 1)
                *cols = true;
            else
                *rows = true;
        }
        if (dims == 1) *rows = true;
        return true;
    }
    virtual int forward(const Mat& x, Mat& top, const Option& opt) const {
        Shape s;
        bool rr, rc;
        if (!shape_of(x, &s) || !resolve(s.dims, &rr, &rc)) return -1;
        HipDeviceAllocator* dev = device_allocator_of(x);
        if (!dev && !host_ok(x)) return -1;
        // output shape
        int dims, orow, ocol;
        if (rr && rc) {
            dims = keepdims ? s.dims : 1;
            orow = 1;
            ocol = 1;
        } else if (rc) {   // each row to a value
            dims = keepdims ? 2 : 1;
            orow = keepdims ? s.rows : 1;
            ocol = keepdims ? 1 : s.rows;
        } else {   // each column
            dims = keepdims ? 2 : 1;
            orow = 1;
            ocol = s.cols;
        }
        top = new_blob(dev, dims, orow, ocol, dev ? x.elemsize : 4, opt);
        if (top.empty()) return -100;
        if (dev) {
            int ret;
            if (rr && rc)   // the whole blob as one row
                ret = s2_reduce(operation, coeff, 1, x.data, dtype_of(x, opt), 1, s.rows * s.cols,
                                s.rows * s.cols, top.data, dtype_of(top, opt), dev->stream());
            else
                ret = s2_reduce(operation, coeff, rc ? 1 : 0, x.data, dtype_of(x, opt), s.rows, s.cols,
                                s.cols, top.data, dtype_of(top, opt), dev->stream());
            return layer_status(ret);
        }
        const int groups = (rr && rc) ? 1 : rc ? s.rows : s.cols;
        const int n = (rr && rc) ? s.rows * s.cols : rc ? s.cols : s.rows;
        for (int g = 0; g < groups; g++) {
            double acc = operation == 4 ? -INFINITY : operation == 5 ? INFINITY : operation == 6 ? 1.0 : 0.0;
            for (int i = 0; i < n; i++) {
                size_t idx;
                if (rr && rc)
                    idx = i;
                else if (rc)
                    idx = (size_t)g * s.cols + i;
                else
                    idx = (size_t)i * s.cols + g;
                float v = fdata(x)[idx];
                if (operation == 1 || operation == 7) v = fabsf(v);
                if (operation == 2 || operation == 8) v = v * v;
                if (operation == 10) v = expf(v);
                if (operation == 4)
                    acc = std::max(acc, (double)v);
                else if (operation == 5)
                    acc = std::min(acc, (double)v);
                else if (operation == 6)
                    acc *= v;
                else
                    acc += v;
            }
            if (operation == 3) acc /= n;
            if (operation == 8) acc = sqrt(acc);
            if (operation == 9 || operation == 10) acc = log(acc);
            fdata(top)[g] = (float)(acc * coeff);
        }
        return 0;
    }
    int operation, reduce_all;
    float coeff;
    int keepdims;
    std::vector<int> axes;
};

// ---- RMSNorm --------------------------------------------------------------------

// Params 0 affine_size, 1 eps (default 0.001), 2 affine (default 1); with
// affine, gamma[affine_size] follows as raw fp32.  Each row (the last axis)
// is normalised: y = x / sqrt(mean(x^2) + eps) * gamma.
class RMSNormLayer : public Layer {
public:
    RMSNormLayer() : affine_size(0), eps(0.001f), affine(1) {
        one_blob_only = true;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        affine_size = pd.get(0, 0);
        eps = pd.get(1, 0.001f);
        affine = pd.get(2, 1);
        return (affine && affine_size <= 0) || !(eps >= 0.f) ? -1 : 0;
    }
    virtual int load_model(const ModelBin& mb) {
        std::lock_guard<std::mutex> lock(mutex);
        gamma_copy.release();
        if (!affine) return 0;
        gamma = mb.load(affine_size, 1);
        return gamma.empty() ? -100 : 0;
    }
    virtual int create_pipeline(const Option&) {
        std::lock_guard<std::mutex> lock(mutex);
        return (affine && have_device()) ? layer_status(gamma_copy.ensure(gamma)) : 0;
    }
    virtual int destroy_pipeline(const Option&) {
        std::lock_guard<std::mutex> lock(mutex);
        gamma_copy.release();
        return 0;
    }
    virtual int forward(const Mat& x, Mat& top, const Option& opt) const {
        Shape s;
        if (!shape_of(x, &s) || (affine && s.cols != affine_size)) return -1;
        HipDeviceAllocator* dev = device_allocator_of(x);
        if (!dev && !host_ok(x)) return -1;
        top = new_blob(dev, s.dims, s.rows, s.cols, dev ? x.elemsize : 4, opt);
        if (top.empty()) return -100;
        if (dev) {
            std::lock_guard<std::mutex> lock(mutex);
            if (affine) {
                const int ret = gamma_copy.ensure(gamma);
                if (ret != S2_OK) return layer_status(ret);
            }
            return layer_status(s2_rms_norm(x.data, dtype_of(x, opt), s.rows, s.cols, s.cols,
                                            affine ? (const float*)gamma_copy.get() : 0, eps, top.data,
                                            dtype_of(top, opt), s.cols, dev->stream()));
        }
        for (int r = 0; r < s.rows; r++) {
            const float* xr = fdata(x) + (size_t)r * s.cols;
            float ss = 0.f;
            for (int c = 0; c < s.cols; c++) ss = fmaf(xr[c], xr[c], ss);
            const float inv = 1.f / sqrtf(ss / (float)s.cols + eps);
            for (int c = 0; c < s.cols; c++)
                fdata(top)[(size_t)r * s.cols + c] = xr[c] * inv * (affine ? fdata(gamma)[c] : 1.f);
        }
        return 0;
    }
    int affine_size;
    float eps;
    int affine;
    Mat gamma;
    mutable std::mutex mutex;
    mutable DeviceCopy gamma_copy;
};

// ---- Reshape ----------------------------------------------------------------------

// Params 0 w, 1 h, 11 d, 2 c (-233: absent; 0: the input's; -1: inferred).
// Blobs of at most two dimensions: the output shares the input's data.
class ReshapeLayer : public Layer {
public:
    ReshapeLayer() : w(-233), h(-233) {
        one_blob_only = true;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        w = pd.get(0, -233);
        h = pd.get(1, -233);
        const int d = pd.get(11, -233), c = pd.get(2, -233), permute = pd.get(3, 0);
        return (d != -233 || c != -233 || permute != 0 || w == -233) ? -1 : 0;
    }
    virtual int forward(const Mat& x, Mat& top, const Option&) const {
        Shape s;
        if (!shape_of(x, &s)) return -1;
        const long total = (long)s.rows * s.cols;
        long ow = w == 0 ? x.w : w;
        long oh = h == -233 ? 1 : (h == 0 ? (x.dims == 2 ? x.h : 1) : h);
        if (ow == -1 && oh == -1) return -1;
        if (ow == -1) ow = oh > 0 ? total / oh : -1;
        if (oh == -1) oh = ow > 0 ? total / ow : -1;
        if (ow <= 0 || oh <= 0 || ow * oh != total) return -1;
        // a view that keeps the input's reference (host blobs) or names the
        // same device block (whose slots the extractor counts together)
        top = h == -233 ? x.reshape((int)ow) : x.reshape((int)ow, (int)oh);
        return top.empty() ? -1 : 0;
    }
    int w, h;
};

// ---- copies: Slice, Concat, Crop ---------------------------------------------------

// dst[dr0 + r][dc0 + c] = src[sr0 + r][sc0 + c] for r < rows, c < cols.
int copy_block(const Mat& src, int s_cols, int sr0, int sc0, Mat& dst, int d_cols, int dr0, int dc0,
               int rows, int cols, const Option& opt) {
    if (rows <= 0 || cols <= 0) return 0;
    HipDeviceAllocator* dev = device_allocator_of(src);
    if (dev) {
        const char* sp = static_cast<const char*>(src.data) + ((size_t)sr0 * s_cols + sc0) * src.elemsize;
        char* dp = static_cast<char*>(dst.data) + ((size_t)dr0 * d_cols + dc0) * dst.elemsize;
        return layer_status(s2_copy_2d(sp, dtype_of(src, opt), s_cols, dp, dtype_of(dst, opt), d_cols,
                                       rows, cols, dev->stream()));
    }
    for (int r = 0; r < rows; r++)
        memcpy(fdata(dst) + (size_t)(dr0 + r) * d_cols + dc0,
               fdata(src) + (size_t)(sr0 + r) * s_cols + sc0, (size_t)cols * sizeof(float));
    return 0;
}

// numpy axis of a blob of dims 1 or 2 -> 0 rows, 1 columns; -1 when out of range
int axis_of(int axis, int dims) {
    if (axis < 0) axis += dims;
    if (axis < 0 || axis >= dims) return -1;
    return dims == 1 ? 1 : axis;
}

// Params 0 slices (array; -233: an even share of what is left), 1 axis,
// 2 indices (array of split points).  Without either, an even split.
class SliceLayer : public Layer {
public:
    SliceLayer() : axis(0) {
        one_blob_only = false;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        const Mat sl = pd.get(0, Mat());
        const Mat ix = pd.get(2, Mat());
        axis = pd.get(1, 0);
        slices.assign(static_cast<const int*>(sl.data), static_cast<const int*>(sl.data) + sl.w);
        indices.assign(static_cast<const int*>(ix.data), static_cast<const int*>(ix.data) + ix.w);
        return 0;
    }
    virtual int forward(const std::vector<Mat>& bottoms, std::vector<Mat>& tops,
                        const Option& opt) const {
        if (bottoms.size() != 1 || tops.empty()) return -1;
        const Mat& x = bottoms[0];
        Shape s;
        if (!shape_of(x, &s)) return -1;
        const int ax = axis_of(axis, s.dims);
        if (ax < 0) return -1;
        HipDeviceAllocator* dev = device_allocator_of(x);
        if (!dev && !host_ok(x)) return -1;
        const int len = ax == 0 ? s.rows : s.cols;
        const int n = (int)tops.size();
        std::vector<int> size(n);
        int q = 0;
        for (int i = 0; i < n; i++) {
            int sz;
            if (!slices.empty()) {
                if ((int)slices.size() != n) return -1;
                sz = slices[i] == -233 ? (len - q) / (n - i) : slices[i];
            } else if (!indices.empty()) {
                if ((int)indices.size() != n - 1) return -1;
                int end = i + 1 < n ? indices[i] : len;
                if (end < 0) end += len;
                sz = std::min(end, len) - q;
            } else {
                sz = (len - q) / (n - i);
            }
            if (sz <= 0 || q + sz > len) return -1;
            size[i] = sz;
            q += sz;
        }
        q = 0;
        for (int i = 0; i < n; i++) {
            const int orow = ax == 0 ? size[i] : s.rows, ocol = ax == 0 ? s.cols : size[i];
            tops[i] = new_blob(dev, s.dims, orow, ocol, dev ? x.elemsize : 4, opt);
            if (tops[i].empty()) return -100;
            const int ret = copy_block(x, s.cols, ax == 0 ? q : 0, ax == 0 ? 0 : q, tops[i], ocol, 0, 0,
                                       orow, ocol, opt);
            if (ret != 0) return ret;
            q += size[i];
        }
        return 0;
    }
    int axis;
    std::vector<int> slices, indices;
};

// Param 0 axis.
class ConcatLayer : public Layer {
public:
    ConcatLayer() : axis(0) {
        one_blob_only = false;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        axis = pd.get(0, 0);
        return 0;
    }
    virtual int forward(const std::vector<Mat>& bottoms, std::vector<Mat>& tops,
                        const Option& opt) const {
        if (bottoms.empty() || tops.size() != 1) return -1;
        Shape s0;
        if (!shape_of(bottoms[0], &s0)) return -1;
        const int ax = axis_of(axis, s0.dims);
        if (ax < 0) return -1;
        HipDeviceAllocator* dev = device_allocator_of(bottoms[0]);
        int total = 0;
        for (size_t i = 0; i < bottoms.size(); i++) {
            Shape si;
            if (!shape_of(bottoms[i], &si) || si.dims != s0.dims ||
                (device_allocator_of(bottoms[i]) != 0) != (dev != 0) ||
                (!dev && !host_ok(bottoms[i])) || (ax == 0 ? si.cols != s0.cols : si.rows != s0.rows))
                return -1;
            total += ax == 0 ? si.rows : si.cols;
        }
        const int orow = ax == 0 ? total : s0.rows, ocol = ax == 0 ? s0.cols : total;
        tops[0] = new_blob(dev, s0.dims, orow, ocol, dev ? bottoms[0].elemsize : 4, opt);
        if (tops[0].empty()) return -100;
        int q = 0;
        for (size_t i = 0; i < bottoms.size(); i++) {
            Shape si = {0, 0, 0};
            shape_of(bottoms[i], &si);
            const int ret = copy_block(bottoms[i], si.cols, 0, 0, tops[0], ocol, ax == 0 ? q : 0,
                                       ax == 0 ? 0 : q, si.rows, si.cols, opt);
            if (ret != 0) return ret;
            q += ax == 0 ? si.rows : si.cols;
        }
        return 0;
    }
    int axis;
};

// Params 0 woffset, 1 hoffset, 3 outw, 4 outh, 6 woffset2, 7 hoffset2 (the
// legacy form: out* 0 keeps what the offsets leave), or 9 starts, 10 ends,
// 11 axes (arrays, Python slice bounds).
class CropLayer : public Layer {
public:
    CropLayer() : woffset(0), hoffset(0), outw(0), outh(0), woffset2(0), hoffset2(0) {
        one_blob_only = true;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        woffset = pd.get(0, 0);
        hoffset = pd.get(1, 0);
        outw = pd.get(3, 0);
        outh = pd.get(4, 0);
        woffset2 = pd.get(6, 0);
        hoffset2 = pd.get(7, 0);
        if (pd.get(13, 0) || pd.get(2, 0) || pd.get(14, 0) || pd.get(5, 0) || pd.get(15, 0) || pd.get(8, 0))
            return -1;
        const Mat st = pd.get(9, Mat()), en = pd.get(10, Mat()), ax = pd.get(11, Mat());
        starts.assign(static_cast<const int*>(st.data), static_cast<const int*>(st.data) + st.w);
        ends.assign(static_cast<const int*>(en.data), static_cast<const int*>(en.data) + en.w);
        axes.assign(static_cast<const int*>(ax.data), static_cast<const int*>(ax.data) + ax.w);
        if (starts.size() != ends.size() || (!axes.empty() && axes.size() != starts.size())) return -1;
        return 0;
    }
    virtual int forward(const Mat& x, Mat& top, const Option& opt) const {
        Shape s;
        if (!shape_of(x, &s)) return -1;
        HipDeviceAllocator* dev = device_allocator_of(x);
        if (!dev && !host_ok(x)) return -1;
        int r0 = 0, r1 = s.rows, c0 = 0, c1 = s.cols;
        if (!starts.empty()) {
            for (size_t i = 0; i < starts.size(); i++) {
                const int ax = axis_of(axes.empty() ? (int)i : axes[i], s.dims);
                if (ax < 0) return -1;
                const int len = ax == 0 ? s.rows : s.cols;
                long b = starts[i], e = ends[i];
                if (b < 0) b += len;
                if (e < 0) e += len;
                b = std::min<long>(std::max<long>(b, 0), len);
                e = std::min<long>(std::max<long>(e, 0), len);
                if (ax == 0) {
                    r0 = (int)b;
                    r1 = (int)e;
                } else {
                    c0 = (int)b;
                    c1 = (int)e;
                }
            }
        } else {
            c0 = woffset;
            c1 = outw > 0 ? woffset + outw : s.cols - woffset2;
            if (s.dims == 2) {
                r0 = hoffset;
                r1 = outh > 0 ? hoffset + outh : s.rows - hoffset2;
            }
        }
        if (r0 < 0 || c0 < 0 || r1 > s.rows || c1 > s.cols || r1 <= r0 || c1 <= c0) return -1;
        top = new_blob(dev, s.dims, r1 - r0, c1 - c0, dev ? x.elemsize : 4, opt);
        if (top.empty()) return -100;
        return copy_block(x, s.cols, r0, c0, top, c1 - c0, 0, 0, r1 - r0, c1 - c0, opt);
    }
    int woffset, hoffset, outw, outh, woffset2, hoffset2;
    std::vector<int> starts, ends, axes;
};

// ---- Gemm ------------------------------------------------------------------------

// y = alpha A B + beta C with A the bottom blob ([M][K], or [K] for M = 1),
// B constant (param 5 constantB = 1; [N][K] when transB = 1, else [K][N])
// and C constant or absent (param 6 constantC; broadcast type 10: -1 none,
// 0 a scalar, 4 one value per output column).  Params: 0 alpha, 1 beta,
// 2 transA, 3 transB, 4 constantA, 5 constantB, 6 constantC, 7 constantM,
// 8 constantN, 9 constantK, 10 constant_broadcast_type_C, 11 output_N1M,
// 14 output_transpose.  Weights are read with ModelBin type 0 (a 4-byte
// tag, then raw fp32 or fp16).  The device path is s2_shared_linear_forward
// with one token stream (bf16 B, fp32 beta C as the bias), as ncnn's Gemm
// stands behind the reference's SharedLinear (shared_linear.cpp:36-57).
class GemmLayer : public Layer {
public:
    GemmLayer()
        : alpha(1.f), beta(1.f), transB(0), constantC(0), N(0), K(0), broadcast_C(0),
          weight_gpu(0), bias_gpu(0) {
        one_blob_only = true;
        support_inplace = false;
    }
    ~GemmLayer() { release(); }
    virtual int load_param(const ParamDict& pd) {
        alpha = pd.get(0, 1.f);
        beta = pd.get(1, 1.f);
        const int transA = pd.get(2, 0);
        transB = pd.get(3, 0);
        const int constantA = pd.get(4, 0), constantB = pd.get(5, 0);
        constantC = pd.get(6, 0);
        N = pd.get(8, 0);
        K = pd.get(9, 0);
        broadcast_C = pd.get(10, 0);
        const int output_N1M = pd.get(11, 0), output_transpose = pd.get(14, 0);
        if (transA || constantA || !constantB || output_N1M || output_transpose || N <= 0 || K <= 0)
            return -1;
        if (constantC && broadcast_C != -1 && broadcast_C != 0 && broadcast_C != 4) return -1;
        return 0;
    }
    virtual int load_model(const ModelBin& mb) {
        std::lock_guard<std::mutex> lock(mutex);
        release();
        Mat b = transB ? mb.load(K, N, 0) : mb.load(N, K, 0);
        if (b.empty()) return -100;
        weight.create(K, N);   // [N][K]
        if (weight.empty()) return -100;
        for (int n = 0; n < N; n++)
            for (int k = 0; k < K; k++)
                fdata(weight)[(size_t)n * K + k] = transB ? fdata(b)[(size_t)n * K + k] : fdata(b)[(size_t)k * N + n];
        bias.release();
        if (constantC && broadcast_C != -1) {
            Mat c = broadcast_C == 0 ? mb.load(1, 0) : mb.load(N, 0);
            if (c.empty()) return -100;
            bias.create(N);
            if (bias.empty()) return -100;
            for (int n = 0; n < N; n++) fdata(bias)[n] = beta * fdata(c)[broadcast_C == 0 ? 0 : n];
        }
        return 0;
    }
    virtual int create_pipeline(const Option&) {
        std::lock_guard<std::mutex> lock(mutex);
        return have_device() ? layer_status(upload()) : 0;
    }
    virtual int destroy_pipeline(const Option&) {
        std::lock_guard<std::mutex> lock(mutex);
        release();
        return 0;
    }
    virtual int forward(const Mat& a, Mat& top, const Option& opt) const {
        Shape s;
        if (!shape_of(a, &s) || s.cols != K) return -1;
        HipDeviceAllocator* dev = device_allocator_of(a);
        if (dev) {
            if (alpha != 1.f || K % 8 != 0) return -1;
            std::lock_guard<std::mutex> lock(mutex);
            int ret = upload();
            if (ret != S2_OK) return layer_status(ret);
            top = new_blob(dev, s.dims, s.rows, N, a.elemsize, opt);
            if (top.empty()) return -100;
            ret = s2_shared_linear_forward(a.data, s.rows, 0, 0, dtype_of(a, opt),
                                           static_cast<const uint16_t*>(weight_gpu),
                                           static_cast<const float*>(bias_gpu), N, K, S2_ACT_NONE, top.data,
                                           0, dtype_of(top, opt), dev->stream());
            return layer_status(ret);
        }
        if (!host_ok(a)) return -1;
        top = new_blob(0, s.dims, s.rows, N, 4, opt);
        if (top.empty()) return -100;
        for (int m = 0; m < s.rows; m++)
            for (int n = 0; n < N; n++) {
                float acc = 0.f;
                for (int k = 0; k < K; k++) acc += fdata(a)[(size_t)m * K + k] * fdata(weight)[(size_t)n * K + k];
                fdata(top)[(size_t)m * N + n] = alpha * acc + (bias.empty() ? 0.f : fdata(bias)[n]);
            }
        return 0;
    }
    float alpha, beta;
    int transB, constantC, N, K, broadcast_C;
    Mat weight, bias;   // host fp32 [N][K] and beta C [N]

private:
    // bf16 weight and fp32 bias on the device, made once
    int upload() const {
        if (weight_gpu) return S2_OK;
        const size_t count = (size_t)N * K;
        float* staging = 0;
        int ret = s2_malloc(&weight_gpu, count * 2);
        if (ret == S2_OK) ret = s2_malloc((void**)&staging, count * 4);
        if (ret == S2_OK) ret = s2_memcpy_h2d(staging, weight.data, count * 4, 0);
        if (ret == S2_OK) ret = s2_cast_f32_to_bf16(staging, static_cast<uint16_t*>(weight_gpu), count, 0);
        if (ret == S2_OK && !bias.empty()) {
            ret = s2_malloc(&bias_gpu, (size_t)N * 4);
            if (ret == S2_OK) ret = s2_memcpy_h2d(bias_gpu, bias.data, (size_t)N * 4, 0);
        }
        if (ret == S2_OK) ret = s2_stream_synchronize(0);
        if (staging) s2_free(staging);
        if (ret != S2_OK) release();
        return ret;
    }
    void release() const {
        if (weight_gpu) s2_free(weight_gpu);
        if (bias_gpu) s2_free(bias_gpu);
        weight_gpu = bias_gpu = 0;
    }
    mutable std::mutex mutex;
    mutable void* weight_gpu;
    mutable void* bias_gpu;
};

}  // namespace

Layer* create_builtin_layer(const std::string& type) {
    if (type == "MemoryData") return new MemoryDataLayer();
    if (type == "BinaryOp") return new BinaryOpLayer();
    if (type == "UnaryOp") return new UnaryLayer(-1);
    if (type == "Sigmoid") return new UnaryLayer(100);
    if (type == "Swish") return new UnaryLayer(101);
    if (type == "Reduction") return new ReductionLayer();
    if (type == "RMSNorm") return new RMSNormLayer();
    if (type == "Reshape") return new ReshapeLayer();
    if (type == "Slice") return new SliceLayer();
    if (type == "Concat") return new ConcatLayer();
    if (type == "Crop") return new CropLayer();
    if (type == "Gemm") return new GemmLayer();
    return 0;
}

const Mat* memory_data_of(const Layer* layer) {
    const MemoryDataLayer* m = dynamic_cast<const MemoryDataLayer*>(layer);
    return m ? &m->data : 0;
}

int binary_op_of(const Layer* layer, int* with_scalar, float* b) {
    const BinaryOpLayer* l = dynamic_cast<const BinaryOpLayer*>(layer);
    if (!l) return -1;
    *with_scalar = l->with_scalar;
    *b = l->b;
    return l->op_type;
}

int unary_op_of(const Layer* layer) {
    const UnaryLayer* l = dynamic_cast<const UnaryLayer*>(layer);
    return l ? l->op_type : -1;
}

int reduction_of(const Layer* layer, int* reduce_all, float* coeff, int* keepdims,
                 bool* last_axis_only) {
    const ReductionLayer* l = dynamic_cast<const ReductionLayer*>(layer);
    if (!l) return -1;
    *reduce_all = l->reduce_all;
    *coeff = l->coeff;
    *keepdims = l->keepdims;
    *last_axis_only = !l->reduce_all && l->axes.size() == 1 && (l->axes[0] == -1 || l->axes[0] == 1);
    return l->operation;
}

int rms_norm_of(const Layer* layer, float* eps, int* affine) {
    const RMSNormLayer* l = dynamic_cast<const RMSNormLayer*>(layer);
    if (!l) return -1;
    *eps = l->eps;
    *affine = l->affine;
    return 0;
}

}  // namespace ncnn
