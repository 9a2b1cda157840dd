// ncnn-compatible subset: ModelBin (see allocator.h for the scope of this directory).
//
// load(w, type): type 1 reads w raw little-endian fp32 values (the form the
// SeedVR2 custom layers use); type 0 reads a 4-byte tag first and accepts
// the raw fp32 tag (0) and the fp16 tag (0x01306B47).
#ifndef NCNN_MODELBIN_H
#define NCNN_MODELBIN_H

#include <stddef.h>

#include "mat.h"

namespace ncnn {

class ModelBin {
public:
    ModelBin();
    virtual ~ModelBin();
    virtual Mat load(int w, int type) const = 0;
    virtual Mat load(int w, int h, int type) const;
    virtual Mat load(int w, int h, int c, int type) const;
};

// Hands out the given Mats in order, ignoring w and type.
class ModelBinFromMatArray : public ModelBin {
public:
    explicit ModelBinFromMatArray(const Mat* weights);
    virtual ~ModelBinFromMatArray();
    virtual Mat load(int w, int type) const;

private:
    mutable const Mat* weights;
};

// Reads consecutive weights from a memory buffer (a .bin file's bytes).
// An out-of-range read returns an empty Mat.
class ModelBinFromMemory : public ModelBin {
public:
    ModelBinFromMemory(const unsigned char* data, size_t size);
    virtual ~ModelBinFromMemory();
    virtual Mat load(int w, int type) const;
    size_t consumed() const { return offset; }

private:
    const unsigned char* data;
    size_t size;
    mutable size_t offset;
};

}  // namespace ncnn

#endif  // NCNN_MODELBIN_H
