// ncnn-compatible subset: ParamDict (see allocator.h for the scope of this directory).
//
// id -> int / float / array value, as parsed from a .param layer line
// ("0=20 1=128 6=1.000000e-05 ...").  get() returns the default when the id
// was not set.
#ifndef NCNN_PARAMDICT_H
#define NCNN_PARAMDICT_H

#include "mat.h"

#define NCNN_MAX_PARAM_COUNT 32

namespace ncnn {

class ParamDict {
public:
    ParamDict();

    int type(int id) const;   // 0 = unset, 2 = int, 3 = float, 4 = array
    int get(int id, int def) const;
    float get(int id, float def) const;
    Mat get(int id, const Mat& def) const;

    void set(int id, int i);
    void set(int id, float f);
    void set(int id, const Mat& v);

    void clear();

    // Parses the "id=value" fields of one .param layer line (the text after
    // the blob names); "-23300=n,a,b,..." array form included.  Returns 0 or -1.
    int load_param_text(const char* fields);

private:
    struct Entry {
        int type;
        int i;
        float f;
        Mat v;
    } params[NCNN_MAX_PARAM_COUNT];
};

}  // namespace ncnn

#endif  // NCNN_PARAMDICT_H
