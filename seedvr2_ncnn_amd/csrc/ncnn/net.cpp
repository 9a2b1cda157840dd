// ncnn-compatible subset: Net and Extractor (net.h).
#include "net.h"

#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <map>
#include <sstream>

#include "builtin_layers.h"
#include "hip_allocator.h"
#include "modelbin.h"
#include "adaptive_window_attention.h"
#include "shared_linear.h"
#include "paramdict.h"
#include "seedvr2_hip.h"

namespace ncnn {

// ---- built-in layers -------------------------------------------------------

namespace {

// Input: declares a blob the caller provides (params 0/1/2 = w/h/c, unused).
class InputLayer : public Layer {
public:
    InputLayer() {
        one_blob_only = true;
        support_inplace = true;
    }
    virtual int forward_inplace(Mat&, const Option&) const { return 0; }
};

// Split: every top is the bottom blob (a shared reference, no copy).
class SplitLayer : public Layer {
public:
    SplitLayer() {
        one_blob_only = false;
        support_inplace = false;
    }
    virtual int forward(const std::vector<Mat>& bottom_blobs, std::vector<Mat>& top_blobs,
                        const Option&) const {
        for (size_t i = 0; i < top_blobs.size(); i++) top_blobs[i] = bottom_blobs[0];
        return 0;
    }
};

// GELU: y = x * Phi(x), erf form (param 0 fast_gelu must be 0).  Device
// blobs run s2_gelu on the blob allocator's stream; host fp32 Mats run
// on the CPU.
class GeluLayer : public Layer {
public:
    GeluLayer() : fast_gelu(0), passthrough(false) {
        one_blob_only = true;
        support_inplace = false;
    }
    virtual int load_param(const ParamDict& pd) {
        fast_gelu = pd.get(0, 0);
        return fast_gelu == 0 ? 0 : -1;
    }
    virtual int forward(const Mat& bottom, Mat& top, const Option& opt) const {
        if (passthrough) {
            top = bottom;
            return 0;
        }
        seedvr2::HipDeviceAllocator* dev = seedvr2::device_allocator_of(bottom);
        if (dev) {
            if (bottom.dims != 2 || bottom.elempack != 1) return -1;
            seedvr2::HipDeviceAllocator* out = dynamic_cast<seedvr2::HipDeviceAllocator*>(opt.blob_allocator);
            if (!out) out = dev;
            top = out->create_blob(bottom.w, bottom.h, bottom.elemsize);
            if (top.empty()) return -100;
            const int ret = s2_gelu(bottom.data, top.data, (size_t)bottom.w * bottom.h,
                                    seedvr2::device_blob_dtype(bottom.elemsize, opt), dev->stream());
            return seedvr2::layer_status(ret);
        }
        if (bottom.elemsize != 4) return -1;
        top.create_like(bottom, opt.blob_allocator);
        if (top.empty()) return -100;
        const size_t n = bottom.total();
        const float* x = (const float*)bottom.data;
        float* y = (float*)top.data;
        for (size_t i = 0; i < n; i++) y[i] = 0.5f * x[i] * (1.f + erff(x[i] * 0.70710678118654752f));
        return 0;
    }
    int fast_gelu;
    bool passthrough;
};

}  // namespace

// Device blob references held by the blob slots of an extractor and of its
// copies (which share one table): a device block goes back to its
// allocator's pool when the last slot naming it is released (Split tops and
// Input aliases share one block) unless it is pinned (the caller's own, or
// handed out by extract).
class DeviceRefs {
public:
    void add(const Mat& m) {
        seedvr2::HipDeviceAllocator* a = seedvr2::device_allocator_of(m);
        if (a && m.data) ++refs[m.data].count, refs[m.data].alloc = a;
    }
    void pin(const Mat& m) {
        if (seedvr2::device_allocator_of(m) && m.data) refs[m.data].pinned = true;
    }
    void drop(const Mat& m) {
        if (!seedvr2::device_allocator_of(m) || !m.data) return;
        std::map<void*, Ref>::iterator it = refs.find(m.data);
        if (it == refs.end()) return;
        if (--it->second.count <= 0) {
            if (!it->second.pinned) it->second.alloc->release_blob(it->first);
            refs.erase(it);
        }
    }

private:
    struct Ref {
        Ref() : count(0), pinned(false), alloc(0) {}
        int count;
        bool pinned;   // given by the caller or handed out by extract: never pooled
        seedvr2::HipDeviceAllocator* alloc;
    };
    std::map<void*, Ref> refs;
};

// ---- Net -------------------------------------------------------------------

Net::Net() {}

Net::~Net() { clear(); }

int Net::register_custom_layer(const char* type, layer_creator_func creator,
                               layer_destroyer_func destroyer, void* userdata) {
    for (size_t i = 0; i < custom_.size(); i++)
        if (custom_[i].type == type) return -1;
    CustomLayer c;
    c.type = type;
    c.creator = creator;
    c.destroyer = destroyer;
    c.userdata = userdata;
    custom_.push_back(c);
    return 0;
}

Layer* Net::create_layer(const std::string& type, int* custom_index) const {
    *custom_index = -1;
    for (size_t i = 0; i < custom_.size(); i++)
        if (custom_[i].type == type) {
            *custom_index = (int)i;
            Layer* l = custom_[i].creator(custom_[i].userdata);
            if (l) l->userdata = custom_[i].userdata;
            return l;
        }
    if (type == "Input") return new InputLayer();
    if (type == "Split") return new SplitLayer();
    if (type == "GELU") return new GeluLayer();
    return create_builtin_layer(type);
}

void Net::clear() {
    for (size_t i = 0; i < layers_.size(); i++) {
        layers_[i]->destroy_pipeline(opt);
        const int ci = layer_custom_[i];
        if (ci >= 0 && custom_[ci].destroyer)
            custom_[ci].destroyer(layers_[i], custom_[ci].userdata);
        else
            delete layers_[i];
    }
    layers_.clear();
    layer_custom_.clear();
    consumer_count_.clear();
    passthrough_.clear();
    removed_.clear();
    blobs_.clear();
}

bool Net::host_only_blob(int bi, int depth) const {
    if (bi < 0 || bi >= (int)blobs_.size() || depth > 16) return false;
    bool any = false;
    for (size_t li = 0; li < layers_.size(); li++) {
        const Layer* l = layers_[li];
        for (size_t k = 0; k < l->bottoms.size(); k++) {
            if (l->bottoms[k] != bi) continue;
            any = true;
            // the video_shape / text_length blobs of either input form
            if (l->type == "AdaptiveWindowAttention" && l->bottoms.size() >= 4 &&
                k + 2 >= l->bottoms.size())
                continue;
            if (l->type == "Split") {
                for (size_t t = 0; t < l->tops.size(); t++)
                    if (!host_only_blob(l->tops[t], depth + 1)) return false;
                continue;
            }
            return false;
        }
    }
    return any;
}

int Net::find_blob_index_by_name(const char* name) const {
    for (size_t i = 0; i < blobs_.size(); i++)
        if (blobs_[i].name == name) return (int)i;
    return -1;
}

int Net::load_param(const char* protopath) {
    FILE* fp = fopen(protopath, "rb");
    if (!fp) return -1;
    std::string text;
    char buf[65536];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), fp)) > 0) text.append(buf, n);
    fclose(fp);
    return load_param_mem(text.c_str());
}

int Net::load_param_mem(const char* mem) {
    clear();
    std::istringstream in(mem ? mem : "");
    std::string line;
    if (!std::getline(in, line)) return -1;
    if (atoi(line.c_str()) != 7767517) return -1;
    int layer_count = 0, blob_count = 0;
    if (!std::getline(in, line) || sscanf(line.c_str(), "%d %d", &layer_count, &blob_count) != 2 ||
        layer_count <= 0 || blob_count <= 0)
        return -1;
    blobs_.reserve(blob_count);
    while ((int)layers_.size() < layer_count && std::getline(in, line)) {
        std::istringstream ls(line);
        std::string type, name;
        int nb = 0, nt = 0;
        if (!(ls >> type)) continue;   // blank line
        if (!(ls >> name >> nb >> nt) || nb < 0 || nt < 0) {
            clear();
            return -1;
        }
        int ci = -1;
        Layer* layer = create_layer(type, &ci);
        if (!layer) {
            fprintf(stderr, "layer %s not exists or registered\n", type.c_str());
            clear();
            return -1;
        }
        layer->type = type;
        layer->name = name;
        const int li = (int)layers_.size();
        layers_.push_back(layer);
        layer_custom_.push_back(ci);
        passthrough_.push_back(0);
        removed_.push_back(0);
        for (int i = 0; i < nb; i++) {
            std::string b;
            if (!(ls >> b)) {
                clear();
                return -1;
            }
            const int bi = find_blob_index_by_name(b.c_str());
            if (bi < 0) {
                fprintf(stderr, "blob %s of layer %s has no producer\n", b.c_str(), name.c_str());
                clear();
                return -1;
            }
            blobs_[bi].consumer = li;
            consumer_count_[bi]++;
            layer->bottoms.push_back(bi);
        }
        for (int i = 0; i < nt; i++) {
            std::string t;
            if (!(ls >> t)) {
                clear();
                return -1;
            }
            if (find_blob_index_by_name(t.c_str()) >= 0 || (int)blobs_.size() >= blob_count) {
                clear();
                return -1;
            }
            Blob blob;
            blob.name = t;
            blob.producer = li;
            blobs_.push_back(blob);
            consumer_count_.push_back(0);
            layer->tops.push_back((int)blobs_.size() - 1);
        }
        std::string rest;
        std::getline(ls, rest);
        ParamDict pd;
        if (pd.load_param_text(rest.c_str()) != 0 || layer->load_param(pd) != 0) {
            fprintf(stderr, "layer %s load_param failed\n", name.c_str());
            clear();
            return -1;
        }
    }
    if ((int)layers_.size() != layer_count || (int)blobs_.size() != blob_count) {
        clear();
        return -1;
    }
    return 0;
}

int Net::load_model(const char* modelpath) {
    FILE* fp = fopen(modelpath, "rb");
    if (!fp) return -1;
    std::vector<unsigned char> data;
    unsigned char buf[1 << 16];
    size_t n;
    while ((n = fread(buf, 1, sizeof(buf), fp)) > 0) data.insert(data.end(), buf, buf + n);
    fclose(fp);
    return load_model(data.empty() ? 0 : &data[0], data.size());
}

int Net::load_model(const unsigned char* mem, size_t size) {
    if (layers_.empty()) return -1;
    ModelBinFromMemory mb(mem, size);
    for (size_t i = 0; i < layers_.size(); i++) {
        const int ret = layers_[i]->load_model(mb);
        if (ret != 0) {
            fprintf(stderr, "layer %s load_model failed (%d)\n", layers_[i]->name.c_str(), ret);
            return ret;
        }
    }
    if (mb.consumed() != size) return -1;
    for (size_t i = 0; i < layers_.size(); i++) {
        const int ret = layers_[i]->create_pipeline(opt);
        if (ret != 0) return ret;
    }
    return 0;
}

int Net::fuse_shared_linear_gelu() {
    int fused = 0;
    for (size_t li = 0; li < layers_.size(); li++) {
        Layer* l = layers_[li];
        if (l->type != "SharedLinear" || l->tops.empty()) continue;
        std::vector<int> gelus;
        for (size_t t = 0; t < l->tops.size(); t++) {
            const int bi = l->tops[t];
            const int c = blobs_[bi].consumer;
            if (consumer_count_[bi] != 1 || c < 0 || layers_[c]->type != "GELU") break;
            gelus.push_back(c);
        }
        if (gelus.size() != l->tops.size()) continue;
        // only a projection without an epilogue activation of its own: a
        // GELU after a GELU or SwiGLU epilogue stays a layer
        seedvr2::SharedLinear* sl = dynamic_cast<seedvr2::SharedLinear*>(l);
        if (!sl || sl->activation_kind() != S2_ACT_NONE || sl->set_activation(S2_ACT_GELU) != 0)
            continue;
        for (size_t g = 0; g < gelus.size(); g++) {
            static_cast<GeluLayer*>(layers_[gelus[g]])->passthrough = true;
            passthrough_[gelus[g]] = 1;
        }
        ++fused;
    }
    return fused;
}

int Net::fuse_qkv_attention() {
    int fused = 0;
    for (size_t ai = 0; ai < layers_.size(); ai++) {
        Layer* a = layers_[ai];
        if (a->type != "AdaptiveWindowAttention" || a->bottoms.size() != 4) continue;
        const int b0 = a->bottoms[0], b1 = a->bottoms[1];
        const int pi = blobs_[b0].producer;
        if (pi < 0 || blobs_[b1].producer != pi) continue;
        Layer* p = layers_[pi];
        if (p->type != "SharedLinear" || p->bottoms.size() != 2 || p->tops.size() != 2 ||
            p->tops[0] != b0 || p->tops[1] != b1 || consumer_count_[b0] != 1 ||
            consumer_count_[b1] != 1)
            continue;
        seedvr2::SharedLinear* sl = dynamic_cast<seedvr2::SharedLinear*>(p);
        seedvr2::AdaptiveWindowAttention* awa = dynamic_cast<seedvr2::AdaptiveWindowAttention*>(a);
        if (!sl || !awa || awa->set_qkv_projection(sl) != 0) continue;
        // the attention layer reads the projection's inputs in its place
        for (int i = 0; i < 2; i++) {
            const int in = p->bottoms[i];
            a->bottoms[i] = in;
            blobs_[in].consumer = (int)ai;
        }
        p->bottoms.clear();
        for (int i = 0; i < 2; i++) {
            blobs_[p->tops[i]].producer = -1;
            consumer_count_[p->tops[i]] = 0;
        }
        ++fused;
    }
    return fused;
}

int Net::replace_layers(const std::vector<int>& remove, Layer* fused, const std::vector<int>& bottoms,
                        const std::vector<int>& tops) {
    for (size_t i = 0; i < tops.size(); i++) {
        const int p = blobs_[tops[i]].producer;
        bool ok = false;
        for (size_t r = 0; r < remove.size(); r++) ok = ok || remove[r] == p;
        if (!ok) return -1;
    }
    for (size_t r = 0; r < remove.size(); r++) {
        Layer* l = layers_[remove[r]];
        for (size_t i = 0; i < l->bottoms.size(); i++) consumer_count_[l->bottoms[i]]--;
        for (size_t i = 0; i < l->tops.size(); i++) blobs_[l->tops[i]].producer = -1;
        l->bottoms.clear();
        l->tops.clear();
        removed_[remove[r]] = 1;
    }
    const int li = (int)layers_.size();
    layers_.push_back(fused);
    layer_custom_.push_back(-1);
    passthrough_.push_back(0);
    removed_.push_back(0);
    fused->bottoms = bottoms;
    fused->tops = tops;
    for (size_t i = 0; i < bottoms.size(); i++) {
        consumer_count_[bottoms[i]]++;
        blobs_[bottoms[i]].consumer = li;
    }
    for (size_t i = 0; i < tops.size(); i++) blobs_[tops[i]].producer = li;
    return li;
}

int Net::prune_splits() {
    int dropped = 0;
    for (bool again = true; again;) {
        again = false;
        for (size_t li = 0; li < layers_.size(); li++) {
            Layer* l = layers_[li];
            if (removed_[li] || l->type != "Split") continue;
            std::vector<int> keep;
            for (size_t t = 0; t < l->tops.size(); t++) {
                if (consumer_count_[l->tops[t]] > 0) {
                    keep.push_back(l->tops[t]);
                } else {
                    blobs_[l->tops[t]].producer = -1;
                    ++dropped;
                }
            }
            if (keep.size() == l->tops.size()) continue;
            l->tops = keep;
            if (keep.empty()) {
                for (size_t i = 0; i < l->bottoms.size(); i++) consumer_count_[l->bottoms[i]]--;
                l->bottoms.clear();
                removed_[li] = 1;
                again = true;
            }
        }
    }
    return dropped;
}

int Net::split_source(int blob) const {
    for (int guard = 0; guard < 64 && blob >= 0; guard++) {
        const int p = blobs_[blob].producer;
        if (p < 0 || layers_[p]->type != "Split") break;
        blob = layers_[p]->bottoms[0];
    }
    return blob;
}

int Net::fuse_split_qkv_attention() {
    int fused = 0;
    const size_t count = layers_.size();
    for (size_t ai = 0; ai < count; ai++) {
        Layer* a = layers_[ai];
        if (removed_[ai] || a->type != "AdaptiveWindowAttention" || a->bottoms.size() != 8) continue;
        seedvr2::AdaptiveWindowAttention* awa = dynamic_cast<seedvr2::AdaptiveWindowAttention*>(a);
        std::vector<const seedvr2::SharedLinear*> parts;
        std::vector<int> part_layers;
        bool ok = awa != 0;
        for (int j = 0; ok && j < 3; j++) {
            // q, k, v: one projection each, its video top in slot j, its
            // text top in slot 3 + j, read by nothing else
            const int bv = a->bottoms[j], bt = a->bottoms[3 + j];
            const int p = blobs_[bv].producer;
            const seedvr2::SharedLinear* sl =
                p >= 0 ? dynamic_cast<const seedvr2::SharedLinear*>(layers_[p]) : 0;
            ok = sl && blobs_[bt].producer == p && layers_[p]->bottoms.size() == 2 &&
                 layers_[p]->tops.size() == 2 && layers_[p]->tops[0] == bv && layers_[p]->tops[1] == bt &&
                 consumer_count_[bv] == 1 && consumer_count_[bt] == 1;
            if (ok && j > 0)   // all three read the same two token streams
                ok = split_source(layers_[p]->bottoms[0]) == split_source(layers_[part_layers[0]]->bottoms[0]) &&
                     split_source(layers_[p]->bottoms[1]) == split_source(layers_[part_layers[0]]->bottoms[1]);
            if (ok) {
                parts.push_back(sl);
                part_layers.push_back(p);
            }
        }
        if (!ok) continue;
        seedvr2::SharedLinear* qkv = seedvr2::SharedLinear::stack(parts, S2_ACT_NONE);
        if (!qkv) continue;
        qkv->name = layers_[part_layers[0]]->name + "_stacked_qkv";
        if (qkv->create_pipeline(opt) != 0 || awa->set_qkv_projection(qkv) != 0) {
            qkv->destroy_pipeline(opt);
            delete qkv;
            continue;
        }
        const int in_v = layers_[part_layers[0]]->bottoms[0];
        const int in_t = layers_[part_layers[0]]->bottoms[1];
        // the three projections stop running; the stacked one (owned by the
        // net, run by the attention layer) takes their place
        replace_layers(part_layers, qkv, std::vector<int>(), std::vector<int>());
        // the attention now reads the token streams and the two shape blobs
        for (int j = 0; j < 6; j++) consumer_count_[a->bottoms[j]]--;
        const int shape = a->bottoms[6], length = a->bottoms[7];
        a->bottoms.clear();
        a->bottoms.push_back(in_v);
        a->bottoms.push_back(in_t);
        a->bottoms.push_back(shape);
        a->bottoms.push_back(length);
        consumer_count_[in_v]++;
        consumer_count_[in_t]++;
        blobs_[in_v].consumer = blobs_[in_t].consumer = (int)ai;
        ++fused;
    }
    if (fused) prune_splits();
    return fused;
}

int Net::fuse_swiglu() {
    int fused = 0;
    const size_t count = layers_.size();
    for (size_t gi = 0; gi < count; gi++) {
        seedvr2::SharedLinear* gate = dynamic_cast<seedvr2::SharedLinear*>(layers_[gi]);
        if (removed_[gi] || !gate || layers_[gi]->tops.size() != 2 || layers_[gi]->bottoms.size() != 2) continue;
        // per stream: y = mul(swish(g), u) with g this projection's top and
        // u the matching top of one other projection of the same inputs
        std::vector<int> remove(1, (int)gi);
        std::vector<int> outs;
        int ui = -1;
        bool ok = true;
        for (int t = 0; ok && t < 2; t++) {
            const int g = layers_[gi]->tops[t];
            ok = consumer_count_[g] == 1;
            int si = -1, mi = -1;
            for (size_t li = 0; ok && li < count && si < 0; li++)
                if (!removed_[li] && layers_[li]->type == "Swish" && layers_[li]->bottoms.size() == 1 &&
                    layers_[li]->bottoms[0] == g)
                    si = (int)li;
            ok = ok && si >= 0 && consumer_count_[layers_[si]->tops[0]] == 1;
            const int act = ok ? layers_[si]->tops[0] : -1;
            int with_scalar = 0;
            float bs = 0.f;
            for (size_t li = 0; ok && li < count && mi < 0; li++)
                if (!removed_[li] && binary_op_of(layers_[li], &with_scalar, &bs) == 2 && !with_scalar &&
                    layers_[li]->bottoms.size() == 2 &&
                    (layers_[li]->bottoms[0] == act || layers_[li]->bottoms[1] == act))
                    mi = (int)li;
            ok = ok && mi >= 0;
            if (!ok) break;
            const int u = layers_[mi]->bottoms[0] == act ? layers_[mi]->bottoms[1] : layers_[mi]->bottoms[0];
            const int up = blobs_[u].producer;
            ok = up >= 0 && up != (int)gi && (ui < 0 || ui == up) && consumer_count_[u] == 1 &&
                 layers_[up]->tops.size() == 2 && layers_[up]->tops[t] == u &&
                 dynamic_cast<seedvr2::SharedLinear*>(layers_[up]) != 0;
            ui = up;
            remove.push_back(si);
            remove.push_back(mi);
            outs.push_back(layers_[mi]->tops[0]);
        }
        if (!ok || layers_[ui]->bottoms.size() != 2 ||
            split_source(layers_[ui]->bottoms[0]) != split_source(layers_[gi]->bottoms[0]) ||
            split_source(layers_[ui]->bottoms[1]) != split_source(layers_[gi]->bottoms[1]))
            continue;
        std::vector<const seedvr2::SharedLinear*> parts;
        parts.push_back(gate);
        parts.push_back(dynamic_cast<seedvr2::SharedLinear*>(layers_[ui]));
        seedvr2::SharedLinear* sw = seedvr2::SharedLinear::stack(parts, S2_ACT_SWIGLU);
        if (!sw) continue;
        sw->name = layers_[gi]->name + "_swiglu";
        if (sw->create_pipeline(opt) != 0) {
            sw->destroy_pipeline(opt);
            delete sw;
            continue;
        }
        const std::vector<int> bottoms = layers_[gi]->bottoms;
        remove.push_back(ui);
        replace_layers(remove, sw, bottoms, outs);
        ++fused;
    }
    if (fused) prune_splits();
    return fused;
}

Extractor Net::create_extractor() const { return Extractor(this, blobs_.size()); }

// Runs layer `li` after every producer of its bottoms (depth-first with an
// explicit stack), as ncnn's Extractor does.
int Net::forward_layer(int li, std::vector<Mat>& blob_mats, std::vector<int>& pending,
                       const Option& opt, DeviceRefs* refs) const {
    std::vector<int> stack(1, li);
    while (!stack.empty()) {
        const int cur = stack.back();
        const Layer* layer = layers_[cur];
        bool ready = true;
        for (size_t i = 0; i < layer->bottoms.size(); i++) {
            const int bi = layer->bottoms[i];
            if (blob_mats[bi].dims == 0) {
                const int p = blobs_[bi].producer;
                if (p < 0 || p == cur) return -1;
                for (size_t s = 0; s < stack.size(); s++)
                    if (stack[s] == p) return -1;   // a cycle: not a valid graph
                if (layers_[p]->type == "Input") {
                    fprintf(stderr, "blob %s has no input\n", blobs_[bi].name.c_str());
                    return -1;
                }
                stack.push_back(p);
                ready = false;
                break;
            }
        }
        if (!ready) continue;
        stack.pop_back();
        // already computed through another path
        bool done = !layer->tops.empty();
        for (size_t i = 0; i < layer->tops.size(); i++)
            if (blob_mats[layer->tops[i]].dims == 0) done = false;
        if (done) continue;

        std::vector<Mat> bottoms(layer->bottoms.size());
        for (size_t i = 0; i < layer->bottoms.size(); i++) bottoms[i] = blob_mats[layer->bottoms[i]];
        std::vector<Mat> tops(layer->tops.size());
        int ret = 0;
        if (layer->one_blob_only) {
            if (bottoms.size() != 1 || tops.size() != 1) return -1;
            if (layer->support_inplace) {
                tops[0] = bottoms[0];
                ret = layer->forward_inplace(tops[0], opt);
            } else {
                ret = layer->forward(bottoms[0], tops[0], opt);
            }
        } else if (layer->support_inplace) {
            tops = bottoms;
            ret = layer->forward_inplace(tops, opt);
        } else {
            ret = layer->forward(bottoms, tops, opt);
        }
        if (ret != 0) {
            fprintf(stderr, "layer %s forward failed (%d)\n", layer->name.c_str(), ret);
            return ret;
        }
        for (size_t i = 0; i < tops.size(); i++) {
            blob_mats[layer->tops[i]] = tops[i];
            if (refs) refs->add(tops[i]);
        }
        // light mode: a bottom every consumer has taken is released; a device
        // block no slot names any more returns to its allocator's pool
        for (size_t i = 0; i < layer->bottoms.size(); i++) {
            const int bi = layer->bottoms[i];
            if (--pending[bi] == 0 && opt.lightmode) {
                if (refs) refs->drop(blob_mats[bi]);
                blob_mats[bi].release();
            }
        }
    }
    return 0;
}

// ---- Extractor ---------------------------------------------------------------

Extractor::Extractor(const Net* net, size_t blob_count)
    : net_(net), blob_mats_(blob_count), pending_(net->consumer_count_), opt_(net->opt),
      refs_(new DeviceRefs()) {}

Extractor::~Extractor() { clear(); }

// A copy shares rhs's reference table and adds its own references to the
// blobs it names, so a block goes back to the pool only when neither
// extractor names it any more.
Extractor::Extractor(const Extractor& rhs)
    : net_(rhs.net_), blob_mats_(rhs.blob_mats_), pending_(rhs.pending_), opt_(rhs.opt_),
      refs_(rhs.refs_) {
    for (size_t i = 0; i < blob_mats_.size(); i++) refs_->add(blob_mats_[i]);
}

Extractor& Extractor::operator=(const Extractor& rhs) {
    if (this == &rhs) return *this;
    clear();
    net_ = rhs.net_;
    blob_mats_ = rhs.blob_mats_;
    pending_ = rhs.pending_;
    opt_ = rhs.opt_;
    refs_ = rhs.refs_;
    for (size_t i = 0; i < blob_mats_.size(); i++) refs_->add(blob_mats_[i]);
    return *this;
}

// Releases every slot; device blocks this extractor alone still named (its
// intermediates and uploads) go back to their allocator's pool.
void Extractor::clear() {
    for (size_t i = 0; i < blob_mats_.size(); i++) {
        if (refs_) refs_->drop(blob_mats_[i]);
        blob_mats_[i].release();
    }
    refs_.reset(new DeviceRefs());
    if (net_) pending_ = net_->consumer_count_;
}

void Extractor::set_light_mode(bool enable) { opt_.lightmode = enable; }
void Extractor::set_num_threads(int num_threads) { opt_.num_threads = num_threads; }
void Extractor::set_blob_allocator(Allocator* allocator) { opt_.blob_allocator = allocator; }
void Extractor::set_workspace_allocator(Allocator* allocator) { opt_.workspace_allocator = allocator; }

int Extractor::input(const char* blob_name, const Mat& in) {
    const int bi = net_->find_blob_index_by_name(blob_name);
    if (bi < 0) return -1;
    return input(bi, in);
}

int Extractor::input(int blob_index, const Mat& in) {
    if (blob_index < 0 || blob_index >= (int)blob_mats_.size()) return -1;
    seedvr2::HipDeviceAllocator* dev =
        dynamic_cast<seedvr2::HipDeviceAllocator*>(opt_.blob_allocator);
    seedvr2::HipDeviceAllocator* src = seedvr2::device_allocator_of(in);
    Mat m = in;
    bool upload = false;
    if (dev && src && src != dev) {
        // a device blob of another allocator: this graph's stream waits for
        // the work its producer enqueued, and its consumers run on this
        // graph's stream (layers launch on their bottom blob's allocator's)
        if (s2_stream_wait(dev->stream(), src->stream()) != S2_OK) return -100;
        m.allocator = dev;
    } else if (dev && !src && (in.dims == 1 || in.dims == 2) && !in.empty() &&
               (in.elemsize == 4 || in.elemsize == 2) && !net_->host_only_blob(blob_index)) {
        // host blob into a device graph: one upload on the allocator's
        // stream, owned by this extractor (pooled again once consumed)
        m = dev->create_blob(in.w, in.dims == 1 ? 1 : in.h, in.elemsize);
        if (m.empty()) return -100;
        if (in.dims == 1) m.dims = 1;
        if (s2_memcpy_h2d(m.data, in.data, (size_t)in.w * in.h * in.elemsize, dev->stream()) != S2_OK)
            return -100;
        upload = true;
    }
    if (blob_mats_[blob_index].dims) {
        refs_->drop(blob_mats_[blob_index]);
        blob_mats_[blob_index].release();
    }
    blob_mats_[blob_index] = m;
    refs_->add(m);
    if (!upload) refs_->pin(m);
    return 0;
}

int Extractor::extract(const char* blob_name, Mat& feat, int type) {
    const int bi = net_->find_blob_index_by_name(blob_name);
    if (bi < 0) return -1;
    return extract(bi, feat, type);
}

int Extractor::extract(int blob_index, Mat& feat, int /*type*/) {
    if (blob_index < 0 || blob_index >= (int)blob_mats_.size()) return -1;
    if (blob_mats_[blob_index].dims == 0) {
        const int p = net_->blobs_[blob_index].producer;
        if (p < 0) return -1;
        const int ret = net_->forward_layer(p, blob_mats_, pending_, opt_, refs_.get());
        if (ret != 0) return ret;
    }
    feat = blob_mats_[blob_index];
    refs_->pin(feat);
    return feat.dims == 0 ? -1 : 0;
}

}  // namespace ncnn
