// ncnn-compatible subset: Net and Extractor (see allocator.h for the scope of
// this directory).
//
// Loads a text .param graph (magic 7767517, then "layer_count blob_count",
// then one line per layer: type, name, bottom and top counts, bottom and top
// blob names, id=value params) and its .bin weights (each layer's load_model
// reads its own weights, in layer order), and runs it through an Extractor
// that computes a requested blob from the blobs it depends on, as ncnn's
// does.  Layer types come from the registered custom layers first, then the
// built-ins Input, Split and GELU and those of builtin_layers.h.
//
// Device residency (this build): when the extractor's blob allocator is a
// HipDeviceAllocator (layers/hip_allocator.h), every layer output is a
// device blob of that allocator; host Mats given to input() are uploaded
// once (except blobs only read on the host, Net::host_only_blob), and device
// blobs of another allocator are re-tagged to this one after its stream has
// been ordered behind theirs (s2_stream_wait), so every layer runs on the
// extractor's stream.  In light mode a device blob no slot references any
// more goes back to the allocator's pool for a later layer to reuse.
#ifndef NCNN_NET_H
#define NCNN_NET_H

#include <stddef.h>

#include <memory>
#include <string>
#include <vector>

#include "layer.h"
#include "mat.h"
#include "option.h"

namespace ncnn {

class Blob {
public:
    Blob() : producer(-1), consumer(-1) {}
    std::string name;
    int producer;   // layer index
    int consumer;   // last consuming layer index (-1: none)
    Mat shape;
};

class Extractor;

class Net {
public:
    Net();
    virtual ~Net();

    Option opt;

    // Same contract as ncnn: a creator for a layer type name, an optional
    // destroyer, and the userdata handed to both.  Register before
    // load_param.  Returns 0, or -1 when the type is already registered.
    int register_custom_layer(const char* type, layer_creator_func creator,
                              layer_destroyer_func destroyer = 0, void* userdata = 0);

    // Text .param from a file or from memory.  Returns 0, or -1 on a
    // malformed file, an unknown layer type or a layer's load_param error.
    int load_param(const char* protopath);
    int load_param_mem(const char* mem);

    // .bin weights from a file or from memory, then every layer's
    // create_pipeline(opt).  Returns 0 or the first failing code; the
    // memory form also fails when the data is not consumed exactly.
    int load_model(const char* modelpath);
    int load_model(const unsigned char* mem, size_t size);

    void clear();

    Extractor create_extractor() const;

    // This build: true when every consumer of blob bi reads it on the host
    // (the video_shape / text_length bottoms of AdaptiveWindowAttention,
    // directly or through Split layers).  A device extractor does not upload
    // such a blob when it is given as a host Mat.
    bool host_only_blob(int bi, int depth = 0) const;

    const std::vector<Blob>& blobs() const { return blobs_; }
    const std::vector<Layer*>& layers() const { return layers_; }
    int find_blob_index_by_name(const char* name) const;

    // This build: SharedLinear -> GELU folding.  A GELU layer whose bottom
    // is a SharedLinear top consumed by nothing else becomes a pass-through
    // and the SharedLinear applies erf-GELU in its epilogue (both of its
    // tops must be so followed).  Call after load_model; returns the number
    // of SharedLinear layers folded.
    int fuse_shared_linear_gelu();

    // This build: SharedLinear -> AdaptiveWindowAttention fusion.  When the
    // two tops of a SharedLinear are exactly the video and text QKV blobs of
    // an attention layer (4-input form) and nothing else reads them, the
    // attention layer takes the projection's inputs and runs the projection
    // in its own kernel (s2_awa_qkv_forward): the QKV blobs are never formed.
    // The projection's tops then have no producer (extracting them fails).
    // Device bf16 blobs only (the attention layer returns -1 otherwise).
    // Call after load_model; returns the number of pairs fused.
    int fuse_qkv_attention();

    // This build: the split q / k / v form.  Three SharedLinear layers of
    // the same two token streams whose tops are exactly the video and text
    // q, k and v bottoms of an 8-input AdaptiveWindowAttention (and read by
    // nothing else) become one stacked projection that the attention layer
    // runs itself (s2_awa_qkv_forward, as fuse_qkv_attention).  Returns the
    // number of attention layers so fused.
    int fuse_split_qkv_attention();

    // This build: SwiGLU.  A gate and an up SharedLinear of the same two
    // token streams, whose tops feed, per stream, mul(Swish(gate), up) and
    // nothing else, become one SharedLinear with the fused SwiGLU epilogue
    // (param 3 = 2).  Returns the number of pairs fused.
    int fuse_swiglu();

    // This build: graph rewriting for fusion passes.  The layers `remove`
    // stop running (their objects live until clear()); `fused`, owned by the
    // net from now on, reads `bottoms` and produces `tops`, each a top of a
    // removed layer, and the removed layers' other tops lose their producer
    // (they can no longer be extracted).  Returns the new layer's index, or
    // -1 when a top was not produced by a removed layer.
    int replace_layers(const std::vector<int>& remove, Layer* fused, const std::vector<int>& bottoms,
                       const std::vector<int>& tops);
    // Drops the tops of Split layers that nothing consumes, and Split layers
    // left without a top; returns the number of tops dropped.
    int prune_splits();
    int consumer_count(int blob) const { return consumer_count_[blob]; }
    // The blob a Split top aliases, through any number of Splits.
    int split_source(int blob) const;
    bool removed(int layer) const { return removed_[layer] != 0; }

protected:
    friend class Extractor;
    int forward_layer(int layer_index, std::vector<Mat>& blob_mats, std::vector<int>& pending,
                      const Option& opt, class DeviceRefs* refs) const;

private:
    Net(const Net&);
    Net& operator=(const Net&);
    Layer* create_layer(const std::string& type, int* custom_index) const;

    struct CustomLayer {
        std::string type;
        layer_creator_func creator;
        layer_destroyer_func destroyer;
        void* userdata;
    };
    std::vector<CustomLayer> custom_;
    std::vector<Layer*> layers_;
    std::vector<int> layer_custom_;     // index into custom_ or -1 (built-in)
    std::vector<int> consumer_count_;   // per blob
    std::vector<char> passthrough_;     // per layer: forward copies bottom to top
    std::vector<char> removed_;         // per layer: replaced by a fusion pass
    std::vector<Blob> blobs_;
};

class Extractor {
public:
    ~Extractor();
    Extractor(const Extractor& rhs);
    Extractor& operator=(const Extractor& rhs);

    void clear();
    void set_light_mode(bool enable);
    void set_num_threads(int num_threads);
    void set_blob_allocator(Allocator* allocator);
    void set_workspace_allocator(Allocator* allocator);

    int input(const char* blob_name, const Mat& in);
    int input(int blob_index, const Mat& in);
    // Computes the blob (and what it depends on) and returns it: a device
    // blob when the blob allocator is a HipDeviceAllocator.  type is
    // accepted for source compatibility and ignored.
    int extract(const char* blob_name, Mat& feat, int type = 0);
    int extract(int blob_index, Mat& feat, int type = 0);

protected:
    friend Extractor Net::create_extractor() const;
    Extractor(const Net* net, size_t blob_count);

private:
    const Net* net_;
    std::vector<Mat> blob_mats_;
    std::vector<int> pending_;   // consumers of each blob that have not run yet
    Option opt_;
    std::shared_ptr<class DeviceRefs> refs_;   // shared with copies of this extractor
};

}  // namespace ncnn

#endif  // NCNN_NET_H
