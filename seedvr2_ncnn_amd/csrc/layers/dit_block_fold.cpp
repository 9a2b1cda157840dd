// Folding of the DiT block's norm / modulation / residual chains written with
// ncnn built-ins onto DiTStreamOp passes (dit_block_fold.h).
#include "dit_block_fold.h"

#include <builtin_layers.h>

#include "dit_block_ops.h"

namespace seedvr2 {

namespace {

class Folder
{
public:
    Folder(ncnn::Net& _net, const AdaptiveWindowRuntimeState* _state, const ncnn::Option& _opt)
        : net(_net), state(_state), opt(_opt)
    {
    }

    int run()
    {
        label_streams();
        int made = 0;
        made += pass_ada_in();
        made += pass_ada_out();
        made -= pass_merge();   // two passes become one
        net.prune_splits();
        return made;
    }

private:
    struct Mod
    {
        int input;           // the per-sample [batch][hidden] blob
        ncnn::Mat vec;       // the block's own [hidden] vector, or empty
        std::vector<int> remove;
    };

    const ncnn::Layer* layer(int li) const { return net.layers()[li]; }
    int producer(int blob) const { return blob < 0 ? -1 : net.blobs()[blob].producer; }
    bool single_use(int blob) const { return net.consumer_count(blob) == 1; }

    // The blob a Split top aliases (through any number of Splits).
    int source(int blob) const
    {
        for (int guard = 0; guard < 64; guard++)
        {
            const int p = producer(blob);
            if (p < 0 || layer(p)->type != "Split")
                return blob;
            blob = layer(p)->bottoms[0];
        }
        return blob;
    }

    // Row-stream label of every blob: 0 the video stream (from in0), 1 the
    // text stream (from in1), -1 neither (modulation vectors, shapes).
    void label_streams()
    {
        const std::vector<ncnn::Blob>& blobs = net.blobs();
        labels.assign(blobs.size(), -1);
        for (size_t b = 0; b < blobs.size(); b++)
        {
            if (blobs[b].name == "in0")
                labels[b] = 0;
            if (blobs[b].name == "in1")
                labels[b] = 1;
        }
        const std::vector<ncnn::Layer*>& layers = net.layers();
        for (size_t li = 0; li < layers.size(); li++)
        {
            const ncnn::Layer* l = layers[li];
            if (net.removed((int)li) || l->tops.empty() || l->bottoms.empty())
                continue;   // inputs keep the labels given above
            if (l->type == "AdaptiveWindowAttention" && l->tops.size() == 2)
            {
                labels[l->tops[0]] = 0;
                labels[l->tops[1]] = 1;
                continue;
            }
            if (l->type == "SharedLinear")
            {
                for (size_t t = 0; t < l->tops.size() && t < l->bottoms.size(); t++)
                    labels[l->tops[t]] = labels[l->bottoms[t]];
                continue;
            }
            int s = -1;
            for (size_t i = 0; i < l->bottoms.size() && s < 0; i++)
                s = labels[l->bottoms[i]];
            for (size_t t = 0; t < l->tops.size(); t++)
                labels[l->tops[t]] = s;
        }
    }

    bool is_binary(int li, int op, bool scalar) const
    {
        int with_scalar = 0;
        float b = 0.f;
        return li >= 0 && !net.removed(li) && ncnn::binary_op_of(layer(li), &with_scalar, &b) == op &&
               (with_scalar != 0) == scalar && (int)layer(li)->bottoms.size() == (scalar ? 1 : 2);
    }

    // A modulation operand: the per-sample input, or that input plus a
    // MemoryData [hidden] vector of the block (add, either order).
    bool resolve_mod(int blob, Mod* m) const
    {
        m->vec = ncnn::Mat();
        m->remove.clear();
        const int p = producer(blob);
        if (is_binary(p, 0, false) && single_use(blob))
        {
            for (int j = 0; j < 2; j++)
            {
                const int vb = layer(p)->bottoms[j];
                const int in = layer(p)->bottoms[1 - j];
                const int mp = producer(vb);
                const ncnn::Mat* data = mp >= 0 ? ncnn::memory_data_of(layer(mp)) : 0;
                if (!data || data->dims != 1 || !single_use(vb) || !is_input(in))
                    continue;
                m->input = in;
                m->vec = *data;
                m->remove.push_back(p);
                m->remove.push_back(mp);
                return true;
            }
            return false;
        }
        if (!is_input(blob))
            return false;
        m->input = blob;
        return true;
    }

    // A graph input (or a Split of one) that carries no token stream.
    bool is_input(int blob) const
    {
        const int src = source(blob);
        const int p = producer(src);
        return labels[src] < 0 && p >= 0 && layer(p)->type == "Input";
    }

    // n = rmsnorm(x) without affine: an RMSNorm layer, or
    // x * rsqrt(mean(square(x), last axis, keepdims) + eps).
    bool resolve_norm(int n, int* x, float* eps, std::vector<int>* remove) const
    {
        remove->clear();
        const int p = producer(n);
        if (p < 0 || net.removed(p))
            return false;
        int affine = 1;
        if (ncnn::rms_norm_of(layer(p), eps, &affine) == 0)
        {
            if (affine)
                return false;
            *x = layer(p)->bottoms[0];
            remove->push_back(p);
            return true;
        }
        if (!is_binary(p, 2, false))
            return false;
        for (int k = 0; k < 2; k++)
        {
            const int r = layer(p)->bottoms[k];
            const int xb = layer(p)->bottoms[1 - k];
            const int rp = producer(r);
            if (rp < 0 || !single_use(r) || ncnn::unary_op_of(layer(rp)) != 6)
                continue;
            const int e = layer(rp)->bottoms[0];
            const int ep = producer(e);
            int with_scalar = 0;
            float b = 0.f;
            if (!single_use(e) || ep < 0 || ncnn::binary_op_of(layer(ep), &with_scalar, &b) != 0 ||
                !with_scalar)
                continue;
            const int ms = layer(ep)->bottoms[0];
            const int mp = producer(ms);
            int reduce_all = 0, keepdims = 0;
            float coeff = 0.f;
            bool last = false;
            if (!single_use(ms) || mp < 0 ||
                ncnn::reduction_of(layer(mp), &reduce_all, &coeff, &keepdims, &last) != 3 || !last ||
                !keepdims || coeff != 1.f)
                continue;
            const int sq = layer(mp)->bottoms[0];
            const int sp = producer(sq);
            if (!single_use(sq) || sp < 0)
                continue;
            int xa = -1;
            if (ncnn::unary_op_of(layer(sp)) == 4)
                xa = layer(sp)->bottoms[0];
            else if (is_binary(sp, 2, false) && source(layer(sp)->bottoms[0]) == source(layer(sp)->bottoms[1]))
                xa = layer(sp)->bottoms[0];
            if (xa < 0 || source(xa) != source(xb))
                continue;
            *x = xa;
            *eps = b;
            const int chain[5] = {p, rp, ep, mp, sp};
            remove->assign(chain, chain + 5);
            return true;
        }
        return false;
    }

    int replace(const std::vector<int>& remove, DiTStreamOp* op, const std::vector<int>& bottoms,
                const std::vector<int>& tops)
    {
        op->type = "DiTStreamOp";
        op->name = layer(remove[0])->name;
        if (net.replace_layers(remove, op, bottoms, tops) < 0)
        {
            delete op;
            return -1;
        }
        return op->create_pipeline(opt);
    }

    // h = add(mul(norm(x), S), T)
    int pass_ada_in()
    {
        int made = 0;
        const size_t count = net.layers().size();
        for (size_t li = 0; li < count; li++)
        {
            if (!is_binary((int)li, 0, false))
                continue;
            const ncnn::Layer* add = layer((int)li);
            for (int i = 0; i < 2; i++)
            {
                const int m1 = add->bottoms[i];
                const int T = add->bottoms[1 - i];
                const int mp = producer(m1);
                if (!single_use(m1) || !is_binary(mp, 2, false))
                    continue;
                bool done = false;
                for (int k = 0; k < 2 && !done; k++)
                {
                    const int n = layer(mp)->bottoms[k];
                    const int S = layer(mp)->bottoms[1 - k];
                    int x = -1;
                    float eps = 0.f;
                    std::vector<int> norm;
                    Mod ms, mt;
                    if (!single_use(n) || labels[n] < 0 || !resolve_norm(n, &x, &eps, &norm) ||
                        !resolve_mod(S, &ms) || !resolve_mod(T, &mt) || labels[source(x)] != labels[n])
                        continue;
                    std::vector<int> remove(1, (int)li);
                    remove.push_back(mp);
                    remove.insert(remove.end(), norm.begin(), norm.end());
                    remove.insert(remove.end(), ms.remove.begin(), ms.remove.end());
                    remove.insert(remove.end(), mt.remove.begin(), mt.remove.end());
                    DiTStreamOp* op = new DiTStreamOp(0, labels[n], state, eps, ncnn::Mat(), mt.vec, ms.vec);
                    const int bottoms[3] = {x, mt.input, ms.input};
                    if (replace(remove, op, std::vector<int>(bottoms, bottoms + 3),
                                std::vector<int>(1, add->tops.empty() ? -1 : add->tops[0])) == 0)
                        ++made;
                    done = true;
                }
                if (done)
                    break;
            }
        }
        return made;
    }

    // out = add(x, mul(y, G)), x and y of one token stream
    int pass_ada_out()
    {
        int made = 0;
        const size_t count = net.layers().size();
        for (size_t li = 0; li < count; li++)
        {
            if (!is_binary((int)li, 0, false))
                continue;
            const ncnn::Layer* add = layer((int)li);
            for (int i = 0; i < 2; i++)
            {
                const int g = add->bottoms[i];
                const int xres = add->bottoms[1 - i];
                const int gp = producer(g);
                if (!single_use(g) || !is_binary(gp, 2, false) || labels[xres] < 0)
                    continue;
                bool done = false;
                for (int k = 0; k < 2 && !done; k++)
                {
                    const int y = layer(gp)->bottoms[k];
                    const int G = layer(gp)->bottoms[1 - k];
                    Mod mg;
                    if (labels[y] != labels[xres] || !resolve_mod(G, &mg))
                        continue;
                    std::vector<int> remove(1, (int)li);
                    remove.push_back(gp);
                    remove.insert(remove.end(), mg.remove.begin(), mg.remove.end());
                    DiTStreamOp* op = new DiTStreamOp(1, labels[y], state, 0.f, mg.vec, ncnn::Mat(), ncnn::Mat());
                    const int bottoms[3] = {xres, y, mg.input};
                    if (replace(remove, op, std::vector<int>(bottoms, bottoms + 3),
                                std::vector<int>(1, add->tops[0])) == 0)
                        ++made;
                    done = true;
                }
                if (done)
                    break;
            }
        }
        return made;
    }

    // ada_out whose output feeds an ada_in of the same stream -> ada_out_in
    int pass_merge()
    {
        int merged = 0;
        const size_t count = net.layers().size();
        for (size_t bi = 0; bi < count; bi++)
        {
            if (net.removed((int)bi))
                continue;
            const DiTStreamOp* in = dynamic_cast<const DiTStreamOp*>(layer((int)bi));
            if (!in || in->kind_of() != 0)
                continue;
            const int r = source(in->bottoms[0]);
            const int ap = producer(r);
            const DiTStreamOp* out = ap >= 0 ? dynamic_cast<const DiTStreamOp*>(layer(ap)) : 0;
            if (!out || out->kind_of() != 1 || out->stream_of() != in->stream_of() || net.removed(ap))
                continue;
            DiTStreamOp* op = new DiTStreamOp(2, in->stream_of(), state, in->epsilon_of(), out->vector(0),
                                              in->vector(1), in->vector(2));
            const int bottoms[5] = {out->bottoms[0], out->bottoms[1], out->bottoms[2], in->bottoms[1],
                                    in->bottoms[2]};
            const int tops[2] = {r, in->tops[0]};
            std::vector<int> remove(1, ap);
            remove.push_back((int)bi);
            if (replace(remove, op, std::vector<int>(bottoms, bottoms + 5), std::vector<int>(tops, tops + 2)) == 0)
                ++merged;
        }
        return merged;
    }

    ncnn::Net& net;
    const AdaptiveWindowRuntimeState* state;
    ncnn::Option opt;
    std::vector<int> labels;
};

}  // namespace

int fold_dit_modulation(ncnn::Net& net, const AdaptiveWindowRuntimeState* state)
{
    Folder f(net, state, net.opt);
    return f.run();
}

}  // namespace seedvr2
