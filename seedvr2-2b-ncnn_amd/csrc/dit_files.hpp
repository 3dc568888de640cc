// dit_files.hpp — host readers of the reference's on-disk formats (read_raw_f,
// ncnn InnerProduct .param/.bin, the merged graph), shared by the C readers
// (dit_files.cpp) and the device loader (dit_model.cpp).  Plain C++: no HIP,
// so that the readers can be built and fuzzed with AddressSanitizer on a host.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <map>
#include <string>
#include <vector>

namespace dit_files {

// Records a formatted message as the thread's last error; returns -1.
int fail(const char* fmt, ...);
const std::string& last_error();

// One InnerProduct layer: weights [n_out][n_in] and optional bias, on the host.
struct HostLinear {
    std::vector<float> w, b;
    int n_out = 0, n_in = 0;
};

// InnerProduct weights at byte off of f (a tagged [n_out * n_in] blob, then
// n_out raw float32 bias values when has_bias), and the same from a layer's
// <base>.param / <base>.bin pair.
int read_tagged_at(std::ifstream& f, int64_t size, int64_t off, int64_t n, const std::string& what,
                   std::vector<float>& v);
int read_linear_at(std::ifstream& f, int64_t size, int64_t off, int n_out, int n_in, bool has_bias,
                   const std::string& what, HostLinear& L);
int read_linear_host(const std::string& base, bool has_bias, HostLinear& L);
// A read_raw_f file: int64 ndim, int64 shape[ndim], float32 data.
int read_raw_host(const std::string& path, std::vector<float>& data, std::vector<int64_t>& shape);

// Where one weight of the model lies in the graph's .bin.
struct GraphBlob {
    enum Kind { LINEAR, TAGGED, RAW } kind;
    int64_t off;
    int64_t n;       // values (LINEAR: n_out * n_in)
    int n_out, n_in;
    bool bias;
};

// The weights of a whole merged graph by their model-directory names
// (vid_in_proj, b3_vid_qkv, b12_all_nq, vid_out_ada_shift, ...).  The .bin
// is the concatenation, in layer order, of what each layer's load_model
// reads (export_dit_graph.py:112-226): AdaCompose 2 x 6 tagged vectors per
// layer (attn_shift, attn_scale, attn_gate, mlp_shift, mlp_scale, mlp_gate,
// ada_compose.cpp:50-79) then the final shift and scale; InnerProduct a
// tagged weight then a raw bias; AWA four tagged 128-vectors (nq_v, nk_v,
// nq_t, nk_t, awa_layer.cpp:38-52); RMSNorm with affine a raw gamma.  Shared
// layers (b<i>_all) appear twice, once per flow; the first is indexed.
struct GraphIndex {
    std::string bin;
    int64_t bin_size = 0;
    int n_layers = 0, mm_layers = -1;
    std::map<std::string, GraphBlob> w;
};

// Indexes the weights of a merged graph (.param text and .bin); mm_hint: the
// number of dual-branch layers when the graph has no AdaCompose layer (-1:
// take it from the graph).
int index_graph(const std::string& param, const std::string& bin, int mm_hint, GraphIndex& G);

// Weights by model-directory name, from a directory or a merged graph.
struct WeightSource {
    virtual ~WeightSource() = default;
    virtual int linear(const std::string& name, bool bias, HostLinear& L) = 0;  // 0 or -1 (fail)
    virtual int vec(const std::string& name, std::vector<float>& v) = 0;
};

struct DirSource : WeightSource {
    std::string root;
    explicit DirSource(const std::string& dir) : root(dir) {
        if (!root.empty() && root.back() != '/') root += '/';
    }
    int linear(const std::string& name, bool bias, HostLinear& L) override {
        return read_linear_host(root + name, bias, L);
    }
    int vec(const std::string& name, std::vector<float>& v) override {
        std::vector<int64_t> sh;
        return read_raw_host(root + name + ".bin", v, sh);
    }
};

// The graph's weights; what it does not hold (the timestep MLP, which the
// host runs outside the graph, dit_graph.cpp:270) comes from the directory.
struct GraphSource : WeightSource {
    GraphIndex G;
    DirSource* dir = nullptr;
    std::ifstream f;
    const GraphBlob* find(const std::string& name) {
        auto it = G.w.find(name);
        return it == G.w.end() ? nullptr : &it->second;
    }
    int open() {
        f.open(G.bin, std::ios::binary);
        return f ? 0 : fail("cannot open %s", G.bin.c_str());
    }
    int missing(const std::string& name) {
        return fail("%s: not in the graph%s", name.c_str(), dir ? "" : " (and no model directory was given)");
    }
    int linear(const std::string& name, bool bias, HostLinear& L) override {
        const GraphBlob* b = find(name);
        if (!b) return dir ? dir->linear(name, bias, L) : missing(name);
        if (b->kind != GraphBlob::LINEAR || b->bias != bias)
            return fail("%s: the graph holds it %s", name.c_str(), b->kind != GraphBlob::LINEAR ? "as a vector"
                                                                   : bias ? "without bias" : "with a bias");
        return read_linear_at(f, G.bin_size, b->off, b->n_out, b->n_in, bias, G.bin + ":" + name, L);
    }
    int vec(const std::string& name, std::vector<float>& v) override {
        const GraphBlob* b = find(name);
        if (!b) return dir ? dir->vec(name, v) : missing(name);
        if (b->kind == GraphBlob::LINEAR) return fail("%s: the graph holds it as an InnerProduct", name.c_str());
        if (b->kind == GraphBlob::TAGGED) return read_tagged_at(f, G.bin_size, b->off, b->n, G.bin + ":" + name, v);
        v.resize(b->n);
        f.clear();
        f.seekg(b->off);
        f.read(reinterpret_cast<char*>(v.data()), 4 * b->n);
        return f ? 0 : fail("%s: read error", name.c_str());
    }
};

template <typename T>
T* copy_out(const std::vector<T>& v) {
    T* p = static_cast<T*>(std::malloc(v.empty() ? 1 : v.size() * sizeof(T)));
    if (p && !v.empty()) std::memcpy(p, v.data(), v.size() * sizeof(T));
    return p;
}

}  // namespace dit_files
