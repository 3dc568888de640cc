// dit_model.cpp — readers of the reference's on-disk formats (read_raw_f,
// ncnn InnerProduct .param/.bin, window files) and the loader of a model
// directory in its layout onto the device.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <algorithm>
#include <fstream>
#include <map>
#include <memory>
#include <sstream>
#include <string>
#include <vector>

#include "dit_internal.hpp"
#include "dit_model.h"

using namespace awa;

namespace {

thread_local std::string g_err;

int fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}

// IEEE 754 binary16 -> binary32 (exact): sign, 5-bit exponent (bias 15),
// 10-bit fraction; exponent 0: subnormal (fraction x 2^-24), 31: inf / NaN.
float half_to_float(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    float v;
    if (e == 0) v = std::ldexp((float)m, -24);
    else if (e == 31) v = m ? NAN : INFINITY;
    else v = std::ldexp((float)(m | 1024), e - 25);
    return (h & 0x8000) ? -v : v;
}

bool file_size(std::ifstream& f, int64_t* n) {
    f.seekg(0, std::ios::end);
    *n = (int64_t)f.tellg();
    f.seekg(0, std::ios::beg);
    return *n >= 0;
}

constexpr uint32_t TAG_FP16 = 0x01306B47u;  // ncnn weight storage tags
constexpr uint32_t TAG_FP32 = 0u;

// One InnerProduct layer: weights [n_out][n_in] and optional bias, on the host.
struct HostLinear {
    std::vector<float> w, b;
    int n_out = 0, n_in = 0;
};

// Bytes of an ncnn "type 0" blob of n values after its 4-byte tag: fp16
// values padded to a multiple of 4 bytes, or fp32 (ModelBinFromDataReader).
bool tagged_bytes(uint32_t tag, int64_t n, int64_t* bytes) {
    if (tag == TAG_FP16) *bytes = (2 * n + 3) / 4 * 4;
    else if (tag == TAG_FP32) *bytes = 4 * n;
    else return false;
    return true;
}

// n values of a "type 0" blob at byte off of f (the tag first).
int read_tagged_at(std::ifstream& f, int64_t size, int64_t off, int64_t n, const std::string& what,
                   std::vector<float>& v) {
    uint32_t tag = 0;
    f.clear();
    f.seekg(off);
    f.read(reinterpret_cast<char*>(&tag), 4);
    int64_t bytes = 0;
    if (!f) return fail("%s: read error", what.c_str());
    if (!tagged_bytes(tag, n, &bytes)) return fail("%s: unsupported weight storage tag 0x%08x", what.c_str(), tag);
    if (size < off + 4 + bytes)
        return fail("%s: %lld bytes, short of %lld values", what.c_str(), (long long)size, (long long)n);
    v.resize(n);
    if (tag == TAG_FP16) {
        std::vector<uint16_t> h(n);
        f.read(reinterpret_cast<char*>(h.data()), 2 * n);
        for (int64_t i = 0; i < n; i++) v[i] = half_to_float(h[i]);
    } else {
        f.read(reinterpret_cast<char*>(v.data()), 4 * n);
    }
    if (!f) return fail("%s: read error", what.c_str());
    return 0;
}

// InnerProduct weights at byte off: a tagged [n_out * n_in] blob, then for
// layers with bias n_out raw float32 values (InnerProduct::load_model).
int read_linear_at(std::ifstream& f, int64_t size, int64_t off, int n_out, int n_in, bool has_bias,
                   const std::string& what, HostLinear& L) {
    L.n_out = n_out;
    L.n_in = n_in;
    const int64_t n = (int64_t)n_out * n_in;
    if (read_tagged_at(f, size, off, n, what, L.w)) return -1;
    L.b.clear();
    if (has_bias) {
        uint32_t tag = 0;
        f.seekg(off);
        f.read(reinterpret_cast<char*>(&tag), 4);
        int64_t bytes = 0;
        tagged_bytes(tag, n, &bytes);
        const int64_t boff = off + 4 + bytes;
        if (size < boff + 4 * (int64_t)n_out)
            return fail("%s: %lld bytes, short of the %d x %d weight and bias", what.c_str(), (long long)size, n_out,
                        n_in);
        L.b.resize(n_out);
        f.seekg(boff);
        f.read(reinterpret_cast<char*>(L.b.data()), 4 * (int64_t)n_out);
        if (!f) return fail("%s: read error", what.c_str());
    }
    return 0;
}

int read_linear_host(const std::string& base, bool has_bias, HostLinear& L) {
    std::ifstream pf(base + ".param");
    if (!pf) return fail("cannot open %s.param", base.c_str());
    std::string line;
    long numout = -1, total = -1;
    while (std::getline(pf, line)) {
        std::istringstream ss(line);
        std::string type;
        if (!(ss >> type) || type != "InnerProduct") continue;
        std::string tok;
        while (ss >> tok) {
            if (tok.rfind("0=", 0) == 0) numout = std::strtol(tok.c_str() + 2, nullptr, 10);
            if (tok.rfind("2=", 0) == 0) total = std::strtol(tok.c_str() + 2, nullptr, 10);
        }
        break;
    }
    if (numout <= 0 || total <= 0 || total % numout)
        return fail("%s.param: no InnerProduct line with 0=num_output and 2=weight_data_size", base.c_str());
    std::ifstream bf(base + ".bin", std::ios::binary);
    if (!bf) return fail("cannot open %s.bin", base.c_str());
    int64_t size;
    file_size(bf, &size);
    return read_linear_at(bf, size, 0, (int)numout, (int)(total / numout), has_bias, base + ".bin", L);
}

int read_raw_host(const std::string& path, std::vector<float>& data, std::vector<int64_t>& shape) {
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail("cannot open %s", path.c_str());
    int64_t size;
    file_size(f, &size);
    int64_t nd = -1;
    f.read(reinterpret_cast<char*>(&nd), 8);
    if (!f || nd < 0 || nd > 8) return fail("%s: bad ndim %lld", path.c_str(), (long long)nd);
    shape.resize(nd);
    int64_t total = 1;
    for (auto& d : shape) {
        f.read(reinterpret_cast<char*>(&d), 8);
        if (!f || d < 0 || (d > 0 && total > ((int64_t)1 << 40) / d)) return fail("%s: bad shape", path.c_str());
        total *= d;
    }
    if (size < 8 + 8 * nd + 4 * total)
        return fail("%s: %lld bytes, short of %lld floats", path.c_str(), (long long)size, (long long)total);
    data.resize(total);
    f.read(reinterpret_cast<char*>(data.data()), 4 * total);
    if (!f) return fail("%s: read error", path.c_str());
    return 0;
}

// ---- the merged 32-layer graph (export_dit_graph.py) ----

// One layer line of an ncnn .param: type, name, bottom/top counts and the
// integer-keyed parameters (values kept as text).
struct ParamLayer {
    std::string type, name;
    std::map<int, std::string> kv;
    long geti(int k, long dflt) const {
        auto it = kv.find(k);
        return it == kv.end() ? dflt : std::strtol(it->second.c_str(), nullptr, 10);
    }
};

int parse_param(const std::string& path, std::vector<ParamLayer>& layers) {
    std::ifstream f(path);
    if (!f) return fail("cannot open %s", path.c_str());
    long magic = 0, n_layers = -1, n_blobs = -1;
    f >> magic >> n_layers >> n_blobs;
    if (!f || magic != 7767517 || n_layers < 0) return fail("%s: not an ncnn .param (magic %ld)", path.c_str(), magic);
    std::string line;
    std::getline(f, line);
    while ((long)layers.size() < n_layers && std::getline(f, line)) {
        std::istringstream ss(line);
        ParamLayer L;
        int nb = -1, nt = -1;
        if (!(ss >> L.type)) continue;  // blank line
        if (!(ss >> L.name >> nb >> nt) || nb < 0 || nt < 0)
            return fail("%s: bad layer line '%s'", path.c_str(), line.c_str());
        std::string tok;
        for (int i = 0; i < nb + nt; i++)
            if (!(ss >> tok)) return fail("%s: layer %s lists too few blobs", path.c_str(), L.name.c_str());
        while (ss >> tok) {
            const size_t eq = tok.find('=');
            if (eq == std::string::npos) return fail("%s: layer %s: bad parameter '%s'", path.c_str(), L.name.c_str(), tok.c_str());
            L.kv[std::atoi(tok.substr(0, eq).c_str())] = tok.substr(eq + 1);
        }
        layers.push_back(std::move(L));
    }
    if ((long)layers.size() != n_layers)
        return fail("%s: %ld layers declared, %zu found", path.c_str(), n_layers, layers.size());
    return 0;
}

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

// Split "<kind>_<i>_<flow>" (qkv_3_v); false if the name has another form.
bool split_name(const std::string& name, std::string& kind, int& idx, char& flow) {
    const size_t a = name.find('_'), b = name.rfind('_');
    if (a == std::string::npos || b == a || b + 2 != name.size()) return false;
    kind = name.substr(0, a);
    const std::string mid = name.substr(a + 1, b - a - 1);
    if (mid.empty() || mid.find_first_not_of("0123456789") != std::string::npos) return false;
    idx = std::atoi(mid.c_str());
    flow = name[b + 1];
    return flow == 'v' || flow == 't';
}

int index_graph(const std::string& param, const std::string& bin, int mm_hint, GraphIndex& G) {
    std::vector<ParamLayer> layers;
    if (parse_param(param, layers)) return -1;
    std::ifstream f(bin, std::ios::binary);
    if (!f) return fail("cannot open %s", bin.c_str());
    G.bin = bin;
    file_size(f, &G.bin_size);
    // the dual/shared split names the weights: from AdaCompose's 2=, else the caller
    int mm = mm_hint;
    bool whole = false;
    for (const ParamLayer& L : layers) {
        if (L.type == "AdaCompose") {
            const int m = (int)L.geti(2, 10);
            if (mm >= 0 && mm != m)
                return fail("%s: AdaCompose has %d dual-branch layers, %d were asked for", param.c_str(), m, mm);
            mm = m;
        }
        if (L.type == "Input" && L.name == "in_vid0") whole = true;
    }
    if (!whole) return fail("%s: no in_vid0 input: a block of layers, not a whole model graph", param.c_str());
    if (mm < 0) return fail("%s: no AdaCompose layer: pass the number of dual-branch layers", param.c_str());
    G.mm_layers = mm;
    auto branch = [&](int i, char flow) {
        return "b" + std::to_string(i) + (i < mm ? (flow == 'v' ? "_vid" : "_txt") : "_all");
    };
    int64_t off = 0;
    auto add = [&](const std::string& name, GraphBlob b) {
        if (!name.empty() && !G.w.count(name)) G.w[name] = b;
    };
    // a tagged blob of n values at off: its extent
    auto tagged = [&](const std::string& name, int64_t n, const std::string& layer) -> int {
        uint32_t tag = 0;
        f.clear();
        f.seekg(off);
        f.read(reinterpret_cast<char*>(&tag), 4);
        int64_t bytes = 0;
        if (!f) return fail("%s: ends inside layer %s", bin.c_str(), layer.c_str());
        if (!tagged_bytes(tag, n, &bytes))
            return fail("%s: layer %s: unsupported weight storage tag 0x%08x", bin.c_str(), layer.c_str(), tag);
        add(name, GraphBlob{GraphBlob::TAGGED, off, n, (int)n, 0, false});
        off += 4 + bytes;
        return 0;
    };
    int n_awa = 0, max_awa = -1;
    for (const ParamLayer& L : layers) {
        const std::string& t = L.type;
        if (t == "Input" || t == "BinaryOp" || t == "Swish" || t == "Cast" || t == "Split" || t == "Noop") continue;
        if (t == "InnerProduct") {
            const long nout = L.geti(0, 0), bias = L.geti(1, 0), total = L.geti(2, 0);
            if (nout <= 0 || total <= 0 || total % nout)
                return fail("%s: InnerProduct %s: 0=%ld 2=%ld", param.c_str(), L.name.c_str(), nout, total);
            std::string name, kind;
            int i;
            char fl;
            if (L.name == "proj_vid_in") name = "vid_in_proj";
            else if (L.name == "proj_txt_in") name = "txt_in";
            else if (L.name == "outproj") name = "vid_out_proj";
            else if (split_name(L.name, kind, i, fl)) {
                const char* suf = kind == "qkv" ? "_qkv" : kind == "out" ? "_out" : kind == "min" ? "_mlp_in"
                                : kind == "mig" ? "_mlp_g" : kind == "mout" ? "_mlp_out" : nullptr;
                if (suf) name = branch(i, fl) + suf;
            }
            if (name.empty()) return fail("%s: unknown InnerProduct layer %s", param.c_str(), L.name.c_str());
            const int64_t start = off;
            if (tagged("", total, L.name)) return -1;
            off += bias ? 4 * nout : 0;
            add(name, GraphBlob{GraphBlob::LINEAR, start, total, (int)nout, (int)(total / nout), bias != 0});
        } else if (t == "AWA") {
            std::string kind;
            int i;
            char fl;
            if (!split_name(L.name + "_v", kind, i, fl) || kind != "awa")
                return fail("%s: unknown AWA layer %s", param.c_str(), L.name.c_str());
            n_awa++;
            max_awa = std::max(max_awa, i);
            for (const char* nm : {"_nq", "_nk"}) if (tagged(branch(i, 'v') + nm, 128, L.name)) return -1;
            for (const char* nm : {"_nq", "_nk"}) if (tagged(branch(i, 't') + nm, 128, L.name)) return -1;
        } else if (t == "AdaCompose") {
            const long nl = L.geti(1, 32), dim = L.geti(3, 2560), fin = L.geti(4, 1);
            for (int i = 0; i < nl; i++)
                for (char fl : {'v', 't'})
                    for (const char* nm : {"_attn_shift", "_attn_scale", "_attn_gate", "_mlp_shift", "_mlp_scale",
                                           "_mlp_gate"})
                        if (tagged(branch(i, fl) + nm, dim, L.name)) return -1;
            if (fin && (tagged("vid_out_ada_shift", dim, L.name) || tagged("vid_out_ada_scale", dim, L.name)))
                return -1;
        } else if (t == "RMSNorm") {
            if (L.geti(2, 0)) {
                const long n = L.geti(0, 0);
                if (L.name == "rn_fin") add("vid_out_norm_w", GraphBlob{GraphBlob::RAW, off, n, (int)n, 0, false});
                off += 4 * n;
            }
        } else {
            return fail("%s: layer type %s (%s) is not part of the DiT graph", param.c_str(), t.c_str(),
                        L.name.c_str());
        }
        if (off > G.bin_size)
            return fail("%s: %lld bytes end inside layer %s", bin.c_str(), (long long)G.bin_size, L.name.c_str());
    }
    if (off != G.bin_size)
        return fail("%s: the layers read %lld of its %lld bytes", bin.c_str(), (long long)off, (long long)G.bin_size);
    if (n_awa != max_awa + 1) return fail("%s: AWA layers are not numbered 0..%d", param.c_str(), n_awa - 1);
    G.n_layers = n_awa;
    return 0;
}

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

}  // namespace

struct dit_model {
    int device = 0;
    int n_layers = 0, mm_layers = 0, mlp = 0;
    std::vector<void*> allocs;       // every device buffer of the model
    std::vector<dit_branch> vb, tb;  // per layer (tb[i] == vb[i] for shared layers)
    dit_io* io = nullptr;
    dit_time_weights tw{};
};

extern "C" {

const char* dit_host_last_error(void) { return g_err.c_str(); }
void dit_free_host(void* p) { std::free(p); }

int dit_read_raw_f(const char* path, float** data, int64_t* count, int64_t shape[8], int* ndim) {
    if (!path || !data || !count) return fail("dit_read_raw_f: null argument");
    std::vector<float> d;
    std::vector<int64_t> sh;
    if (read_raw_host(path, d, sh)) return -1;
    *data = copy_out(d);
    *count = (int64_t)d.size();
    if (ndim) *ndim = (int)sh.size();
    if (shape)
        for (size_t i = 0; i < sh.size(); i++) shape[i] = sh[i];
    return 0;
}

int dit_read_linear(const char* base, int has_bias, float** w, float** b, int* n_out, int* n_in) {
    if (!base || !w) return fail("dit_read_linear: null argument");
    HostLinear L;
    if (read_linear_host(base, has_bias != 0, L)) return -1;
    *w = copy_out(L.w);
    if (b) *b = has_bias ? copy_out(L.b) : nullptr;
    if (n_out) *n_out = L.n_out;
    if (n_in) *n_in = L.n_in;
    return 0;
}

int dit_read_win(const char* path, int txt_len, int64_t header[10], int32_t** slices, float** vid_freq,
                 int64_t* n_vid, float** txt_freq, int64_t* n_txt) {
    if (!path || !header || !slices || !vid_freq || !txt_freq || txt_len < 0)
        return fail("dit_read_win: bad argument");
    std::ifstream f(path, std::ios::binary);
    if (!f) return fail("cannot open %s", path);
    int64_t size;
    file_size(f, &size);
    f.read(reinterpret_cast<char*>(header), 80);
    const int64_t nwin = header[9];
    if (!f || nwin < 1 || nwin > 4096) return fail("%s: bad header (nwin %lld)", path, (long long)nwin);
    std::vector<int64_t> sl(nwin * 6);
    f.read(reinterpret_cast<char*>(sl.data()), nwin * 48);
    const int64_t nf = (size - 80 - nwin * 48) / 4;
    const int64_t nt = nwin * txt_len * 126;
    if (!f || nf < nt || (nf - nt) % 126)
        return fail("%s: %lld floats do not split into vid_freq and %lld txt_freq floats", path, (long long)nf,
                    (long long)nt);
    std::vector<float> all(nf);
    f.read(reinterpret_cast<char*>(all.data()), nf * 4);
    if (!f) return fail("%s: read error", path);
    std::vector<int32_t> s32(sl.begin(), sl.end());
    *slices = copy_out(s32);
    *vid_freq = copy_out(std::vector<float>(all.begin(), all.end() - nt));
    *txt_freq = copy_out(std::vector<float>(all.end() - nt, all.end()));
    if (n_vid) *n_vid = nf - nt;
    if (n_txt) *n_txt = nt;
    return 0;
}

void dit_model_destroy(awa_ctx* ctx, dit_model* m) {
    if (!m) return;
    DeviceGuard dg(ctx ? ctx->device : m->device);
    if (m->io) dit_io_destroy(ctx, m->io);
    for (void* p : m->allocs) (void)hipFree(p);
    delete m;
}

}  // extern "C"

namespace {

// The model's weights from src onto the device: linear weights as bf16, the
// SwiGLU pair packed, vectors and the timestep MLP as float32.
int load_model_from(awa_ctx* ctx, WeightSource& src, int n_layers, int mm_layers, dit_model** out,
                    awa_stream_t stream) {
    *out = nullptr;
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    dit_model* m = new dit_model();
    m->device = ctx->device;
    m->n_layers = n_layers;
    m->mm_layers = mm_layers;
    float* stage = nullptr;  // fp32 staging of one matrix on its way to bf16
    size_t stage_n = 0;
    int rc = AWA_OK;

    auto bad = [&](const char* fmt, const char* a, long x, long y) {
        set_err(ctx, fmt, a, x, y);
        rc = AWA_EARG;
    };
    auto dev_alloc = [&](size_t bytes) -> void* {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, bytes);
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: hipMalloc(%zu): %s", bytes, hipGetErrorString(e));
            rc = AWA_EHIP;
            return nullptr;
        }
        m->allocs.push_back(p);
        return p;
    };
    auto upload_f32 = [&](const std::vector<float>& v) -> float* {
        float* p = static_cast<float*>(dev_alloc(v.size() * 4));
        if (!p) return nullptr;
        hipError_t e = hipMemcpy(p, v.data(), v.size() * 4, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
            rc = AWA_EHIP;
            return nullptr;
        }
        return p;
    };
    auto upload_bf16 = [&](const std::vector<float>& v) -> uint16_t* {
        if (stage_n < v.size()) {
            if (stage) (void)hipFree(stage);
            stage = nullptr;
            stage_n = 0;
            if (hipMalloc(reinterpret_cast<void**>(&stage), v.size() * 4) != hipSuccess) {
                set_err(ctx, "dit_model_load: hipMalloc of the staging buffer failed");
                rc = AWA_EHIP;
                return nullptr;
            }
            stage_n = v.size();
        }
        uint16_t* p = static_cast<uint16_t*>(dev_alloc(v.size() * 2));
        if (!p) return nullptr;
        hipError_t e = hipMemcpy(stage, v.data(), v.size() * 4, hipMemcpyHostToDevice);
        if (e == hipSuccess) e = launch_cast_f32_bf16(stage, p, (int64_t)v.size(), s);
        if (e == hipSuccess) e = hipStreamSynchronize(s);  // the staging buffer is reused
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
            rc = AWA_EHIP;
            return nullptr;
        }
        return p;
    };
    auto linear = [&](const std::string& name, bool bias, int n_out, int n_in, HostLinear& L) {
        if (rc != AWA_OK) return false;
        if (src.linear(name, bias, L)) {
            set_err(ctx, "dit_model_load: %s", g_err.c_str());
            rc = AWA_EARG;
            return false;
        }
        if ((n_out > 0 && L.n_out != n_out) || (n_in > 0 && L.n_in != n_in)) {
            bad("dit_model_load: %s is %ld x %ld", name.c_str(), L.n_out, L.n_in);
            return false;
        }
        return true;
    };
    auto vec = [&](const std::string& name, size_t n) -> float* {
        if (rc != AWA_OK) return nullptr;
        std::vector<float> v;
        if (src.vec(name, v)) {
            set_err(ctx, "dit_model_load: %s", g_err.c_str());
            rc = AWA_EARG;
            return nullptr;
        }
        if (v.size() != n) {
            bad("dit_model_load: %s holds %ld floats, expected %ld", name.c_str(), (long)v.size(), (long)n);
            return nullptr;
        }
        return upload_f32(v);
    };

    // input / output layers and the timestep MLP
    HostLinear L;
    dit_io_weights iw{};
    if (linear("vid_in_proj", true, DIM, 132, L)) { iw.vid_in_w = upload_bf16(L.w); iw.vid_in_b = upload_f32(L.b); }
    if (linear("txt_in", true, DIM, 5120, L)) { iw.txt_in_w = upload_bf16(L.w); iw.txt_in_b = upload_f32(L.b); }
    if (linear("vid_out_proj", true, 64, DIM, L)) { iw.vid_out_w = upload_bf16(L.w); iw.vid_out_b = upload_f32(L.b); }
    iw.out_norm_w = vec("vid_out_norm_w", DIM);
    iw.out_ada_shift = vec("vid_out_ada_shift", DIM);
    iw.out_ada_scale = vec("vid_out_ada_scale", DIM);
    if (linear("emb_proj_in", true, DIM, 256, L)) { m->tw.w_in = upload_f32(L.w); m->tw.b_in = upload_f32(L.b); }
    if (linear("emb_proj_hid", true, DIM, DIM, L)) { m->tw.w_hid = upload_f32(L.w); m->tw.b_hid = upload_f32(L.b); }
    if (linear("emb_proj_out", true, DIT_EMB, DIM, L)) { m->tw.w_out = upload_f32(L.w); m->tw.b_out = upload_f32(L.b); }
    if (rc == AWA_OK) rc = dit_io_create(ctx, &iw, &m->io, stream);

    // layers: dual branches below mm_layers, one shared branch above
    auto branch = [&](const std::string& b, dit_branch& br) {
        HostLinear qkv, o, mi, mg, mo;
        if (linear(b + "_qkv", false, QKV, DIM, qkv)) br.qkv_w = upload_bf16(qkv.w);
        if (linear(b + "_out", true, DIM, DIM, o)) { br.out_w = upload_bf16(o.w); br.out_b = upload_f32(o.b); }
        if (linear(b + "_mlp_in", false, m->mlp > 0 ? m->mlp : 0, DIM, mi) &&
            linear(b + "_mlp_g", false, mi.n_out, DIM, mg) && linear(b + "_mlp_out", false, DIM, mi.n_out, mo)) {
            if (mi.n_out % 128) {
                bad("dit_model_load: %s MLP width %ld (%ld) is not a multiple of 128", b.c_str(), mi.n_out, 0);
            } else {
                m->mlp = mi.n_out;
                uint16_t* win = upload_bf16(mi.w);
                uint16_t* wg = upload_bf16(mg.w);
                uint16_t* cat = static_cast<uint16_t*>(dev_alloc((size_t)2 * m->mlp * DIM * 2));
                if (rc == AWA_OK && win && wg && cat) {
                    hipError_t e = launch_pack_mlp(win, wg, m->mlp, cat, s);
                    if (e != hipSuccess) {
                        set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
                        rc = AWA_EHIP;
                    }
                }
                br.mlp_w = cat;
                br.mlp_out_w = upload_bf16(mo.w);
            }
        }
        br.nq = vec(b + "_nq", 128);
        br.nk = vec(b + "_nk", 128);
        br.attn_shift = vec(b + "_attn_shift", DIM);
        br.attn_scale = vec(b + "_attn_scale", DIM);
        br.attn_gate = vec(b + "_attn_gate", DIM);
        br.mlp_shift = vec(b + "_mlp_shift", DIM);
        br.mlp_scale = vec(b + "_mlp_scale", DIM);
        br.mlp_gate = vec(b + "_mlp_gate", DIM);
    };
    m->vb.resize(n_layers);
    m->tb.resize(n_layers);
    for (int i = 0; i < n_layers && rc == AWA_OK; i++) {
        const std::string p = "b" + std::to_string(i);
        if (i < mm_layers) {
            branch(p + "_vid", m->vb[i]);
            branch(p + "_txt", m->tb[i]);
        } else {
            branch(p + "_all", m->vb[i]);
            m->tb[i] = m->vb[i];
        }
    }
    if (rc == AWA_OK) {
        hipError_t e = hipStreamSynchronize(s);
        if (e != hipSuccess) {
            set_err(ctx, "dit_model_load: %s", hipGetErrorString(e));
            rc = AWA_EHIP;
        }
    }
    if (stage) (void)hipFree(stage);
    if (rc != AWA_OK) {
        dit_model_destroy(ctx, m);
        return rc;
    }
    *out = m;
    return AWA_OK;
}

}  // namespace

extern "C" {

int dit_model_load(awa_ctx* ctx, const char* dir, int n_layers, int mm_layers, dit_model** out,
                   awa_stream_t stream) {
    if (!ctx || !dir || !out || n_layers < 0 || mm_layers < 0 || mm_layers > n_layers) {
        set_err(ctx, "dit_model_load: bad argument (n_layers=%d mm_layers=%d)", n_layers, mm_layers);
        return AWA_EARG;
    }
    DirSource src(dir);
    return load_model_from(ctx, src, n_layers, mm_layers, out, stream);
}

int dit_model_load_graph(awa_ctx* ctx, const char* param, const char* bin, const char* dir, int mm_layers,
                         dit_model** out, awa_stream_t stream) {
    if (!ctx || !param || !bin || !out) {
        set_err(ctx, "dit_model_load_graph: null argument");
        return AWA_EARG;
    }
    *out = nullptr;
    GraphSource src;
    std::unique_ptr<DirSource> d(dir ? new DirSource(dir) : nullptr);
    src.dir = d.get();
    if (index_graph(param, bin, mm_layers, src.G) || src.open()) {
        set_err(ctx, "dit_model_load_graph: %s", g_err.c_str());
        return AWA_EARG;
    }
    return load_model_from(ctx, src, src.G.n_layers, src.G.mm_layers, out, stream);
}

int dit_graph_file_info(const char* param, const char* bin, int mm_layers, int* n_layers, int* mm_out,
                        int* n_weights) {
    if (!param || !bin) return fail("dit_graph_file_info: null argument");
    GraphIndex G;
    if (index_graph(param, bin, mm_layers, G)) return -1;
    if (n_layers) *n_layers = G.n_layers;
    if (mm_out) *mm_out = G.mm_layers;
    if (n_weights) *n_weights = (int)G.w.size();
    return 0;
}

int dit_read_graph_weight(const char* param, const char* bin, int mm_layers, const char* name, float** w,
                          float** b, int* n_out, int* n_in) {
    if (!param || !bin || !name || !w) return fail("dit_read_graph_weight: null argument");
    GraphSource src;
    if (index_graph(param, bin, mm_layers, src.G) || src.open()) return -1;
    const GraphBlob* g = src.find(name);
    if (!g) return src.missing(name);
    if (g->kind == GraphBlob::LINEAR) {
        HostLinear L;
        if (src.linear(name, g->bias, L)) return -1;
        *w = copy_out(L.w);
        if (b) *b = g->bias ? copy_out(L.b) : nullptr;
        if (n_out) *n_out = L.n_out;
        if (n_in) *n_in = L.n_in;
    } else {
        std::vector<float> v;
        if (src.vec(name, v)) return -1;
        *w = copy_out(v);
        if (b) *b = nullptr;
        if (n_out) *n_out = (int)v.size();
        if (n_in) *n_in = 0;
    }
    return 0;
}

int dit_model_info(const dit_model* m, int* n_layers, int* mm_layers, int* mlp) {
    if (!m) return AWA_EARG;
    if (n_layers) *n_layers = m->n_layers;
    if (mm_layers) *mm_layers = m->mm_layers;
    if (mlp) *mlp = m->mlp;
    return AWA_OK;
}

int dit_model_forward_grid(awa_ctx* ctx, const dit_model* m, const awa_geom* g_even, const awa_geom* g_odd,
                           int last_txt_vid_only, float eps, float t, const float* d_grid, int T, int H, int W,
                           const float* d_txt, int TXT, float* d_x, float* d_out, awa_stream_t stream) {
    if (!ctx || !m) {
        set_err(ctx, "dit_model_forward_grid: null argument");
        return AWA_EARG;
    }
    std::vector<const dit_branch*> vb(m->n_layers), tb(m->n_layers);
    for (int i = 0; i < m->n_layers; i++) {
        vb[i] = &m->vb[i];
        tb[i] = (i < m->mm_layers) ? &m->tb[i] : &m->vb[i];  // shared layers: the same branch
    }
    return dit_forward_grid(ctx, m->io, &m->tw, vb.data(), tb.data(), m->n_layers, g_even, g_odd, m->mlp,
                            last_txt_vid_only, eps, t, d_grid, T, H, W, d_txt, TXT, d_x, d_out, stream);
}

struct dit_graph {
    int device = 0;
    awa_ctx* priv = nullptr;  // owns the scratch baked into the graph
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
};

void dit_graph_destroy(dit_graph* g) {
    if (!g) return;
    DeviceGuard dg(g->device);
    if (g->exec) (void)hipGraphExecDestroy(g->exec);
    if (g->graph) (void)hipGraphDestroy(g->graph);
    if (g->priv) awa_destroy(g->priv);
    delete g;
}

int dit_graph_create(awa_ctx* ctx, const dit_model* m, const awa_geom* g_even, const awa_geom* g_odd,
                     int last_txt_vid_only, float eps, float t, const float* d_grid, int T, int H, int W,
                     const float* d_txt, int TXT, float* d_x, float* d_out, awa_stream_t stream, dit_graph** out) {
    if (!ctx || !m || !out || !stream) {
        set_err(ctx, "dit_graph_create: null argument (capture needs a created stream, not the null stream)");
        return AWA_EARG;
    }
    *out = nullptr;
    DeviceGuard dg(ctx->device);
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    dit_graph* g = new dit_graph();
    g->device = ctx->device;
    int rc = awa_create(&g->priv, ctx->device);
    if (rc != AWA_OK) {
        set_err(ctx, "dit_graph_create: private context: %s", g->priv ? awa_last_error(g->priv) : "awa_create failed");
        dit_graph_destroy(g);
        return rc;
    }
    // eager run: sizes the private context's buffers (no allocation may happen
    // while capturing) and checks every argument
    rc = dit_model_forward_grid(g->priv, m, g_even, g_odd, last_txt_vid_only, eps, t, d_grid, T, H, W, d_txt, TXT,
                                d_x, d_out, stream);
    hipError_t e = rc == AWA_OK ? hipStreamSynchronize(s) : hipSuccess;
    if (rc == AWA_OK && e == hipSuccess) {
        e = hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal);
        if (e == hipSuccess) {
            rc = dit_model_forward_grid(g->priv, m, g_even, g_odd, last_txt_vid_only, eps, t, d_grid, T, H, W,
                                        d_txt, TXT, d_x, d_out, stream);
            hipError_t e2 = hipStreamEndCapture(s, &g->graph);
            if (rc == AWA_OK) e = e2;
        }
        if (rc == AWA_OK && e == hipSuccess) e = hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0);
    }
    if (rc != AWA_OK || e != hipSuccess) {
        if (rc != AWA_OK) set_err(ctx, "dit_graph_create: %s", awa_last_error(g->priv));
        else set_err(ctx, "dit_graph_create: %s", hipGetErrorString(e));
        dit_graph_destroy(g);
        return rc != AWA_OK ? rc : AWA_EHIP;
    }
    *out = g;
    return AWA_OK;
}

int dit_graph_launch(awa_ctx* ctx, dit_graph* g, awa_stream_t stream) {
    if (!ctx || !g) {
        set_err(ctx, "dit_graph_launch: null argument");
        return AWA_EARG;
    }
    DeviceGuard dg(g->device);
    hipError_t e = hipGraphLaunch(g->exec, reinterpret_cast<hipStream_t>(stream));
    if (e != hipSuccess) {
        set_err(ctx, "dit_graph_launch: %s", hipGetErrorString(e));
        return AWA_EHIP;
    }
    return AWA_OK;
}

}  // extern "C"
