// dit_files.cpp — readers of the reference's on-disk formats: read_raw_f
// vectors (dit_vk.cpp:38-45), ncnn InnerProduct .param/.bin pairs
// (verify_dit.cpp:80-102), window files (load_win, dit_vk.cpp:74-93) and the
// merged whole-model graph (export_dit_graph.py:47-258).  Host-only C++.
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstdint>
#include <exception>
#include <sstream>

#include "dit_files.hpp"
#include "dit_model.h"

namespace dit_files {

namespace {

thread_local std::string g_err;

}  // namespace

int fail(const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return -1;
}

const std::string& last_error() { return g_err; }

namespace {

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


// Bytes of an ncnn "type 0" blob of n values after its 4-byte tag: fp16
// values padded to a multiple of 4 bytes, or fp32 (ModelBinFromDataReader).
bool tagged_bytes(uint32_t tag, int64_t n, int64_t* bytes) {
    if (tag == TAG_FP16) *bytes = (2 * n + 3) / 4 * 4;
    else if (tag == TAG_FP32) *bytes = 4 * n;
    else return false;
    return true;
}

}  // namespace

// n values of a "type 0" blob at byte off of f (the tag first).
int read_tagged_at(std::ifstream& f, int64_t size, int64_t off, int64_t n, const std::string& what,
                   std::vector<float>& v) {
    if (n < 0 || off < 0 || off > size - 4 || n > (size - off - 4) / 2)
        return fail("%s: %lld values at byte %lld exceed the %lld-byte file", what.c_str(), (long long)n,
                    (long long)off, (long long)size);
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
    if (numout > INT32_MAX || total / numout > INT32_MAX)
        return fail("%s.param: InnerProduct 0=%ld 2=%ld out of range", base.c_str(), numout, total);
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

namespace {

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

}  // namespace

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
        if (n <= 0) return fail("%s: layer %s: a blob of %lld values", param.c_str(), layer.c_str(), (long long)n);
        // at least 2 bytes per value (fp16) after the 4-byte tag: bound n
        // before any size arithmetic
        if (off > G.bin_size - 4 || n > (G.bin_size - off - 4) / 2)
            return fail("%s: layer %s: %lld values exceed the %lld bytes of %s", param.c_str(), layer.c_str(),
                        (long long)n, (long long)G.bin_size, bin.c_str());
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
            if (nout <= 0 || total <= 0 || total % nout || nout > INT32_MAX || total / nout > INT32_MAX)
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
            if (bias && nout > (G.bin_size - off) / 4)
                return fail("%s: %lld bytes end inside the bias of %s", bin.c_str(), (long long)G.bin_size,
                            L.name.c_str());
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
            if (nl < 0 || nl > 4096 || dim <= 0 || dim > INT32_MAX)
                return fail("%s: AdaCompose %s: 1=%ld 3=%ld", param.c_str(), L.name.c_str(), nl, dim);
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
                if (n <= 0 || n > (G.bin_size - off) / 4)
                    return fail("%s: RMSNorm %s: 0=%ld values past the end of %s", param.c_str(), L.name.c_str(), n,
                                bin.c_str());
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

}  // namespace dit_files

using namespace dit_files;

namespace {

// Runs a reader body; an exception (bad_alloc of a huge but well-formed
// request, a stream error) becomes a -1 return with its message, never a
// throw across the C ABI.
template <typename F>
int guarded(const char* who, F&& body) {
    try {
        return body();
    } catch (const std::exception& e) {
        return fail("%s: %s", who, e.what());
    } catch (...) {
        return fail("%s: unknown exception", who);
    }
}

}  // namespace

extern "C" {

const char* dit_host_last_error(void) { return last_error().c_str(); }
void dit_free_host(void* p) { std::free(p); }

int dit_read_raw_f(const char* path, float** data, int64_t* count, int64_t shape[8], int* ndim) {
    return guarded("dit_read_raw_f", [&]() -> int {
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
    });
}

int dit_read_linear(const char* base, int has_bias, float** w, float** b, int* n_out, int* n_in) {
    return guarded("dit_read_linear", [&]() -> int {
        if (!base || !w) return fail("dit_read_linear: null argument");
        HostLinear L;
        if (read_linear_host(base, has_bias != 0, L)) return -1;
        *w = copy_out(L.w);
        if (b) *b = has_bias ? copy_out(L.b) : nullptr;
        if (n_out) *n_out = L.n_out;
        if (n_in) *n_in = L.n_in;
        return 0;
    });
}

int dit_read_win(const char* path, int txt_len, int64_t header[10], int32_t** slices, float** vid_freq,
                 int64_t* n_vid, float** txt_freq, int64_t* n_txt) {
    return guarded("dit_read_win", [&]() -> int {
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
    });
}

int dit_graph_file_info(const char* param, const char* bin, int mm_layers, int* n_layers, int* mm_out,
                        int* n_weights) {
    return guarded("dit_graph_file_info", [&]() -> int {
        if (!param || !bin) return fail("dit_graph_file_info: null argument");
        GraphIndex G;
        if (index_graph(param, bin, mm_layers, G)) return -1;
        if (n_layers) *n_layers = G.n_layers;
        if (mm_out) *mm_out = G.mm_layers;
        if (n_weights) *n_weights = (int)G.w.size();
        return 0;
    });
}

int dit_read_graph_weight(const char* param, const char* bin, int mm_layers, const char* name, float** w,
                          float** b, int* n_out, int* n_in) {
    return guarded("dit_read_graph_weight", [&]() -> int {
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
    });
}

}  // extern "C"
