// hx_checkpoint.hip -- host-side EXL3 checkpoint loading behind the C ABI: safetensors shard headers,
// the reference's per-layer expert validation and slab layout, and the load of a layer's routed
// experts into one device slab (pinned staging, reader threads, async copies).  No kernels.
//
// Reference behaviour followed:
//   src/core/safetensors.hpp:1-53, safetensors.cpp:35-120  shard set: the index file's weight map (or
//       every *.safetensors of the directory, by name), 8-byte little-endian header length, JSON map
//       {name: {dtype, shape, data_offsets}}, data region after the header, lookup by name;
//   src/core/expert_layout.cpp:6-55  expert validation (names, trellis shape (in/16, out/16, S) with
//       S % 16 == 0 and 32 <= S <= 128, suh [in], svh [out], mul1 scalar 0x83DCD12D, exact byte
//       sizes and dtypes, one bit width per projection across a layer's experts) and the slab layout
//       (pieces trellis, suh, svh, mul1 per projection, each projection 64-byte aligned);
//   src/core/model.cpp:254-340  the layer's experts copied into their slab.
// One difference: the reference refuses 7-bit experts because its fused kernels are not built for
// them; every width 1..8 (within the shape rule) is accepted here.
#include <hip/hip_runtime.h>

#include <errno.h>
#include <fcntl.h>
#include <stdio.h>
#include <string.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <dirent.h>
#include <map>
#include <memory>
#include <mutex>
#include <stdexcept>
#include <string>
#include <thread>
#include <vector>

#include "../../include/hx/exl3.h"

namespace hx {
void set_error(const char* msg);
}

namespace {

// ------------------------------------------------------------------ minimal JSON (safetensors headers)

struct Json {
    enum Kind { NUL, BOOL, NUM, STR, ARR, OBJ } kind = NUL;
    double num = 0;
    long long inum = 0;
    bool is_int = false;
    std::string str;
    std::vector<Json> arr;
    std::vector<std::pair<std::string, Json>> obj;
    const Json* get(const std::string& k) const
    {
        for (const auto& kv : obj)
            if (kv.first == k) return &kv.second;
        return nullptr;
    }
};

struct JsonParser {
    const char* p;
    const char* end;
    [[noreturn]] void bad(const char* what) { throw std::runtime_error(std::string("bad JSON header: ") + what); }
    void ws()
    {
        while (p < end && (*p == ' ' || *p == '\n' || *p == '\r' || *p == '\t')) ++p;
    }
    bool lit(const char* s)
    {
        const size_t n = strlen(s);
        if ((size_t)(end - p) >= n && memcmp(p, s, n) == 0) {
            p += n;
            return true;
        }
        return false;
    }
    std::string string()
    {
        if (p >= end || *p != '"') bad("expected a string");
        ++p;
        std::string s;
        while (p < end && *p != '"') {
            if (*p == '\\') {
                ++p;
                if (p >= end) bad("unterminated escape");
                switch (*p) {
                    case '"': s += '"'; break;
                    case '\\': s += '\\'; break;
                    case '/': s += '/'; break;
                    case 'b': s += '\b'; break;
                    case 'f': s += '\f'; break;
                    case 'n': s += '\n'; break;
                    case 'r': s += '\r'; break;
                    case 't': s += '\t'; break;
                    case 'u': {  // kept as its escape: tensor names here are ASCII
                        if (end - p < 5) bad("short \\u escape");
                        s += "\\u";
                        s.append(p + 1, 4);
                        p += 4;
                        break;
                    }
                    default: bad("unknown escape");
                }
                ++p;
            } else {
                s += *p++;
            }
        }
        if (p >= end) bad("unterminated string");
        ++p;
        return s;
    }
    Json value(int depth)
    {
        if (depth > 32) bad("nested too deeply");
        ws();
        if (p >= end) bad("unexpected end");
        Json v;
        if (*p == '{') {
            v.kind = Json::OBJ;
            ++p;
            ws();
            if (p < end && *p == '}') {
                ++p;
                return v;
            }
            for (;;) {
                ws();
                std::string k = string();
                ws();
                if (p >= end || *p != ':') bad("expected ':'");
                ++p;
                v.obj.emplace_back(std::move(k), value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == '}') {
                    ++p;
                    return v;
                }
                bad("expected ',' or '}'");
            }
        }
        if (*p == '[') {
            v.kind = Json::ARR;
            ++p;
            ws();
            if (p < end && *p == ']') {
                ++p;
                return v;
            }
            for (;;) {
                v.arr.push_back(value(depth + 1));
                ws();
                if (p < end && *p == ',') {
                    ++p;
                    continue;
                }
                if (p < end && *p == ']') {
                    ++p;
                    return v;
                }
                bad("expected ',' or ']'");
            }
        }
        if (*p == '"') {
            v.kind = Json::STR;
            v.str = string();
            return v;
        }
        if (lit("true")) {
            v.kind = Json::BOOL;
            v.num = 1;
            return v;
        }
        if (lit("false")) {
            v.kind = Json::BOOL;
            return v;
        }
        if (lit("null")) return v;
        // number (RFC 8259 grammar): integers exactly (offsets exceed 2^53 only past 8 PB), others as double
        const char* s = p;
        if (p < end && *p == '-') ++p;
        const char* digits = p;
        while (p < end && *p >= '0' && *p <= '9') ++p;
        if (p == digits) bad("unexpected character");
        bool integral = true;
        if (p < end && *p == '.') {
            integral = false;
            const char* f = ++p;
            while (p < end && *p >= '0' && *p <= '9') ++p;
            if (p == f) bad("malformed number");
        }
        if (p < end && (*p == 'e' || *p == 'E')) {
            integral = false;
            ++p;
            if (p < end && (*p == '-' || *p == '+')) ++p;
            const char* x = p;
            while (p < end && *p >= '0' && *p <= '9') ++p;
            if (p == x) bad("malformed number");
        }
        const std::string t(s, p);
        v.kind = Json::NUM;
        char* stop = nullptr;
        v.num = strtod(t.c_str(), &stop);
        if (stop != t.c_str() + t.size()) bad("malformed number");
        v.is_int = integral;
        if (integral) {
            errno = 0;
            v.inum = strtoll(t.c_str(), &stop, 10);
            if (errno == ERANGE || stop != t.c_str() + t.size()) bad("integer out of range");
        }
        return v;
    }
};

// ------------------------------------------------------------------ shard set

enum Dt { F16, BF16, F32, F64, I32, I16, I8, U8, BOOL_, I64, UNKNOWN };

Dt dtype_of(const std::string& s)
{
    static const std::map<std::string, Dt> m = {{"F16", F16}, {"BF16", BF16}, {"F32", F32}, {"F64", F64},
                                                {"I32", I32}, {"I16", I16}, {"I8", I8},     {"U8", U8},
                                                {"BOOL", BOOL_}, {"I64", I64}};
    auto it = m.find(s);
    return it == m.end() ? UNKNOWN : it->second;
}

uint64_t dtype_size(Dt d)
{
    switch (d) {
        case F64: case I64: return 8;
        case F32: case I32: return 4;
        case F16: case BF16: case I16: return 2;
        case I8: case U8: case BOOL_: return 1;
        default: return 0;
    }
}

struct Tensor {
    std::string name;
    Dt dtype = UNKNOWN;
    std::vector<int64_t> shape;
    int shard = -1;
    uint64_t offset = 0;  // absolute byte offset in the shard file
    uint64_t bytes = 0;
};

}  // namespace

struct hx_ckpt {
    std::vector<std::string> paths;
    std::vector<int> fds;
    std::map<std::string, Tensor> tensors;
    ~hx_ckpt()
    {
        for (int fd : fds)
            if (fd >= 0) close(fd);
    }
    const Tensor* find(const std::string& n) const
    {
        auto it = tensors.find(n);
        return it == tensors.end() ? nullptr : &it->second;
    }
    void read(const Tensor& t, void* dst, uint64_t off = 0, uint64_t n = ~0ull) const
    {
        if (n == ~0ull) n = t.bytes - off;
        char* d = static_cast<char*>(dst);
        uint64_t done = 0;
        while (done < n) {
            const ssize_t r = pread(fds[t.shard], d + done, n - done, (off_t)(t.offset + off + done));
            if (r <= 0) throw std::runtime_error("short read of " + t.name);
            done += (uint64_t)r;
        }
    }
};

namespace {

std::vector<std::string> shard_paths(const std::string& dir)
{
    std::vector<std::string> out;
    // the index file's weight map names the shards (safetensors.cpp:37-49)
    const std::string idx = dir + "/model.safetensors.index.json";
    FILE* f = fopen(idx.c_str(), "rb");
    if (f) {
        std::string text;
        char buf[65536];
        size_t n;
        while ((n = fread(buf, 1, sizeof(buf), f)) > 0) text.append(buf, n);
        fclose(f);
        std::string bad_shard;
        try {
            JsonParser jp{text.data(), text.data() + text.size()};
            const Json j = jp.value(0);
            if (const Json* wm = j.get("weight_map")) {
                std::vector<std::string> files;
                for (const auto& kv : wm->obj)
                    if (kv.second.kind == Json::STR) files.push_back(kv.second.str);
                std::sort(files.begin(), files.end());
                files.erase(std::unique(files.begin(), files.end()), files.end());
                for (const auto& fn : files) {
                    // a shard is a file of the checkpoint directory itself: no separators, no parent
                    if (fn.empty() || fn.find('/') != std::string::npos || fn.find("..") != std::string::npos)
                        bad_shard = fn;
                    out.push_back(dir + "/" + fn);
                }
            }
        } catch (const std::exception&) {
            out.clear();  // an unreadable index falls back to the directory scan, as the reference does
        }
        if (!bad_shard.empty())
            throw std::runtime_error("index names a shard outside the checkpoint directory: " + bad_shard);
    }
    if (out.empty()) {
        DIR* d = opendir(dir.c_str());
        if (!d) throw std::runtime_error("cannot open directory " + dir);
        while (dirent* e = readdir(d)) {
            const std::string nm = e->d_name;
            if (nm.size() > 12 && nm.compare(nm.size() - 12, 12, ".safetensors") == 0) out.push_back(dir + "/" + nm);
        }
        closedir(d);
        std::sort(out.begin(), out.end());
    }
    if (out.empty()) throw std::runtime_error("no *.safetensors shard in " + dir);
    return out;
}

void parse_shard(hx_ckpt& c, const std::string& path)
{
    const int fd = open(path.c_str(), O_RDONLY | O_CLOEXEC);
    if (fd < 0) throw std::runtime_error("cannot open shard " + path);
    const int si = (int)c.paths.size();
    c.paths.push_back(path);
    c.fds.push_back(fd);
    const off_t size = lseek(fd, 0, SEEK_END);
    uint64_t hlen = 0;
    if (pread(fd, &hlen, 8, 0) != 8) throw std::runtime_error("truncated header in " + path);
    if (hlen < 2 || hlen > 512ull * 1024 * 1024 || (off_t)(8 + hlen) > size)
        throw std::runtime_error("bad header length in " + path);
    std::string hdr(hlen, '\0');
    if (pread(fd, hdr.data(), hlen, 8) != (ssize_t)hlen) throw std::runtime_error("truncated header in " + path);
    JsonParser jp{hdr.data(), hdr.data() + hdr.size()};
    const Json j = jp.value(0);
    if (j.kind != Json::OBJ) throw std::runtime_error("header of " + path + " is not an object");
    const uint64_t start = 8 + hlen;
    for (const auto& kv : j.obj) {
        if (kv.first == "__metadata__") continue;
        const Json& v = kv.second;
        const Json* dt = v.get("dtype");
        const Json* sh = v.get("shape");
        const Json* of = v.get("data_offsets");
        if (!dt || dt->kind != Json::STR || !sh || sh->kind != Json::ARR || !of || of->kind != Json::ARR ||
            of->arr.size() != 2 || !of->arr[0].is_int || !of->arr[1].is_int)
            throw std::runtime_error("malformed header entry " + kv.first);
        Tensor t;
        t.name = kv.first;
        t.dtype = dtype_of(dt->str);
        if (t.dtype == UNKNOWN) throw std::runtime_error(kv.first + ": unsupported dtype " + dt->str);
        uint64_t elems = 1;
        for (const Json& d : sh->arr) {
            if (!d.is_int || d.inum < 0) throw std::runtime_error(kv.first + ": bad shape");
            t.shape.push_back(d.inum);
            elems *= (uint64_t)d.inum;
        }
        const long long b = of->arr[0].inum, e = of->arr[1].inum;
        t.shard = si;
        t.offset = start + (uint64_t)b;
        t.bytes = (uint64_t)(e - b);
        if (b < 0 || e < b || t.bytes != elems * dtype_size(t.dtype) || (off_t)(start + (uint64_t)e) > size)
            throw std::runtime_error(kv.first + ": data range does not match its shape and dtype");
        if (c.tensors.count(t.name)) throw std::runtime_error(t.name + ": present in two shards");
        c.tensors.emplace(t.name, std::move(t));
    }
}

int fail(int code, const std::string& msg)
{
    hx::set_error(msg.c_str());
    return code;
}

}  // namespace

// ------------------------------------------------------------------ C ABI

namespace {

// ---- routed-expert tensors of a layer
//
// Each projection of an expert is four tensors named model.language_model.layers.<l>.mlp.experts.<e>.
// <proj>.<kind>; their form follows from the projection's in/out features and bit width.
enum PieceKind { TRELLIS = 0, SUH = 1, SVH = 2, MUL1 = 3 };
struct PieceSpec {
    const char* leaf;
    Dt dtype;
};
const PieceSpec kPieces[4] = {{"trellis", I16}, {"suh", F16}, {"svh", F16}, {"mul1", I32}};
const char* const kProjNames[3] = {"gate_proj", "up_proj", "down_proj"};
constexpr uint32_t kMul1Codebook = 0x83DCD12Du;

std::string expert_tensor_name(int layer, int expert, int proj, PieceKind k)
{
    char buf[160];
    snprintf(buf, sizeof(buf), "model.language_model.layers.%d.mlp.experts.%d.%s.%s", layer, expert,
             kProjNames[proj], kPieces[k].leaf);
    return buf;
}

// Shapes and byte sizes of the four tensors of a projection: gate/up map hidden -> intermediate,
// down maps intermediate -> hidden.
struct ProjForm {
    int in, out;
    std::vector<int64_t> shape[4];
    uint64_t bytes[4];
};
ProjForm proj_form(int proj, int hidden, int intermediate, int bits)
{
    ProjForm f;
    f.in = proj == 2 ? intermediate : hidden;
    f.out = proj == 2 ? hidden : intermediate;
    f.shape[TRELLIS] = {f.in / 16, f.out / 16, 16 * bits};
    f.shape[SUH] = {f.in};
    f.shape[SVH] = {f.out};
    f.shape[MUL1] = {};
    f.bytes[TRELLIS] = (uint64_t)f.in * f.out * bits / 8;
    f.bytes[SUH] = 2ull * f.in;
    f.bytes[SVH] = 2ull * f.out;
    f.bytes[MUL1] = 4;
    return f;
}

// Bit width of a trellis tensor of the projection's tile grid (third dimension 16 * bits, bits 2..8),
// or -1 when it is not one.
int trellis_width(const Tensor& t, const ProjForm& f)
{
    if (t.shape.size() != 3 || t.shape[0] != f.in / 16 || t.shape[1] != f.out / 16) return -1;
    const int64_t d = t.shape[2];
    return (d % 16 == 0 && d >= 32 && d <= 128) ? (int)(d / 16) : -1;
}

uint64_t round_up64(uint64_t v) { return (v + 63) / 64 * 64; }

}  // namespace

extern "C" {

int hx_ckpt_open(const char* dir, hx_ckpt** out)
{
    if (!dir || !out) return fail(HX_ERR_INVALID, "hx_ckpt_open: null argument");
    *out = nullptr;
    try {
        std::unique_ptr<hx_ckpt> c(new hx_ckpt());
        for (const auto& p : shard_paths(dir)) parse_shard(*c, p);
        *out = c.release();
        return 0;
    } catch (const std::exception& e) {
        return fail(HX_ERR_INVALID, std::string("hx_ckpt_open: ") + e.what());
    }
}

void hx_ckpt_close(hx_ckpt* c) { delete c; }

int hx_ckpt_tensor_count(const hx_ckpt* c) { return c ? (int)c->tensors.size() : HX_ERR_INVALID; }

int hx_ckpt_tensor_info(const hx_ckpt* c, const char* name, int* dtype, int64_t* shape, int max_dims, int* ndim,
                        uint64_t* bytes)
{
    if (!c || !name) return fail(HX_ERR_INVALID, "hx_ckpt_tensor_info: null argument");
    const Tensor* t = c->find(name);
    if (!t) return fail(HX_ERR_INVALID, std::string("hx_ckpt_tensor_info: no tensor ") + name);
    if (dtype) *dtype = (int)t->dtype;
    if (ndim) *ndim = (int)t->shape.size();
    if (shape)
        for (int i = 0; i < max_dims && i < (int)t->shape.size(); ++i) shape[i] = t->shape[i];
    if (bytes) *bytes = t->bytes;
    return 0;
}

int hx_ckpt_read(const hx_ckpt* c, const char* name, void* host_dst, uint64_t bytes)
{
    if (!c || !name || (!host_dst && bytes)) return fail(HX_ERR_INVALID, "hx_ckpt_read: null argument");
    const Tensor* t = c->find(name);
    if (!t) return fail(HX_ERR_INVALID, std::string("hx_ckpt_read: no tensor ") + name);
    if (bytes != t->bytes) return fail(HX_ERR_INVALID, std::string("hx_ckpt_read: size mismatch for ") + name);
    try {
        c->read(*t, host_dst);
    } catch (const std::exception& e) {
        return fail(HX_ERR_INVALID, std::string("hx_ckpt_read: ") + e.what());
    }
    return 0;
}


int hx_ckpt_expert_layout(const hx_ckpt* c, int layer, int experts, int hidden, int intermediate,
                          hx_expert_layout* out)
{
    if (!c || !out || experts < 1 || hidden < 16 || intermediate < 16 || hidden % 16 || intermediate % 16)
        return fail(HX_ERR_INVALID, "hx_ckpt_expert_layout: bad arguments");
    // The bit width of each projection is read off expert 0's trellis; every other tensor of every
    // expert must then have exactly the form that width implies (one width per projection, as the
    // slab has one stride).
    int bits[3];
    for (int p = 0; p < 3; ++p) {
        const ProjForm f0 = proj_form(p, hidden, intermediate, 0);
        const std::string tn = expert_tensor_name(layer, 0, p, TRELLIS);
        const Tensor* tr = c->find(tn);
        if (!tr) return fail(HX_ERR_INVALID, "hx_ckpt_expert_layout: no tensor " + tn);
        const int w = trellis_width(*tr, f0);
        if (w < 0)
            return fail(HX_ERR_INVALID, "hx_ckpt_expert_layout: " + tn + " is not a (" + std::to_string(f0.in / 16) +
                                            ", " + std::to_string(f0.out / 16) + ", 16*bits) trellis, bits 2..8");
        bits[p] = w;
    }
    for (int e = 0; e < experts; ++e)
        for (int p = 0; p < 3; ++p) {
            const ProjForm f = proj_form(p, hidden, intermediate, bits[p]);
            for (int k = 0; k < 4; ++k) {
                const std::string tn = expert_tensor_name(layer, e, p, (PieceKind)k);
                const Tensor* t = c->find(tn);
                if (!t) return fail(HX_ERR_INVALID, "hx_ckpt_expert_layout: no tensor " + tn);
                if (k == TRELLIS && e > 0 && trellis_width(*t, f) >= 0 && trellis_width(*t, f) != bits[p])
                    return fail(HX_ERR_INVALID, "hx_ckpt_expert_layout: " + tn + " has " +
                                                    std::to_string(trellis_width(*t, f)) + " bits, expert 0 has " +
                                                    std::to_string(bits[p]) + " (one width per projection)");
                const char* why = nullptr;
                if (t->dtype != kPieces[k].dtype) why = "dtype";
                else if (t->shape != f.shape[k]) why = "shape";
                else if (t->bytes != f.bytes[k]) why = "byte size";
                if (why)
                    return fail(HX_ERR_INVALID, std::string("hx_ckpt_expert_layout: ") + tn + ": unexpected " + why +
                                                    " for a " + std::to_string(f.in) + "->" + std::to_string(f.out) +
                                                    " projection at " + std::to_string(bits[p]) + " bits");
            }
            // codebook 2 is the only codebook of the fused expert kernels
            uint32_t mul = 0;
            const std::string mn = expert_tensor_name(layer, e, p, MUL1);
            try {
                c->read(*c->find(mn), &mul);
            } catch (const std::exception& ex) {
                return fail(HX_ERR_INVALID, "hx_ckpt_expert_layout: " + mn + ": " + ex.what());
            }
            if (mul != kMul1Codebook)
                return fail(HX_ERR_INVALID, "hx_ckpt_expert_layout: " + mn + " selects another codebook than mul1");
        }
    // Slab placement: the pieces in kind order, projection after projection, each projection's block
    // padded to the 64-byte alignment the loaders keep.
    hx_expert_layout L;
    memset(&L, 0, sizeof(L));
    uint64_t at = 0;
    for (int p = 0; p < 3; ++p) {
        const ProjForm f = proj_form(p, hidden, intermediate, bits[p]);
        for (int k = 0; k < 4; ++k) {
            L.off[4 * p + k] = at;
            L.piece[4 * p + k] = f.bytes[k];
            at += f.bytes[k];
        }
        at = round_up64(at);
        L.bits[p] = bits[p];
    }
    L.stride = at;
    *out = L;
    return 0;
}

int hx_ckpt_load_experts(const hx_ckpt* c, int layer, int experts, const hx_expert_layout* L, void* slab,
                         size_t slab_bytes, int readers, hx_stream_t stream)
{
    if (!c || !L || !slab || experts < 1) return fail(HX_ERR_INVALID, "hx_ckpt_load_experts: bad arguments");
    if ((uint64_t)experts * L->stride > slab_bytes)
        return fail(HX_ERR_WORKSPACE, "hx_ckpt_load_experts: slab smaller than experts * layout.stride");
    // the 12 tensors of every expert, found before anything is read
    std::vector<const Tensor*> t((size_t)experts * 12);
    for (int e = 0; e < experts; ++e)
        for (int q = 0; q < 12; ++q) {
            const std::string n = expert_tensor_name(layer, e, q / 4, (PieceKind)(q % 4));
            t[(size_t)e * 12 + q] = c->find(n);
            if (!t[(size_t)e * 12 + q] || t[(size_t)e * 12 + q]->bytes != L->piece[q])
                return fail(HX_ERR_INVALID, "hx_ckpt_load_experts: tensor missing or not as in the layout: " + n);
        }
    // two pinned staging buffers of whole experts; reader threads fill one while the other copies
    const uint64_t stride = L->stride;
    const int per = (int)std::max<uint64_t>(1, std::min<uint64_t>((uint64_t)experts, (128ull << 20) / stride));
    void* stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipStream_t st = (hipStream_t)stream;
    auto cleanup = [&]() {
        for (int b = 0; b < 2; ++b) {
            if (done[b]) {
                (void)hipEventSynchronize(done[b]);
                (void)hipEventDestroy(done[b]);
            }
            if (stage[b]) (void)hipHostFree(stage[b]);
        }
    };
    for (int b = 0; b < 2; ++b) {
        if (hipHostMalloc(&stage[b], (size_t)per * stride, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&done[b], hipEventDisableTiming) != hipSuccess) {
            cleanup();
            return fail(HX_ERR_HIP, "hx_ckpt_load_experts: pinned staging or event allocation failed");
        }
    }
    const int nthreads = std::max(1, std::min(readers > 0 ? readers : 8, 32));
    std::string err;
    std::mutex err_mu;
    int buf = 0;
    bool pending[2] = {false, false};
    for (int e0 = 0; e0 < experts; e0 += per, buf ^= 1) {
        const int n = std::min(per, experts - e0);
        if (pending[buf] && hipEventSynchronize(done[buf]) != hipSuccess) {
            cleanup();
            return fail(HX_ERR_HIP, "hx_ckpt_load_experts: copy failed");
        }
        // pieces of experts e0 .. e0+n-1 into stage[buf] at (e - e0) * stride + off[q]
        std::atomic<int> next(0);
        const int jobs = n * 12;
        auto work = [&]() {
            for (int j; (j = next.fetch_add(1)) < jobs;) {
                const int e = e0 + j / 12, q = j % 12;
                try {
                    c->read(*t[(size_t)e * 12 + q],
                            static_cast<char*>(stage[buf]) + (size_t)(e - e0) * stride + L->off[q]);
                } catch (const std::exception& ex) {
                    std::lock_guard<std::mutex> g(err_mu);
                    err = ex.what();
                }
            }
        };
        std::vector<std::thread> pool;
        for (int i = 1; i < nthreads; ++i) pool.emplace_back(work);
        work();
        for (auto& th : pool) th.join();
        if (!err.empty()) {
            cleanup();
            return fail(HX_ERR_INVALID, "hx_ckpt_load_experts: " + err);
        }
        if (hipMemcpyAsync(static_cast<char*>(slab) + (size_t)e0 * stride, stage[buf], (size_t)n * stride,
                           hipMemcpyHostToDevice, st) != hipSuccess ||
            hipEventRecord(done[buf], st) != hipSuccess) {
            cleanup();
            return fail(HX_ERR_HIP, "hx_ckpt_load_experts: copy failed");
        }
        pending[buf] = true;
    }
    cleanup();  // waits for both copies: the staging buffers are freed before returning
    return 0;
}

int hx_ckpt_expert_tables(const hx_expert_layout* L, const void* slab, int experts, void* table_storage,
                          hx_expert_tables* out, hx_stream_t stream)
{
    if (!L || !slab || !table_storage || !out || experts < 1)
        return fail(HX_ERR_INVALID, "hx_ckpt_expert_tables: bad arguments");
    // table k (gate/up/down x trellis/suh/svh) = piece 4 * (k / 3) + k % 3 of every expert
    std::vector<const void*> host((size_t)9 * experts);
    for (int k = 0; k < 9; ++k)
        for (int e = 0; e < experts; ++e)
            host[(size_t)k * experts + e] =
                static_cast<const char*>(slab) + (size_t)e * L->stride + L->off[4 * (k / 3) + k % 3];
    if (hipMemcpyAsync(table_storage, host.data(), host.size() * sizeof(void*), hipMemcpyHostToDevice,
                       (hipStream_t)stream) != hipSuccess ||
        hipStreamSynchronize((hipStream_t)stream) != hipSuccess)
        return fail(HX_ERR_HIP, "hx_ckpt_expert_tables: copy failed");
    const void* const* d = static_cast<const void* const*>(table_storage);
    hx_expert_tables t;
    t.gate_trellis = d + 0 * experts;
    t.gate_suh = d + 1 * experts;
    t.gate_svh = d + 2 * experts;
    t.up_trellis = d + 3 * experts;
    t.up_suh = d + 4 * experts;
    t.up_svh = d + 5 * experts;
    t.down_trellis = d + 6 * experts;
    t.down_suh = d + 7 * experts;
    t.down_svh = d + 8 * experts;
    t.gate_bits = t.up_bits = t.down_bits = nullptr;
    t.bits_mask = (1u << L->bits[0]) | (1u << L->bits[1]) | (1u << L->bits[2]);
    *out = t;
    return 0;
}

}  // extern "C"
