// gguf_moe.hip -- host code: a GGUF v2/v3 image in memory -> one MoE layer.
//
// Container (gguf.zig:587-657, Cursor gguf.zig:1080-1130, readValue/readArray
// gguf.zig:1131-1200): little-endian header `GGUF`, version 2 or 3, tensor and
// metadata counts; metadata key/value pairs (first occurrence of a key wins);
// tensor table (name, 1..8 dims with ggml's fastest axis first, type, offset);
// tensor data from the header's end rounded up to `general.alignment` (default
// 32, a power of two <= 2^24).
//
// MoE configuration (load_gguf.zig:109-128, 251-289): hidden from
// `<arch>.embedding_length`; experts and top-k from `<arch>.expert_count` /
// `.expert_used_count` (2 when the file declares experts but no count); the
// routed width from blk.0.ffn_gate_exps.weight {hidden, width, experts} (the
// tensor wins over `expert_count`), else `.expert_feed_forward_length`, else
// `.feed_forward_length`; the shared width from
// `.expert_shared_feed_forward_length`, else blk.0.ffn_gate_shexp.weight's second
// dimension, else 0 when there is no shared expert.
//
// Layer N (loadMoeLayerStreaming, load_gguf.zig:767-826): the router
// blk.N.ffn_gate_inp.weight as f16 [E][H] (loadLinear: either dimension order,
// any type, f16 read gguf.zig:555-577); the expert payloads
// blk.N.ffn_{gate,up,down}_exps.weight as stored; the shared expert
// blk.N.ffn_{gate,up,down}_shexp.weight and its gate vector
// blk.N.ffn_gate_inp_shexp.weight {hidden}.
#include <stdio.h>
#include <string.h>

#include <algorithm>
#include <map>
#include <string>
#include <vector>

#include "common.h"
#include "kernels.h"

namespace anedvd {
namespace {

enum VType { kU8 = 0, kI8, kU16, kI16, kU32, kI32, kF32, kBool, kStr, kArr, kU64, kI64, kF64 };

struct Value {
    int type = -1;
    uint64_t u = 0;  // unsigned view of the integer kinds (and bool)
    int64_t i = 0;   // signed view
    double f = 0.0;
    std::string s;   // strings
    int arr_type = -1;
    uint64_t arr_n = 0;
    double arr_max = 0.0;  // largest element of a numeric array (feed_forward_length arrays)
    bool arr_numeric = false;

    // Value.asU32 (gguf.zig:197-211): integers that fit, bool as 0/1.
    bool as_u32(uint32_t &out) const
    {
        switch (type) {
        case kU8: case kU16: case kU32: case kU64: case kBool:
            if (u > 0xFFFFFFFFull) return false;
            out = (uint32_t)u;
            return true;
        case kI8: case kI16: case kI32: case kI64:
            if (i < 0 || i > 0xFFFFFFFFll) return false;
            out = (uint32_t)i;
            return true;
        default:
            return false;
        }
    }
    // Value.asU64 (gguf.zig:213-227).
    bool as_u64(uint64_t &out) const
    {
        switch (type) {
        case kU8: case kU16: case kU32: case kU64: case kBool:
            out = u;
            return true;
        case kI8: case kI16: case kI32: case kI64:
            if (i < 0) return false;
            out = (uint64_t)i;
            return true;
        default:
            return false;
        }
    }
};

struct Tensor {
    std::string name;
    std::vector<uint64_t> dims;
    int type = -1;
    uint64_t offset = 0;
    uint64_t elems() const
    {
        uint64_t n = 1;
        for (uint64_t d : dims) n *= d;
        return n;
    }
};

struct Cursor {
    const uint8_t *p;
    size_t n, pos = 0;
    size_t remaining() const { return n - pos; }
    bool take(void *dst, size_t k)
    {
        if (remaining() < k) return false;
        memcpy(dst, p + pos, k);
        pos += k;
        return true;
    }
    bool u32(uint32_t &v) { return take(&v, 4); }
    bool u64(uint64_t &v) { return take(&v, 8); }
    bool str(std::string &s)
    {
        uint64_t len;
        if (!u64(len) || len > remaining()) return false;
        s.assign((const char *)p + pos, (size_t)len);
        pos += (size_t)len;
        return true;
    }
};

constexpr uint32_t kMagic = 0x46554747u;  // "GGUF"

// Element sizes of the scalar value types (0 = not a fixed-size scalar).
size_t scalar_size(int t)
{
    switch (t) {
    case kU8: case kI8: case kBool: return 1;
    case kU16: case kI16: return 2;
    case kU32: case kI32: case kF32: return 4;
    case kU64: case kI64: case kF64: return 8;
    default: return 0;
    }
}

// Reads one scalar of type t into v; false when truncated.
bool read_scalar(Cursor &c, int t, Value &v)
{
    uint8_t b[8] = {0};
    const size_t k = scalar_size(t);
    if (!c.take(b, k)) return false;
    v.type = t;
    switch (t) {
    case kU8: v.u = b[0]; v.i = b[0]; v.f = b[0]; break;
    case kI8: v.i = (int8_t)b[0]; v.u = (uint64_t)v.i; v.f = (double)v.i; break;
    case kBool: v.u = b[0] != 0; v.i = (int64_t)v.u; v.f = (double)v.u; break;
    case kU16: { uint16_t x; memcpy(&x, b, 2); v.u = x; v.i = x; v.f = x; break; }
    case kI16: { int16_t x; memcpy(&x, b, 2); v.i = x; v.u = (uint64_t)v.i; v.f = x; break; }
    case kU32: { uint32_t x; memcpy(&x, b, 4); v.u = x; v.i = x; v.f = x; break; }
    case kI32: { int32_t x; memcpy(&x, b, 4); v.i = x; v.u = (uint64_t)v.i; v.f = x; break; }
    case kF32: { float x; memcpy(&x, b, 4); v.f = x; break; }
    case kU64: { uint64_t x; memcpy(&x, b, 8); v.u = x; v.i = (int64_t)x; v.f = (double)x; break; }
    case kI64: { int64_t x; memcpy(&x, b, 8); v.i = x; v.u = (uint64_t)x; v.f = (double)x; break; }
    case kF64: { double x; memcpy(&x, b, 8); v.f = x; break; }
    }
    return true;
}

struct Parsed {
    const uint8_t *data = nullptr;
    size_t len = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::map<std::string, Value> kv;
    std::vector<Tensor> tensors;
    std::map<std::string, size_t> index;

    const Value *get(const std::string &k) const
    {
        auto it = kv.find(k);
        return it == kv.end() ? nullptr : &it->second;
    }
    const Tensor *tensor(const std::string &name) const
    {
        auto it = index.find(name);
        return it == index.end() ? nullptr : &tensors[it->second];
    }
};

int fail(int rc, const char *what)
{
    set_error("gguf: %s", what);
    return rc;
}

// Gguf.parse (gguf.zig:587-657) with the reference's errors.
int parse(const uint8_t *data, size_t len, Parsed &g)
{
    Cursor c{data, len};
    g.data = data;
    g.len = len;
    uint32_t magic, version;
    if (!c.u32(magic)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: no header");
    if (magic != kMagic) return fail(ANEDVD_E_NOT_GGUF, "NotGgufFile: bad magic");
    if (!c.u32(version)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: no version");
    if (version < 2 || version > 3) return fail(ANEDVD_E_GGUF_VERSION, "UnsupportedVersion: only GGUF v2 and v3");
    g.version = version;
    uint64_t n_tensors, n_kv;
    if (!c.u64(n_tensors) || !c.u64(n_kv)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: no counts");
    if (n_tensors > c.remaining() + 1) return fail(ANEDVD_E_INVALID_METADATA, "TooManyTensors");
    if (n_kv > c.remaining() + 1) return fail(ANEDVD_E_INVALID_METADATA, "TooManyMetadataEntries");
    for (uint64_t q = 0; q < n_kv; q++) {
        std::string key;
        uint32_t vt;
        if (!c.str(key) || !c.u32(vt)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: metadata key");
        Value v;
        if (vt > kF64) return fail(ANEDVD_E_INVALID_METADATA, "UnsupportedMetadataType");
        if (vt == kStr) {
            v.type = kStr;
            if (!c.str(v.s)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: metadata string");
        } else if (vt == kArr) {
            uint32_t et;
            uint64_t cnt;
            if (!c.u32(et)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: array type");
            if (et > kF64 || et == kArr) return fail(ANEDVD_E_INVALID_METADATA, "UnsupportedMetadataType");
            if (!c.u64(cnt)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: array count");
            if (cnt > c.remaining() + 1) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: array count");
            v.type = kArr;
            v.arr_type = (int)et;
            v.arr_n = cnt;
            if (et == kStr) {
                for (uint64_t j = 0; j < cnt; j++) {
                    uint64_t sl;
                    if (!c.u64(sl) || sl > c.remaining()) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: array string");
                    c.pos += (size_t)sl;
                }
            } else {
                v.arr_numeric = et != kBool;
                for (uint64_t j = 0; j < cnt; j++) {
                    Value e;
                    if (!read_scalar(c, (int)et, e)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: array element");
                    const double x = (et == kF32 || et == kF64) ? e.f : (double)e.i;
                    if (j == 0 || x > v.arr_max) v.arr_max = x;
                }
            }
        } else if (!read_scalar(c, (int)vt, v)) {
            return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: metadata value");
        }
        g.kv.emplace(key, std::move(v));  // emplace keeps the first occurrence
    }
    if (const Value *a = g.get("general.alignment")) {
        uint64_t al;
        if (!a->as_u64(al) || al == 0 || al > (1u << 24) || (al & (al - 1)))
            return fail(ANEDVD_E_INVALID_METADATA, "InvalidMetadata: general.alignment");
        g.alignment = al;
    }
    g.tensors.resize((size_t)n_tensors);
    for (uint64_t q = 0; q < n_tensors; q++) {
        Tensor &t = g.tensors[(size_t)q];
        uint32_t nd, tt;
        if (!c.str(t.name) || !c.u32(nd)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: tensor info");
        if (nd == 0 || nd > 8) return fail(ANEDVD_E_INVALID_SHAPE, "InvalidTensorShape: 1..8 dimensions");
        t.dims.resize(nd);
        for (uint32_t j = 0; j < nd; j++)
            if (!c.u64(t.dims[j])) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: tensor dims");
        if (!c.u32(tt) || !c.u64(t.offset)) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: tensor info");
        t.type = (int)tt;
        g.index.emplace(t.name, (size_t)q);
    }
    g.data_offset = (c.pos + g.alignment - 1) / g.alignment * g.alignment;
    if (g.data_offset > len) return fail(ANEDVD_E_TRUNCATED, "TruncatedFile: data section");
    return ANEDVD_OK;
}

// Gguf.tensorBytes (gguf.zig:425-436).
int tensor_bytes(const Parsed &g, const Tensor &t, const uint8_t *&p, size_t &n)
{
    const int epb = block_elems(t.type), bpb = block_bytes(t.type);
    if (!epb || !bpb) {
        set_error("gguf: %s: UnsupportedType %d", t.name.c_str(), t.type);
        return ANEDVD_E_UNSUPPORTED_TYPE;
    }
    const uint64_t e = t.elems();
    if (e % epb) {
        set_error("gguf: %s: InvalidTensorShape (%llu elements, blocks of %d)", t.name.c_str(),
                  (unsigned long long)e, epb);
        return ANEDVD_E_INVALID_SHAPE;
    }
    const unsigned __int128 nbytes = (unsigned __int128)(e / epb) * bpb;
    const unsigned __int128 end = (unsigned __int128)g.data_offset + t.offset + nbytes;
    if (end > g.len) {
        set_error("gguf: %s: TensorDataOutOfRange", t.name.c_str());
        return ANEDVD_E_OUT_OF_RANGE;
    }
    p = g.data + g.data_offset + t.offset;
    n = (size_t)nbytes;
    return ANEDVD_OK;
}

std::string akey(const std::string &arch, const char *suffix) { return arch + "." + suffix; }

bool get_u32(const Parsed &g, const std::string &k, uint32_t &out)
{
    const Value *v = g.get(k);
    return v && v->as_u32(out);
}

// The MoE configuration of load_gguf.zig:109-128 and 251-289.
int moe_config(const Parsed &g, anedvd_gguf_moe_cfg &info)
{
    memset(&info, 0, sizeof info);
    info.version = g.version;
    info.n_tensors = g.tensors.size();
    info.data_offset = g.data_offset;
    const Value *av = g.get("general.architecture");
    if (!av || av->type != kStr) return fail(ANEDVD_E_INVALID_METADATA, "no general.architecture");
    const std::string arch = av->s;
    snprintf(info.arch, sizeof info.arch, "%s", arch.c_str());
    if (!get_u32(g, akey(arch, "embedding_length"), info.hidden)) {
        set_error("gguf: no %s in this file (arch \"%s\")", akey(arch, "embedding_length").c_str(), arch.c_str());
        return ANEDVD_E_MISSING_TENSOR;
    }
    if (!get_u32(g, akey(arch, "block_count"), info.n_layers)) {
        set_error("gguf: no %s in this file", akey(arch, "block_count").c_str());
        return ANEDVD_E_MISSING_TENSOR;
    }
    // feed_forward_length: a scalar, or an array whose largest entry sizes the layers
    uint32_t inter = 0;
    if (const Value *fv = g.get(akey(arch, "feed_forward_length"))) {
        if (fv->type == kArr && fv->arr_numeric && fv->arr_n && fv->arr_max >= 0 && fv->arr_max <= 4294967295.0)
            inter = (uint32_t)fv->arr_max;
        else
            fv->as_u32(inter);
    }
    if (!get_u32(g, akey(arch, "expert_count"), info.n_experts) || info.n_experts == 0) {
        set_error("gguf: %s declares no experts (%s)", arch.c_str(), akey(arch, "expert_count").c_str());
        return ANEDVD_E_INVALID_METADATA;
    }
    if (!get_u32(g, akey(arch, "expert_used_count"), info.k) || info.k == 0) info.k = 2;
    if (const Tensor *t = g.tensor("blk.0.ffn_gate_exps.weight")) {
        if (t->dims.size() == 3) {
            info.inter = (uint32_t)t->dims[1];
            if (t->dims[2] != info.n_experts) info.n_experts = (uint32_t)t->dims[2];  // the tensor wins
        }
    } else if (!get_u32(g, akey(arch, "expert_feed_forward_length"), info.inter)) {
        info.inter = inter;
    }
    if (!get_u32(g, akey(arch, "expert_shared_feed_forward_length"), info.shared_inter)) {
        const Tensor *s = g.tensor("blk.0.ffn_gate_shexp.weight");
        info.shared_inter = !s ? 0 : (s->dims.size() >= 2 ? (uint32_t)s->dims[1] : inter);
    }
    if (info.inter == 0) return fail(ANEDVD_E_INVALID_METADATA, "IncompleteConfig: no expert width");
    // Gemma's FFN activation is gelu_pytorch_tanh (load_gguf.zig:145-158).
    info.use_gelu = arch.compare(0, 5, "gemma") == 0;
    return ANEDVD_OK;
}

std::string blk(uint32_t layer, const char *what)
{
    char b[96];
    snprintf(b, sizeof b, "blk.%u.%s.weight", layer, what);
    return b;
}

int find(const Parsed &g, const std::string &name, const Tensor *&t)
{
    t = g.tensor(name);
    if (!t) {
        set_error("gguf: no tensor %s", name.c_str());
        return ANEDVD_E_MISSING_TENSOR;
    }
    return ANEDVD_OK;
}

// The block's tensor types into `info` (-1 where absent) and a check of every
// shape the layer needs.
int block_shapes(const Parsed &g, uint32_t layer, anedvd_gguf_moe_cfg &info)
{
    if (layer >= info.n_layers) {
        set_error("gguf: layer %u of %u", layer, info.n_layers);
        return ANEDVD_E_INVALID_ARG;
    }
    const uint64_t H = info.hidden, I = info.inter, E = info.n_experts, Is = info.shared_inter;
    const Tensor *t;
    struct Need {
        const char *what;
        int32_t *type;
        uint64_t d0, d1, d2;  // d2 = 0: a matrix
    } need[] = {{"ffn_gate_exps", &info.gate_type, H, I, E}, {"ffn_up_exps", &info.up_type, H, I, E},
                {"ffn_down_exps", &info.down_type, I, H, E}};
    for (const Need &n : need) {
        ANEDVD_TRY(find(g, blk(layer, n.what), t));
        if (t->dims.size() != 3 || t->dims[0] != n.d0 || t->dims[1] != n.d1 || t->dims[2] != n.d2) {
            set_error("gguf: %s has dims other than {%llu, %llu, %llu}", t->name.c_str(), (unsigned long long)n.d0,
                      (unsigned long long)n.d1, (unsigned long long)n.d2);
            return ANEDVD_E_DIMENSION;
        }
        *n.type = t->type;
    }
    ANEDVD_TRY(find(g, blk(layer, "ffn_gate_inp"), t));
    if (t->elems() != H * E || t->dims.size() < 2 ||
        !((t->dims[0] == H && t->dims[1] == E) || (t->dims[0] == E && t->dims[1] == H))) {
        set_error("gguf: %s is not a %llu x %llu matrix", t->name.c_str(), (unsigned long long)E,
                  (unsigned long long)H);
        return ANEDVD_E_DIMENSION;
    }
    info.router_type = t->type;
    info.shared_type = -1;
    info.has_shared_gate_lin = 0;
    if (Is) {
        // loadLinear (load_gguf.zig:358-386) takes {in, out} as stored or {out, in}
        // transposed, of any type, and keeps the result as f16 [out][in].  Stored
        // {in, out} with one block type for the three, the payloads go to the GPU
        // as they are; otherwise they are read as f16 and transposed as loadLinear
        // does (shared_as_f16).
        int32_t ty[3];
        bool transposed = false;
        const char *names[3] = {"ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp"};
        for (int j = 0; j < 3; j++) {
            ANEDVD_TRY(find(g, blk(layer, names[j]), t));
            const uint64_t a = j < 2 ? H : Is, b = j < 2 ? Is : H;
            const bool as_stored = t->dims.size() >= 2 && t->dims[0] == a && t->dims[1] == b;
            const bool swapped = t->dims.size() >= 2 && t->dims[0] == b && t->dims[1] == a;
            if (t->elems() != a * b || !(as_stored || swapped)) {
                set_error("gguf: %s is not a %llu x %llu matrix", t->name.c_str(), (unsigned long long)b,
                          (unsigned long long)a);
                return ANEDVD_E_DIMENSION;
            }
            if (!as_stored) transposed = true;
            if (!block_elems(t->type)) {
                set_error("gguf: %s has unknown ggml type %d", t->name.c_str(), (int)t->type);
                return ANEDVD_E_UNSUPPORTED_TYPE;
            }
            ty[j] = t->type;
        }
        info.shared_type = ty[0];
        info.shared_as_f16 = transposed || ty[0] != ty[1] || ty[0] != ty[2] || !mm_supported(ty[0]);
        // The gate vector is mandatory once there is a shared expert (load_gguf.zig:818-823).
        ANEDVD_TRY(find(g, blk(layer, "ffn_gate_inp_shexp"), t));
        if (t->elems() != H) {
            set_error("gguf: %s has %llu elements, not %llu", t->name.c_str(), (unsigned long long)t->elems(),
                      (unsigned long long)H);
            return ANEDVD_E_DIMENSION;
        }
        info.has_shared_gate_lin = 1;
    }
    return ANEDVD_OK;
}

uint16_t f32_to_f16(float x)
{
    const _Float16 h = (_Float16)x;  // round to nearest even
    uint16_t b;
    memcpy(&b, &h, 2);
    return b;
}

float f16_to_f32(uint16_t b)
{
    _Float16 h;
    memcpy(&h, &b, 2);
    return (float)h;
}

// Gguf.readF16 / readF32 of a whole tensor: f16 as stored, anything else
// dequantised (on the device, bit-exact) and, for f16, rounded to nearest even.
int read_f32(anedvd_moe_ctx *ctx, const Parsed &g, const Tensor &t, std::vector<float> &out)
{
    const uint8_t *p;
    size_t n;
    ANEDVD_TRY(tensor_bytes(g, t, p, n));
    out.resize((size_t)t.elems());
    if (t.type == ANEDVD_F32) {
        memcpy(out.data(), p, out.size() * 4);
        return ANEDVD_OK;
    }
    if (t.type == ANEDVD_F16) {
        for (size_t i = 0; i < out.size(); i++) {
            uint16_t b;
            memcpy(&b, p + 2 * i, 2);
            out[i] = f16_to_f32(b);
        }
        return ANEDVD_OK;
    }
    return anedvd_dequantize_range(ctx, t.type, p, n, 0, out.data(), out.size());
}

int read_f16(anedvd_moe_ctx *ctx, const Parsed &g, const Tensor &t, std::vector<uint16_t> &out)
{
    out.resize((size_t)t.elems());
    if (t.type == ANEDVD_F16) {
        const uint8_t *p;
        size_t n;
        ANEDVD_TRY(tensor_bytes(g, t, p, n));
        memcpy(out.data(), p, out.size() * 2);
        return ANEDVD_OK;
    }
    std::vector<float> f;
    ANEDVD_TRY(read_f32(ctx, g, t, f));
    for (size_t i = 0; i < f.size(); i++) out[i] = f32_to_f16(f[i]);
    return ANEDVD_OK;
}

}  // namespace
}  // namespace anedvd

using namespace anedvd;

extern "C" {

int anedvd_gguf_moe_info(const void *gguf, size_t len, uint32_t layer, anedvd_gguf_moe_cfg *out)
{
    if (!gguf || !out) {
        set_error("gguf_moe_info: null argument");
        return ANEDVD_E_INVALID_ARG;
    }
    Parsed g;
    ANEDVD_TRY(parse((const uint8_t *)gguf, len, g));
    ANEDVD_TRY(moe_config(g, *out));
    return block_shapes(g, layer, *out);
}

int anedvd_moe_layer_create_gguf(anedvd_moe_ctx *ctx, const void *gguf, size_t len, uint32_t layer,
                                 const anedvd_gguf_moe_opts *opts, anedvd_moe_layer **out)
{
    if (!ctx || !gguf || !out) {
        set_error("layer_create_gguf: null argument");
        return ANEDVD_E_INVALID_ARG;
    }
    *out = nullptr;
    Parsed g;
    anedvd_gguf_moe_cfg info;
    ANEDVD_TRY(parse((const uint8_t *)gguf, len, g));
    ANEDVD_TRY(moe_config(g, info));
    ANEDVD_TRY(block_shapes(g, layer, info));
    const uint32_t H = info.hidden, E = info.n_experts;
    anedvd_moe_layer_desc d{};
    d.hidden = H;
    d.inter = info.inter;
    d.n_experts = E;
    d.k = info.k;
    // The GGUF loader leaves norm_topk_prob false and sets use_gelu for the gemma
    // architectures only (load_gguf.zig:145-158); a caller may override either.
    d.norm_topk_prob = opts && opts->norm_topk_prob >= 0 ? opts->norm_topk_prob : 0;
    d.use_gelu = opts && opts->use_gelu >= 0 ? opts->use_gelu : info.use_gelu;
    const Tensor *t;
    const uint8_t *p;
    size_t n;
    ANEDVD_TRY(find(g, blk(layer, "ffn_gate_exps"), t));
    ANEDVD_TRY(tensor_bytes(g, *t, p, n));
    d.gate_type = t->type, d.gate = p, d.gate_bytes = n;
    ANEDVD_TRY(find(g, blk(layer, "ffn_up_exps"), t));
    ANEDVD_TRY(tensor_bytes(g, *t, p, n));
    d.up_type = t->type, d.up = p, d.up_bytes = n;
    ANEDVD_TRY(find(g, blk(layer, "ffn_down_exps"), t));
    ANEDVD_TRY(tensor_bytes(g, *t, p, n));
    d.down_type = t->type, d.down = p, d.down_bytes = n;
    // router: loadLinear(in = hidden, out = experts) -> [E][H], transposing {E, H}
    ANEDVD_TRY(find(g, blk(layer, "ffn_gate_inp"), t));
    std::vector<uint16_t> router;
    ANEDVD_TRY(read_f16(ctx, g, *t, router));
    if (!(t->dims[0] == H && t->dims[1] == E)) {
        std::vector<uint16_t> tr(router.size());
        for (uint32_t o = 0; o < E; o++)
            for (uint32_t i = 0; i < H; i++) tr[(size_t)o * H + i] = router[(size_t)i * E + o];
        router.swap(tr);
    }
    d.router = router.data();
    std::vector<uint16_t> lin, sh16[3];
    if (info.shared_inter) {
        d.shared_inter = info.shared_inter;
        d.shared_type = info.shared_as_f16 ? ANEDVD_F16 : info.shared_type;
        const char *names[3] = {"ffn_gate_shexp", "ffn_up_shexp", "ffn_down_shexp"};
        const void **ptrs[3] = {&d.shared_gate, &d.shared_up, &d.shared_down};
        size_t *lens[3] = {&d.shared_gate_bytes, &d.shared_up_bytes, &d.shared_down_bytes};
        for (int j = 0; j < 3; j++) {
            ANEDVD_TRY(find(g, blk(layer, names[j]), t));
            if (!info.shared_as_f16) {
                ANEDVD_TRY(tensor_bytes(g, *t, p, n));
                *ptrs[j] = p, *lens[j] = n;
                continue;
            }
            // loadLinear: readF16, then [out][in] (transposed when stored {out, in})
            const uint64_t in = j < 2 ? H : info.shared_inter, outd = j < 2 ? info.shared_inter : H;
            ANEDVD_TRY(read_f16(ctx, g, *t, sh16[j]));
            if (t->dims[0] != in) {
                std::vector<uint16_t> tr(sh16[j].size());
                for (uint64_t o = 0; o < outd; o++)
                    for (uint64_t i = 0; i < in; i++) tr[o * in + i] = sh16[j][i * outd + o];
                sh16[j].swap(tr);
            }
            *ptrs[j] = sh16[j].data(), *lens[j] = sh16[j].size() * 2;
        }
        // readF32 then f16 (load_gguf.zig:818-823)
        ANEDVD_TRY(find(g, blk(layer, "ffn_gate_inp_shexp"), t));
        std::vector<float> f;
        ANEDVD_TRY(read_f32(ctx, g, *t, f));
        lin.resize(f.size());
        for (size_t i = 0; i < f.size(); i++) lin[i] = f32_to_f16(f[i]);
        d.shared_gate_lin = lin.data();
    }
    return anedvd_moe_layer_create(ctx, &d, out);
}

}  // extern "C"
