// gguf.cpp -- GGUF v2/v3 reader: the file is memory-mapped read-only, the
// header, metadata and tensor table are parsed with a bounds check on every
// read, and tensor data is handed out as pointers into the mapping (no copy),
// ready for ulspec_model_set_tensor / ulspec_weight_upload.
//
// Replaces GGUFParser (src/core/gguf_parser.cpp): read_header (:40-70),
// read_metadata (:72-228), read_tensor_infos (:230-290, whose size_bytes uses
// the wrong block sizes of gguf_types.h:35-58) and read_tensor_data_direct
// (:348-361, a seek + read per tensor).  Layout (GGUF spec, little endian):
//   u32 magic "GGUF" | u32 version | u64 n_tensors | u64 n_kv
//   n_kv x { string key | u32 type | value }         string = u64 len + bytes
//   n_tensors x { string name | u32 n_dims | u64 ne[n_dims] | u32 type | u64 offset }
//   padding to general.alignment (default 32) | tensor data (offsets relative here)
// No device work: everything here runs on a host without a GPU.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdarg>
#include <cstdio>
#include <algorithm>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "../../../include/ulspec.h"
#include "model.h"

using namespace ulspec;

struct ulspec_gguf {
    struct Kv {
        std::string key;
        uint32_t type = 0;        // ULSPEC_GGUF_*
        uint32_t arr_type = 0;    // element type of an array
        uint64_t arr_len = 0;
        uint64_t pos = 0;         // file offset of the value (after the type word; arrays: first element)
        uint64_t end = 0;         // file offset after the value
    };
    struct Tensor {
        std::string name;
        uint32_t type = 0, n_dims = 0;
        uint64_t ne[4] = {1, 1, 1, 1};
        uint64_t offset = 0, nbytes = 0;  // nbytes 0: type without a fixed block size
    };
    int fd = -1;
    const uint8_t* base = nullptr;
    uint64_t size = 0;
    uint32_t version = 0;
    uint64_t alignment = 32, data_offset = 0;
    std::vector<Kv> kv;
    std::vector<Tensor> tensors;
    std::map<std::string, uint64_t> kv_index, tensor_index;
    std::string err;
};

namespace {

constexpr uint32_t kGgufMagic = 0x46554747u;  // "GGUF"

struct Cursor {
    const uint8_t* p;
    uint64_t size, pos;
    bool ok = true;
    bool need(uint64_t n)
    {
        if (!ok || n > size - pos) ok = false;
        return ok;
    }
    template <class T>
    T get()
    {
        T v{};
        if (need(sizeof(T))) {
            std::memcpy(&v, p + pos, sizeof(T));
            pos += sizeof(T);
        }
        return v;
    }
    bool skip(uint64_t n)
    {
        if (need(n)) pos += n;
        return ok;
    }
    std::string str()
    {
        const uint64_t n = get<uint64_t>();
        if (!need(n)) return std::string();
        std::string s(reinterpret_cast<const char*>(p + pos), (size_t)n);
        pos += n;
        return s;
    }
};

// bytes of a scalar GGUF value type; 0 for string / array / unknown
uint64_t scalar_size(uint32_t t)
{
    switch (t) {
    case ULSPEC_GGUF_U8: case ULSPEC_GGUF_I8: case ULSPEC_GGUF_BOOL: return 1;
    case ULSPEC_GGUF_U16: case ULSPEC_GGUF_I16: return 2;
    case ULSPEC_GGUF_U32: case ULSPEC_GGUF_I32: case ULSPEC_GGUF_F32: return 4;
    case ULSPEC_GGUF_U64: case ULSPEC_GGUF_I64: case ULSPEC_GGUF_F64: return 8;
    default: return 0;
    }
}

// Skip one value of type t (arrays may nest, depth-limited).
bool skip_value(Cursor& c, uint32_t t, int depth)
{
    if (const uint64_t s = scalar_size(t)) return c.skip(s);
    if (t == ULSPEC_GGUF_STRING) {
        const uint64_t n = c.get<uint64_t>();
        return c.skip(n);
    }
    if (t == ULSPEC_GGUF_ARRAY && depth < 4) {
        const uint32_t et = c.get<uint32_t>();
        const uint64_t n = c.get<uint64_t>();
        if (!c.ok) return false;
        if (const uint64_t s = scalar_size(et)) return n <= (c.size - c.pos) / s ? c.skip(n * s) : (c.ok = false);
        for (uint64_t i = 0; i < n && c.ok; ++i) skip_value(c, et, depth + 1);
        return c.ok;
    }
    return c.ok = false;
}

ulspec_status gfail(ulspec_gguf* g, ulspec_status st, const char* fmt, ...)
{
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g->err = buf;
    return st;
}

ulspec_status parse(ulspec_gguf* g)
{
    Cursor c{g->base, g->size, 0};
    const uint32_t magic = c.get<uint32_t>();
    g->version = c.get<uint32_t>();
    if (!c.ok || magic != kGgufMagic) return gfail(g, ULSPEC_EINVAL, "not a GGUF file (magic)");
    if (g->version < 2 || g->version > 3)
        return gfail(g, ULSPEC_EUNSUPPORTED, "GGUF version %u (2 and 3 are read)", g->version);
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    // every entry takes at least 8 bytes: bounds the counts before reserving
    if (!c.ok || n_tensors > g->size / 8 || n_kv > g->size / 8) return gfail(g, ULSPEC_EINVAL, "GGUF header counts");
    g->kv.reserve((size_t)std::min<uint64_t>(n_kv, 4096));  // a hostile count fails below, before it allocates
    for (uint64_t i = 0; i < n_kv; ++i) {
        ulspec_gguf::Kv e;
        e.key = c.str();
        e.type = c.get<uint32_t>();
        e.pos = c.pos;
        if (e.type == ULSPEC_GGUF_ARRAY) {
            e.arr_type = c.get<uint32_t>();
            e.arr_len = c.get<uint64_t>();
            c.pos = e.pos;
        }
        if (!c.ok || !skip_value(c, e.type, 0))
            return gfail(g, ULSPEC_EINVAL, "GGUF metadata entry %llu ('%s') truncated or of unknown type",
                         (unsigned long long)i, e.key.c_str());
        if (e.type == ULSPEC_GGUF_ARRAY) e.pos += 12;
        e.end = c.pos;
        if (!g->kv_index.emplace(e.key, g->kv.size()).second)
            return gfail(g, ULSPEC_EINVAL, "GGUF metadata key '%s' repeated", e.key.c_str());
        g->kv.push_back(std::move(e));
    }
    // general.alignment (u32 in files written by ggml)
    auto it = g->kv_index.find("general.alignment");
    if (it != g->kv_index.end()) {
        int64_t a = 0;
        if (ulspec_gguf_get_int(g, "general.alignment", &a) != ULSPEC_OK || a <= 0 || (a & (a - 1)))
            return gfail(g, ULSPEC_EINVAL, "general.alignment must be a power of two");
        g->alignment = (uint64_t)a;
    }
    g->tensors.reserve((size_t)std::min<uint64_t>(n_tensors, 4096));
    for (uint64_t i = 0; i < n_tensors; ++i) {
        ulspec_gguf::Tensor t;
        t.name = c.str();
        t.n_dims = c.get<uint32_t>();
        if (!c.ok || t.n_dims < 1 || t.n_dims > 4)
            return gfail(g, ULSPEC_EINVAL, "GGUF tensor %llu: bad dimension count", (unsigned long long)i);
        for (uint32_t d = 0; d < t.n_dims; ++d) t.ne[d] = c.get<uint64_t>();
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) return gfail(g, ULSPEC_EINVAL, "GGUF tensor table truncated");
        if (!g->tensor_index.emplace(t.name, g->tensors.size()).second)
            return gfail(g, ULSPEC_EINVAL, "GGUF tensor '%s' repeated", t.name.c_str());
        g->tensors.push_back(std::move(t));
    }
    g->data_offset = (c.pos + g->alignment - 1) / g->alignment * g->alignment;
    for (auto& t : g->tensors) {
        const int bs = ulspec_ggml_blck_size(t.type), ts = ulspec_ggml_type_size(t.type);
        if (t.offset % g->alignment)
            return gfail(g, ULSPEC_EINVAL, "GGUF tensor '%s': offset not aligned", t.name.c_str());
        if (bs == 0) continue;  // unknown block layout: listed, data not handed out
        if (t.ne[0] % (uint64_t)bs)
            return gfail(g, ULSPEC_EINVAL, "GGUF tensor '%s': row of %llu not a multiple of the block (%d)",
                         t.name.c_str(), (unsigned long long)t.ne[0], bs);
        // bytes = ne0 / bs * ts * ne1 * ne2 * ne3; the product stops growing
        // once it passes the file size, so with every factor below 2^64 it
        // never wraps in 128 bits
        unsigned __int128 n = (unsigned __int128)(t.ne[0] / (uint64_t)bs) * (uint64_t)ts;
        for (int d = 1; d < 4 && n <= g->size; ++d) n *= t.ne[d];
        if (n > g->size || g->data_offset > g->size || t.offset > g->size - g->data_offset ||
            (uint64_t)n > g->size - g->data_offset - t.offset)
            return gfail(g, ULSPEC_EINVAL, "GGUF tensor '%s': data past the end of the file", t.name.c_str());
        t.nbytes = (uint64_t)n;
    }
    return ULSPEC_OK;
}

const ulspec_gguf::Kv* find_kv(const ulspec_gguf* g, const char* key)
{
    auto it = g->kv_index.find(key ? key : "");
    return it == g->kv_index.end() ? nullptr : &g->kv[it->second];
}

template <class T>
T load_at(const ulspec_gguf* g, uint64_t pos)
{
    T v;
    std::memcpy(&v, g->base + pos, sizeof(T));
    return v;
}

}  // namespace

extern "C" ulspec_status ulspec_gguf_open(const char* path, ulspec_gguf** out, char* err, size_t err_len)
{
    auto report = [&](const std::string& m) {
        if (err && err_len) snprintf(err, err_len, "%s", m.c_str());
    };
    if (!path || !out) {
        report("gguf_open: null argument");
        return ULSPEC_EINVAL;
    }
    *out = nullptr;
    ulspec_gguf* g = new ulspec_gguf();
    g->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat sb;
    if (g->fd < 0 || fstat(g->fd, &sb) != 0) {
        report(std::string("gguf_open: cannot open ") + path + ": " + strerror(errno));
        ulspec_gguf_close(g);
        return ULSPEC_EINVAL;
    }
    g->size = (uint64_t)sb.st_size;
    if (g->size < 24) {
        report("gguf_open: file too short for a GGUF header");
        ulspec_gguf_close(g);
        return ULSPEC_EINVAL;
    }
    void* m = mmap(nullptr, (size_t)g->size, PROT_READ, MAP_PRIVATE, g->fd, 0);
    if (m == MAP_FAILED) {
        report(std::string("gguf_open: mmap failed: ") + strerror(errno));
        ulspec_gguf_close(g);
        return ULSPEC_ENOMEM;
    }
    g->base = static_cast<const uint8_t*>(m);
    const ulspec_status st = parse(g);
    if (st != ULSPEC_OK) {
        report(g->err);
        ulspec_gguf_close(g);
        return st;
    }
    *out = g;
    return ULSPEC_OK;
}

extern "C" void ulspec_gguf_close(ulspec_gguf* g)
{
    if (!g) return;
    if (g->base) munmap(const_cast<uint8_t*>(g->base), (size_t)g->size);
    if (g->fd >= 0) close(g->fd);
    delete g;
}

extern "C" const char* ulspec_gguf_last_error(const ulspec_gguf* g)
{
    return g ? g->err.c_str() : "no GGUF handle";
}

extern "C" ulspec_status ulspec_gguf_header(const ulspec_gguf* g, uint32_t* version, uint64_t* n_tensors,
                                            uint64_t* n_kv, uint64_t* alignment, uint64_t* data_offset)
{
    if (!g) return ULSPEC_EINVAL;
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_kv) *n_kv = g->kv.size();
    if (alignment) *alignment = g->alignment;
    if (data_offset) *data_offset = g->data_offset;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_gguf_tensor(const ulspec_gguf* g, uint64_t i, const char** name, uint32_t* ggml_type,
                                            uint32_t* n_dims, uint64_t ne[4], uint64_t* offset, uint64_t* nbytes,
                                            const void** data)
{
    if (!g || i >= g->tensors.size()) return ULSPEC_EINVAL;
    const auto& t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (ggml_type) *ggml_type = t.type;
    if (n_dims) *n_dims = t.n_dims;
    if (ne)
        for (int d = 0; d < 4; ++d) ne[d] = t.ne[d];
    if (offset) *offset = t.offset;
    if (nbytes) *nbytes = t.nbytes;
    if (data) *data = t.nbytes ? g->base + g->data_offset + t.offset : nullptr;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_gguf_find_tensor(const ulspec_gguf* g, const char* name, uint64_t* index)
{
    if (!g || !name || !index) return ULSPEC_EINVAL;
    auto it = g->tensor_index.find(name);
    if (it == g->tensor_index.end()) return ULSPEC_EINVAL;
    *index = it->second;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_gguf_kv(const ulspec_gguf* g, uint64_t i, const char** key, uint32_t* value_type,
                                        uint32_t* array_type, uint64_t* array_len)
{
    if (!g || i >= g->kv.size()) return ULSPEC_EINVAL;
    const auto& e = g->kv[i];
    if (key) *key = e.key.c_str();
    if (value_type) *value_type = e.type;
    if (array_type) *array_type = e.arr_type;
    if (array_len) *array_len = e.arr_len;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_gguf_kv_bytes(const ulspec_gguf* g, uint64_t i, const void** data, uint64_t* nbytes)
{
    if (!g || i >= g->kv.size() || !data || !nbytes) return ULSPEC_EINVAL;
    *data = g->base + g->kv[i].pos;
    *nbytes = g->kv[i].end - g->kv[i].pos;
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_gguf_get_int(const ulspec_gguf* g, const char* key, int64_t* v)
{
    const ulspec_gguf::Kv* e = g ? find_kv(g, key) : nullptr;
    if (!e || !v) return ULSPEC_EINVAL;
    switch (e->type) {
    case ULSPEC_GGUF_U8: *v = load_at<uint8_t>(g, e->pos); break;
    case ULSPEC_GGUF_I8: *v = load_at<int8_t>(g, e->pos); break;
    case ULSPEC_GGUF_BOOL: *v = load_at<uint8_t>(g, e->pos) != 0; break;
    case ULSPEC_GGUF_U16: *v = load_at<uint16_t>(g, e->pos); break;
    case ULSPEC_GGUF_I16: *v = load_at<int16_t>(g, e->pos); break;
    case ULSPEC_GGUF_U32: *v = load_at<uint32_t>(g, e->pos); break;
    case ULSPEC_GGUF_I32: *v = load_at<int32_t>(g, e->pos); break;
    case ULSPEC_GGUF_U64: {
        const uint64_t u = load_at<uint64_t>(g, e->pos);
        if (u > (uint64_t)INT64_MAX) return ULSPEC_EINVAL;
        *v = (int64_t)u;
        break;
    }
    case ULSPEC_GGUF_I64: *v = load_at<int64_t>(g, e->pos); break;
    default: return ULSPEC_EINVAL;
    }
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_gguf_get_float(const ulspec_gguf* g, const char* key, double* v)
{
    const ulspec_gguf::Kv* e = g ? find_kv(g, key) : nullptr;
    if (!e || !v) return ULSPEC_EINVAL;
    if (e->type == ULSPEC_GGUF_F32) *v = load_at<float>(g, e->pos);
    else if (e->type == ULSPEC_GGUF_F64) *v = load_at<double>(g, e->pos);
    else {
        int64_t i = 0;
        if (ulspec_gguf_get_int(g, key, &i) != ULSPEC_OK) return ULSPEC_EINVAL;
        *v = (double)i;
    }
    return ULSPEC_OK;
}

extern "C" ulspec_status ulspec_gguf_get_str(const ulspec_gguf* g, const char* key, const char** v, uint64_t* len)
{
    const ulspec_gguf::Kv* e = g ? find_kv(g, key) : nullptr;
    if (!e || !v || e->type != ULSPEC_GGUF_STRING) return ULSPEC_EINVAL;
    const uint64_t n = load_at<uint64_t>(g, e->pos);
    *v = reinterpret_cast<const char*>(g->base + e->pos + 8);
    if (len) *len = n;
    return ULSPEC_OK;
}

// Llama hyper-parameters from the metadata (keys under the architecture name,
// "<arch>.embedding_length" etc.; head_count_kv defaults to head_count,
// rope.freq_base to 10000, the RMSNorm epsilon to 1e-5), the vocabulary from
// token_embd.weight (ne[1]).  max_ctx 0 takes <arch>.context_length.
extern "C" ulspec_status ulspec_gguf_llama_cfg(const ulspec_gguf* gc, uint32_t max_ctx, ulspec_model_cfg* cfg)
{
    ulspec_gguf* g = const_cast<ulspec_gguf*>(gc);
    if (!g || !cfg) return ULSPEC_EINVAL;
    std::string arch = "llama";
    const char* s = nullptr;
    uint64_t n = 0;
    if (ulspec_gguf_get_str(g, "general.architecture", &s, &n) == ULSPEC_OK) arch.assign(s, (size_t)n);
    if (arch != "llama") return gfail(g, ULSPEC_EUNSUPPORTED, "architecture '%s' (llama only)", arch.c_str());
    auto need = [&](const char* k, int64_t* v) {
        const std::string key = arch + "." + k;
        if (ulspec_gguf_get_int(g, key.c_str(), v) != ULSPEC_OK || *v <= 0 || *v > INT32_MAX) {
            gfail(g, ULSPEC_EINVAL, "metadata '%s' missing or out of range", key.c_str());
            return false;
        }
        return true;
    };
    int64_t dim, layers, heads, kv_heads, ffn, ctx;
    if (!need("embedding_length", &dim) || !need("block_count", &layers) || !need("attention.head_count", &heads) ||
        !need("feed_forward_length", &ffn) || !need("context_length", &ctx))
        return ULSPEC_EINVAL;
    if (ulspec_gguf_get_int(g, (arch + ".attention.head_count_kv").c_str(), &kv_heads) != ULSPEC_OK) kv_heads = heads;
    double eps = 1e-5, base = 10000.0;
    (void)ulspec_gguf_get_float(g, (arch + ".attention.layer_norm_rms_epsilon").c_str(), &eps);
    (void)ulspec_gguf_get_float(g, (arch + ".rope.freq_base").c_str(), &base);
    uint64_t ti = 0;
    if (ulspec_gguf_find_tensor(g, "token_embd.weight", &ti) != ULSPEC_OK)
        return gfail(g, ULSPEC_EINVAL, "tensor 'token_embd.weight' missing");
    const auto& te = g->tensors[ti];
    if (te.ne[0] != (uint64_t)dim || te.ne[1] == 0 || te.ne[1] > INT32_MAX)
        return gfail(g, ULSPEC_EINVAL, "token_embd.weight shape does not match embedding_length");
    cfg->dim = (uint32_t)dim;
    cfg->n_layers = (uint32_t)layers;
    cfg->n_heads = (uint32_t)heads;
    cfg->n_kv_heads = (uint32_t)kv_heads;
    cfg->ffn = (uint32_t)ffn;
    cfg->vocab = (uint32_t)te.ne[1];
    cfg->max_ctx = max_ctx ? max_ctx : (uint32_t)ctx;
    cfg->rms_eps = (float)eps;
    cfg->rope_base = (float)base;
    return ULSPEC_OK;
}

// Create a model from the file: configuration from the metadata, every
// tensor through ulspec_model_set_tensor by its GGUF name (the weight map of
// Model::load_from_gguf, src/inference/model.cpp:190-246).  Matrices may be
// Q4_0, Q4_K, Q6_K, Q8_0 or F16 (the types Q4_K_M files use); a tensor of
// another type fails with ULSPEC_EUNSUPPORTED naming it; tensors the model
// does not use (rope_freqs, ...) are skipped.
extern "C" ulspec_status ulspec_model_load_gguf(ulspec_ctx* ctx, const ulspec_gguf* g, uint32_t max_ctx,
                                                ulspec_model** out)
{
    return ulspec_model_load_gguf_batch(ctx, g, max_ctx, 1, out);
}

extern "C" ulspec_status ulspec_model_load_gguf_batch(ulspec_ctx* ctx, const ulspec_gguf* g, uint32_t max_ctx,
                                                      uint32_t n_seq, ulspec_model** out)
{
    ULSPEC_CHECK_CTX(ctx);
    if (!g || !out) return fail(ctx, ULSPEC_EINVAL, "model_load_gguf: null argument");
    *out = nullptr;
    ulspec_model_cfg cfg{};
    if (ulspec_gguf_llama_cfg(g, max_ctx, &cfg) != ULSPEC_OK)
        return fail(ctx, ULSPEC_EINVAL, "model_load_gguf: %s", g->err.c_str());
    ulspec_model* m = nullptr;
    ulspec_status st = ulspec_model_create_batch(ctx, &cfg, n_seq, &m);
    if (st != ULSPEC_OK) return st;
    for (const auto& t : g->tensors) {
        if (t.name == "rope_freqs.weight") continue;  // angles are computed from rope_base
        if (t.nbytes == 0) {
            ulspec_model_destroy(m);
            return fail(ctx, ULSPEC_EUNSUPPORTED, "model_load_gguf: tensor '%s' has ggml type %u, not read",
                        t.name.c_str(), t.type);
        }
        if (t.n_dims > 2 || t.ne[2] != 1 || t.ne[3] != 1) {
            ulspec_model_destroy(m);
            return fail(ctx, ULSPEC_EINVAL, "model_load_gguf: tensor '%s' has %u dimensions", t.name.c_str(), t.n_dims);
        }
        st = ulspec_model_set_tensor(m, t.name.c_str(), t.type, g->base + g->data_offset + t.offset, (size_t)t.nbytes,
                                     t.ne[0], t.ne[1], 0);
        if (st != ULSPEC_OK) {
            ulspec_model_destroy(m);
            return st;
        }
    }
    *out = m;
    return ULSPEC_OK;
}
