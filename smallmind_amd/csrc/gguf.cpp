// gguf.cpp -- GGUF v2/v3 model files: header, metadata and tensor table parsed from a
// read-only memory map, the model configuration derived from the metadata, and every tensor
// uploaded through smx_model_upload_tensor straight from the mapping (no host copy).
//
// Format (GgufReader.ReadModelInfo, GgufReader.cs:39-102): "GGUF", u32 version (2..3),
// u64 tensor count, u64 metadata count, metadata entries (GGUF string key, u32 value type,
// value), tensor entries (name, u32 n_dims, u64 dims[n_dims] fastest first, u32 type,
// u64 offset), then the data section at the next multiple of general.alignment (default 32).
// Tensor data sits at data section + the entry's offset, as the GGUF specification and
// llama.cpp's writer lay it out.  (GgufReader instead re-derives the offsets as a running sum
// of tensor sizes, GgufReader.cs:94-100, which agrees only when no tensor needs alignment
// padding; the files written by smallmind_amd.gguf.write_gguf satisfy both readings when every
// tensor size is a multiple of the alignment.)
//
// Configuration (ModelConfig.FromGgufMetadata, ModelConfig.cs:142-214): general.architecture
// (llama, or mistral* / phi* read with llama keys, or gpt2), then under that prefix
// vocab_size (else the tokenizer.ggml.tokens array length, else token_embd.weight's rows),
// context_length, embedding_length, block_count, attention.head_count (required),
// attention.head_count_kv (default head_count), feed_forward_length (default 4 d),
// rope.freq_base (default 10000), attention.layer_norm_rms_epsilon or
// attention.layer_norm_epsilon (default 1e-5).
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "smx_internal.h"

using namespace smx;

namespace {

#define GG_FAIL(code, ...)                        \
    do {                                          \
        char _b[512];                             \
        snprintf(_b, sizeof(_b), __VA_ARGS__);    \
        set_error(_b);                            \
        return (code);                            \
    } while (0)

enum GgType : uint32_t {
    GG_U8 = 0, GG_I8 = 1, GG_U16 = 2, GG_I16 = 3, GG_U32 = 4, GG_I32 = 5, GG_F32 = 6, GG_BOOL = 7,
    GG_STRING = 8, GG_ARRAY = 9, GG_U64 = 10, GG_I64 = 11, GG_F64 = 12
};

struct GgValue {
    enum Kind { NONE, INT, FLOAT, STRING, ARRAY } kind = NONE;
    int64_t i = 0;
    double f = 0.0;
    std::string s;
    uint64_t count = 0;   // array length
};

struct GgTensor {
    std::string name;
    std::vector<int64_t> dims;
    uint32_t type = 0;
    uint64_t offset = 0;
};

struct GgFile {
    uint32_t version = 0;
    std::map<std::string, GgValue> meta;
    std::vector<GgTensor> tensors;
    uint64_t data_off = 0;
};

// Bounds-checked little-endian cursor over the mapping.
struct Cur {
    const uint8_t *p;
    uint64_t n, at = 0;
    bool ok = true;
    bool need(uint64_t k)
    {
        if (!ok || k > n - at) ok = false;
        return ok;
    }
    template <typename T>
    T get()
    {
        T v{};
        if (need(sizeof(T))) {
            memcpy(&v, p + at, sizeof(T));
            at += sizeof(T);
        }
        return v;
    }
    std::string str()
    {
        const uint64_t len = get<uint64_t>();
        if (!need(len)) return std::string();
        std::string s((const char *)p + at, (size_t)len);
        at += len;
        return s;
    }
};

uint64_t scalar_bytes(uint32_t t)
{
    switch (t) {
    case GG_U8: case GG_I8: case GG_BOOL: return 1;
    case GG_U16: case GG_I16: return 2;
    case GG_U32: case GG_I32: case GG_F32: return 4;
    case GG_U64: case GG_I64: case GG_F64: return 8;
    default: return 0;
    }
}

bool read_scalar(Cur &c, uint32_t t, GgValue &v)
{
    switch (t) {
    case GG_U8: v.kind = GgValue::INT; v.i = c.get<uint8_t>(); break;
    case GG_I8: v.kind = GgValue::INT; v.i = c.get<int8_t>(); break;
    case GG_U16: v.kind = GgValue::INT; v.i = c.get<uint16_t>(); break;
    case GG_I16: v.kind = GgValue::INT; v.i = c.get<int16_t>(); break;
    case GG_U32: v.kind = GgValue::INT; v.i = c.get<uint32_t>(); break;
    case GG_I32: v.kind = GgValue::INT; v.i = c.get<int32_t>(); break;
    case GG_U64: v.kind = GgValue::INT; v.i = (int64_t)c.get<uint64_t>(); break;
    case GG_I64: v.kind = GgValue::INT; v.i = c.get<int64_t>(); break;
    case GG_BOOL: v.kind = GgValue::INT; v.i = c.get<uint8_t>() != 0; break;
    case GG_F32: v.kind = GgValue::FLOAT; v.f = c.get<float>(); break;
    case GG_F64: v.kind = GgValue::FLOAT; v.f = c.get<double>(); break;
    case GG_STRING: v.kind = GgValue::STRING; v.s = c.str(); break;
    default: return false;
    }
    return c.ok;
}

// Metadata value; arrays keep only their length (tokenizer tables are skipped over).
bool read_value(Cur &c, uint32_t t, GgValue &v)
{
    if (t != GG_ARRAY) return read_scalar(c, t, v);
    const uint32_t et = c.get<uint32_t>();
    const uint64_t count = c.get<uint64_t>();
    if (!c.ok) return false;
    v.kind = GgValue::ARRAY;
    v.count = count;
    if (et == GG_STRING) {
        for (uint64_t i = 0; i < count && c.ok; i++) {
            const uint64_t len = c.get<uint64_t>();
            if (c.need(len)) c.at += len;
        }
        return c.ok;
    }
    const uint64_t eb = scalar_bytes(et);
    if (!eb || count > (c.n - c.at) / eb) return false;   // nested arrays are not GGUF metadata
    c.at += count * eb;
    return true;
}

int parse(const uint8_t *p, uint64_t n, GgFile &f)
{
    Cur c{p, n};
    if (n < 4 || memcmp(p, "GGUF", 4) != 0) GG_FAIL(SMX_EINVAL, "gguf: bad magic (not a GGUF file)");
    c.at = 4;
    f.version = c.get<uint32_t>();
    if (f.version < 2 || f.version > 3) GG_FAIL(SMX_EUNSUPPORTED, "gguf: version %u not supported (2..3)", f.version);
    const uint64_t n_tensors = c.get<uint64_t>(), n_kv = c.get<uint64_t>();
    if (!c.ok || n_tensors > (1u << 20) || n_kv > (1u << 24)) GG_FAIL(SMX_EINVAL, "gguf: bad header counts");
    for (uint64_t i = 0; i < n_kv; i++) {
        std::string key = c.str();
        const uint32_t t = c.get<uint32_t>();
        GgValue v;
        if (!c.ok || !read_value(c, t, v)) GG_FAIL(SMX_EINVAL, "gguf: bad metadata entry %llu (type %u)", (unsigned long long)i, t);
        f.meta[key] = v;
    }
    for (uint64_t i = 0; i < n_tensors; i++) {
        GgTensor t;
        t.name = c.str();
        const uint32_t nd = c.get<uint32_t>();
        if (!c.ok || nd < 1 || nd > 4) GG_FAIL(SMX_EINVAL, "gguf: tensor %llu has %u dims", (unsigned long long)i, nd);
        for (uint32_t k = 0; k < nd; k++) t.dims.push_back((int64_t)c.get<uint64_t>());
        t.type = c.get<uint32_t>();
        t.offset = c.get<uint64_t>();
        if (!c.ok) GG_FAIL(SMX_EINVAL, "gguf: truncated tensor table");
        f.tensors.push_back(std::move(t));
    }
    uint64_t align = 32;
    auto it = f.meta.find("general.alignment");
    if (it != f.meta.end() && it->second.kind == GgValue::INT) align = (uint64_t)it->second.i;
    if (align == 0 || (align & (align - 1))) GG_FAIL(SMX_EINVAL, "gguf: alignment %llu is not a power of two", (unsigned long long)align);
    f.data_off = (c.at + align - 1) / align * align;
    return SMX_OK;
}

const GgValue *meta(const GgFile &f, const std::string &k)
{
    auto it = f.meta.find(k);
    return it == f.meta.end() ? nullptr : &it->second;
}

bool meta_int(const GgFile &f, const std::string &k, int64_t &out)
{
    const GgValue *v = meta(f, k);
    if (!v) return false;
    if (v->kind == GgValue::INT) { out = v->i; return true; }
    if (v->kind == GgValue::FLOAT) { out = (int64_t)v->f; return true; }
    return false;
}

bool meta_float(const GgFile &f, const std::string &k, double &out)
{
    const GgValue *v = meta(f, k);
    if (!v) return false;
    if (v->kind == GgValue::FLOAT) { out = v->f; return true; }
    if (v->kind == GgValue::INT) { out = (double)v->i; return true; }
    return false;
}

int config_from_meta(const GgFile &f, smx_model_config &cfg)
{
    memset(&cfg, 0, sizeof(cfg));
    std::string arch = "llama";
    if (const GgValue *a = meta(f, "general.architecture"); a && a->kind == GgValue::STRING) arch = a->s;
    std::string pre = arch;
    if (arch.rfind("mistral", 0) == 0 || arch.rfind("phi", 0) == 0) pre = "llama";
    if (pre == "llama") cfg.arch = SMX_ARCH_LLAMA;
    else if (pre == "gpt2") cfg.arch = SMX_ARCH_GPT2;
    else GG_FAIL(SMX_EUNSUPPORTED, "gguf: unsupported architecture '%s' (llama, mistral, phi, gpt2)", arch.c_str());
    int64_t v = 0;
    auto req = [&](const char *key, int32_t &dst) -> int {
        if (!meta_int(f, pre + "." + key, v) || v <= 0 || v > INT32_MAX)
            GG_FAIL(SMX_EINVAL, "gguf: missing or invalid metadata %s.%s", pre.c_str(), key);
        dst = (int32_t)v;
        return SMX_OK;
    };
    int rc;
    if ((rc = req("context_length", cfg.ctx)) || (rc = req("embedding_length", cfg.d_model)) ||
        (rc = req("block_count", cfg.n_layer)) || (rc = req("attention.head_count", cfg.n_head)))
        return rc;
    cfg.n_kv_head = meta_int(f, pre + ".attention.head_count_kv", v) && v > 0 ? (int32_t)v : cfg.n_head;
    cfg.d_ff = meta_int(f, pre + ".feed_forward_length", v) && v > 0 ? (int32_t)v : 4 * cfg.d_model;
    if (meta_int(f, pre + ".vocab_size", v) && v > 0) {
        cfg.vocab = (int32_t)v;
    } else if (const GgValue *tok = meta(f, "tokenizer.ggml.tokens"); tok && tok->kind == GgValue::ARRAY && tok->count) {
        cfg.vocab = (int32_t)tok->count;   // InferVocabSizeFromTokenizer
    } else {
        for (const GgTensor &t : f.tensors)
            if (t.name == "token_embd.weight" && t.dims.size() == 2) cfg.vocab = (int32_t)t.dims[1];
        if (!cfg.vocab) GG_FAIL(SMX_EINVAL, "gguf: no vocab_size, tokenizer table or token_embd.weight");
    }
    double d = 0.0;
    cfg.rope_theta = meta_float(f, pre + ".rope.freq_base", d) ? (float)d : 10000.0f;
    cfg.norm_eps = meta_float(f, pre + ".attention.layer_norm_rms_epsilon", d) ? (float)d
                 : meta_float(f, pre + ".attention.layer_norm_epsilon", d) ? (float)d : 1e-5f;
    return SMX_OK;
}

// Byte size of a tensor of `type` with GGUF dims; 0 if the type has no known layout, a
// dimension is not positive, or the size does not fit 64 bits (the products are checked, so a
// corrupt table cannot wrap to a size that passes the file-bounds check).
uint64_t tensor_bytes(uint32_t type, const std::vector<int64_t> &dims)
{
    uint64_t rows = 1;
    for (size_t k = 1; k < dims.size(); k++) {
        if (dims[k] <= 0 || rows > UINT64_MAX / (uint64_t)dims[k]) return 0;
        rows *= (uint64_t)dims[k];
    }
    const int64_t rb = smx_type_row_bytes((int)type, dims[0]);
    if (rb <= 0 || (uint64_t)rb > UINT64_MAX / rows) return 0;
    return (uint64_t)rb * rows;
}

struct Mapping {
    int fd = -1;
    void *p = MAP_FAILED;
    uint64_t n = 0;
    ~Mapping()
    {
        if (p != MAP_FAILED) munmap(p, n);
        if (fd >= 0) close(fd);
    }
    int open_file(const char *path)
    {
        fd = open(path, O_RDONLY);
        if (fd < 0) GG_FAIL(SMX_EINVAL, "gguf: cannot open '%s'", path);
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) GG_FAIL(SMX_EINVAL, "gguf: cannot stat '%s' or empty file", path);
        n = (uint64_t)st.st_size;
        p = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) GG_FAIL(SMX_EINVAL, "gguf: cannot map '%s'", path);
        return SMX_OK;
    }
};

// Tensors a llama.cpp GGUF may carry that this model does not use.
bool ignorable(const std::string &name) { return name == "rope_freqs.weight"; }

}  // namespace

SMX_API int smx_gguf_read_config(const char *path, smx_model_config *cfg, int64_t *n_tensors)
{
    if (!path || !cfg) GG_FAIL(SMX_EINVAL, "smx_gguf_read_config: null argument");
    Mapping mp;
    int rc = mp.open_file(path);
    if (rc) return rc;
    GgFile f;
    if ((rc = parse((const uint8_t *)mp.p, mp.n, f))) return rc;
    if ((rc = config_from_meta(f, *cfg))) return rc;
    if (n_tensors) *n_tensors = (int64_t)f.tensors.size();
    return SMX_OK;
}

SMX_API int smx_model_load_gguf(smx_context *ctx, const char *path, smx_model **out)
{
    if (!ctx || !path || !out) GG_FAIL(SMX_EINVAL, "smx_model_load_gguf: null argument");
    *out = nullptr;
    Mapping mp;
    int rc = mp.open_file(path);
    if (rc) return rc;
    GgFile f;
    if ((rc = parse((const uint8_t *)mp.p, mp.n, f))) return rc;
    smx_model_config cfg;
    if ((rc = config_from_meta(f, cfg))) return rc;
    // every tensor's bytes lie inside the file before anything is allocated
    for (const GgTensor &t : f.tensors) {
        const uint64_t nb = tensor_bytes(t.type, t.dims);
        if (!nb && !ignorable(t.name))
            GG_FAIL(SMX_EUNSUPPORTED, "gguf: %s: tensor type %u with ne0=%lld is not supported", t.name.c_str(),
                    t.type, (long long)t.dims[0]);
        if (t.offset > mp.n || f.data_off > mp.n - t.offset || nb > mp.n - f.data_off - t.offset)
            GG_FAIL(SMX_EINVAL, "gguf: %s: data [%llu, +%llu) outside the file", t.name.c_str(),
                    (unsigned long long)(f.data_off + t.offset), (unsigned long long)nb);
    }
    smx_model *m = nullptr;
    if ((rc = smx_model_create(ctx, &cfg, &m))) return rc;
    for (const GgTensor &t : f.tensors) {
        if (ignorable(t.name)) continue;
        const uint8_t *src = (const uint8_t *)mp.p + f.data_off + t.offset;
        rc = smx_model_upload_tensor(m, t.name.c_str(), (int)t.type, t.dims.data(), (int)t.dims.size(), src,
                                     (size_t)tensor_bytes(t.type, t.dims), 0);
        if (rc) {
            const std::string msg = last_error();
            smx_model_destroy(m);
            set_error(msg);
            return rc;
        }
    }
    if ((rc = smx_model_finalize(m))) {
        const std::string msg = last_error();
        smx_model_destroy(m);
        set_error(msg);
        return rc;
    }
    *out = m;
    return SMX_OK;
}
