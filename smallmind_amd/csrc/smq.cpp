// smq.cpp -- SmallMind's own .smq model files: header, JSON metadata and tensor directory parsed
// from a read-only memory map, every tensor re-laid for upload without rounding and uploaded
// through smx_model_upload_tensor.
//
// Format (SmqFormat.cs:15-121, SmqReader.cs:33-232): "SMQv0001", u32 version (1), u32 header
// size (32), u32 tensor count, u32 metadata JSON length, u64 reserved; the UTF-8 JSON metadata;
// then one 156-byte entry per tensor: name (64 bytes, NUL-padded), u32 data type (QuantScheme.cs:
// F32 = 1, Q8_0 = 10, Q4_0 = 11), i32 rank, i32 dims[8], u32 block size, u64 data offset, u64
// data length, u64 aux offset, u64 aux length, 16 reserved bytes.  F32 data is rank-any floats;
// Q8 (Q8Tensor) is one int8 per element, Q4 (Q4Tensor) two elements per byte (element 2i in the
// low nibble, two's complement), both rank 2 [rows][cols] with one fp32 scale per block of
// `block size` consecutive elements of the flattened tensor (the aux data).
//
// The model (SmqModelLoader.LoadFromSmq, SmqModelLoader.cs:22-100) is SmallMind's GPT-2 style
// TransformerModel (TransformerModel.cs:81-157: learned positions, LayerNorm, GELU MLP of 4 d,
// biases).  Tensors are matched by TransformerModel.GetNamedParameters names
// (TransformerModel.cs:545-728: token_embd.weight, pos_embd.weight, blk.N.attn_norm.*,
// blk.N.attn_qkv.*, blk.N.attn_output.*, blk.N.ffn_norm.*, blk.N.ffn_up.*, blk.N.ffn_down.*,
// output_norm.*, output.weight); a file none of whose names matches -- the quantize command and
// the benchmark-model tool name them param_NNNN / tensor_NNN in parameter order
// (QuantizeCommand.cs:63-97, CreateBenchmarkModel/Program.cs) -- is mapped by that order
// (TransformerModel.cs:132-144, TransformerBlock.cs:64-72, MultiHeadAttention.cs:114-115,
// MLP.cs:32-33, NeuralNet.cs:70-75, :674-675).  One-dimensional tensors (norm weights, biases)
// are dequantized on the host as SmqModelLoader.DequantizeTensor does (SmqModelLoader.cs:320-360);
// weight matrices stay quantized on the device (SQ8 / SQ4, exact scales) or F32.
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cctype>
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <vector>

#include "smx_internal.h"

using namespace smx;

namespace {

#define SQ_FAIL(code, ...)                        \
    do {                                          \
        char _b[512];                             \
        snprintf(_b, sizeof(_b), __VA_ARGS__);    \
        set_error(_b);                            \
        return (code);                            \
    } while (0)

// QuantScheme ids of the SMQ directory (src/SmallMind.Quantization/Tensors/QuantScheme.cs)
constexpr uint32_t kSmqF32 = 1, kSmqF16 = 2, kSmqQ8 = 10, kSmqQ4 = 11;
constexpr uint32_t kEntryBytes = 156, kHeaderBytes = 32;

struct SmqEntry {
    std::string name;
    uint32_t type = 0, block = 0;
    std::vector<int64_t> dims;   // as stored: dims[0] = rows
    uint64_t data_off = 0, data_len = 0, aux_off = 0, aux_len = 0;
    // element count, or -1 when it exceeds 2^60 (so that the byte sizes derived from it, at
    // most 4 bytes per element, cannot wrap)
    int64_t elems() const
    {
        int64_t n = 1;
        for (int64_t d : dims) {
            if (d <= 0 || n > (INT64_C(1) << 60) / d) return -1;
            n *= d;
        }
        return n;
    }
};

struct SmqFile {
    std::string meta;
    std::vector<SmqEntry> tensors;
};

uint32_t rd32(const uint8_t *p) { return (uint32_t)p[0] | ((uint32_t)p[1] << 8) | ((uint32_t)p[2] << 16) | ((uint32_t)p[3] << 24); }
uint64_t rd64(const uint8_t *p) { return (uint64_t)rd32(p) | ((uint64_t)rd32(p + 4) << 32); }

// Directory and size checks of SmqReader (SmqReader.cs:33-75, :153-293).
int parse(const uint8_t *p, uint64_t n, SmqFile &f)
{
    if (n < kHeaderBytes || memcmp(p, "SMQv0001", 8) != 0) SQ_FAIL(SMX_EINVAL, "smq: bad magic (expected 'SMQv0001')");
    if (rd32(p + 8) != 1) SQ_FAIL(SMX_EUNSUPPORTED, "smq: format version %u", rd32(p + 8));
    if (rd32(p + 12) != kHeaderBytes) SQ_FAIL(SMX_EINVAL, "smq: header size %u", rd32(p + 12));
    const uint64_t count = rd32(p + 16), mlen = rd32(p + 20);
    if (mlen > n - kHeaderBytes) SQ_FAIL(SMX_EINVAL, "smq: metadata past the end of the file");
    f.meta.assign((const char *)p + kHeaderBytes, (size_t)mlen);
    const uint64_t dir = kHeaderBytes + mlen;
    if (count > (n - dir) / kEntryBytes) SQ_FAIL(SMX_EINVAL, "smq: tensor directory past the end of the file");
    for (uint64_t i = 0; i < count; i++) {
        const uint8_t *e = p + dir + i * kEntryBytes;
        SmqEntry t;
        size_t nl = 0;
        while (nl < 64 && e[nl]) nl++;
        t.name.assign((const char *)e, nl);
        t.type = rd32(e + 64);
        const int32_t rank = (int32_t)rd32(e + 68);
        if (rank < 0 || rank > 8) SQ_FAIL(SMX_EINVAL, "smq: %s: rank %d", t.name.c_str(), rank);
        for (int k = 0; k < rank; k++) {
            const int32_t d = (int32_t)rd32(e + 72 + 4 * k);
            if (d <= 0) SQ_FAIL(SMX_EINVAL, "smq: %s: dimension %d", t.name.c_str(), d);
            t.dims.push_back(d);
        }
        t.block = rd32(e + 104);
        t.data_off = rd64(e + 108);
        t.data_len = rd64(e + 116);
        t.aux_off = rd64(e + 124);
        t.aux_len = rd64(e + 132);
        if (t.elems() < 0) SQ_FAIL(SMX_EINVAL, "smq: %s: too many elements", t.name.c_str());
        const uint64_t ne = (uint64_t)t.elems();
        if (t.type == kSmqF32) {
            if (t.data_len != ne * 4 || t.aux_len != 0) SQ_FAIL(SMX_EINVAL, "smq: %s: F32 sizes", t.name.c_str());
        } else if (t.type == kSmqQ8 || t.type == kSmqQ4) {
            if (rank != 2) SQ_FAIL(SMX_EINVAL, "smq: %s: quantized tensors are rank 2, got %d", t.name.c_str(), rank);
            if (t.block == 0) SQ_FAIL(SMX_EINVAL, "smq: %s: block size 0", t.name.c_str());
            const uint64_t want = t.type == kSmqQ8 ? ne : (ne + 1) / 2;
            const uint64_t nblk = (ne + t.block - 1) / t.block;
            if (t.data_len != want || t.aux_len != nblk * 4)
                SQ_FAIL(SMX_EINVAL, "smq: %s: data %llu / aux %llu bytes, expected %llu / %llu", t.name.c_str(),
                        (unsigned long long)t.data_len, (unsigned long long)t.aux_len, (unsigned long long)want,
                        (unsigned long long)(nblk * 4));
        } else if (t.type == kSmqF16) {
            SQ_FAIL(SMX_EUNSUPPORTED, "smq: %s: F16 tensors are not read by SmqReader", t.name.c_str());
        } else {
            SQ_FAIL(SMX_EUNSUPPORTED, "smq: %s: data type %u", t.name.c_str(), t.type);
        }
        if (t.data_off > n || t.data_len > n - t.data_off || t.aux_off > n || t.aux_len > n - t.aux_off)
            SQ_FAIL(SMX_EINVAL, "smq: %s: data outside the file", t.name.c_str());
        f.tensors.push_back(std::move(t));
    }
    return SMX_OK;
}

// Integer value of a top-level JSON key (a number or a string holding one), or -1.
int64_t meta_int(const std::string &js, const char *key)
{
    const std::string k = std::string("\"") + key + "\"";
    size_t at = js.find(k);
    if (at == std::string::npos) return -1;
    at = js.find(':', at + k.size());
    if (at == std::string::npos) return -1;
    at++;
    while (at < js.size() && (isspace((unsigned char)js[at]) || js[at] == '"')) at++;
    if (at >= js.size() || !isdigit((unsigned char)js[at])) return -1;
    return strtoll(js.c_str() + at, nullptr, 10);
}

// The GPT-2 style configuration the metadata describes (CreateBenchmarkModel/Program.cs,
// QuantizeCommand.cs:99-110 write vocab_size, block_size, embed_dim, num_heads, num_layers).
int config_from_meta(const std::string &js, smx_model_config &c)
{
    memset(&c, 0, sizeof(c));
    c.arch = SMX_ARCH_GPT2;
    c.vocab = (int32_t)meta_int(js, "vocab_size");
    c.ctx = (int32_t)meta_int(js, "block_size");
    c.d_model = (int32_t)meta_int(js, "embed_dim");
    c.n_layer = (int32_t)meta_int(js, "num_layers");
    c.n_head = (int32_t)meta_int(js, "num_heads");
    if (c.vocab <= 0 || c.ctx <= 0 || c.d_model <= 0 || c.n_layer <= 0 || c.n_head <= 0)
        SQ_FAIL(SMX_EINVAL, "smq: metadata lacks vocab_size / block_size / embed_dim / num_layers / num_heads");
    c.n_kv_head = c.n_head;
    c.d_ff = 4 * c.d_model;     // MLP.cs:25-26
    c.rope_theta = 10000.0f;
    c.norm_eps = 1e-5f;         // LayerNorm default (NeuralNet.cs:667)
    return SMX_OK;
}

// The GPT-2 TransformerModel's parameters in registration order, under the upload names.
std::vector<std::string> parameter_order(int n_layer)
{
    std::vector<std::string> v = {"token_embd.weight", "position_embd.weight"};
    static const char *blk[] = {"attn_norm.weight", "attn_norm.bias", "attn_qkv.weight", "attn_qkv.bias",
                                "attn_output.weight", "attn_output.bias", "ffn_norm.weight", "ffn_norm.bias",
                                "ffn_up.weight", "ffn_up.bias", "ffn_down.weight", "ffn_down.bias"};
    for (int l = 0; l < n_layer; l++)
        for (const char *b : blk) v.push_back("blk." + std::to_string(l) + "." + b);
    v.push_back("output_norm.weight");
    v.push_back("output_norm.bias");
    v.push_back("output.weight");
    return v;
}

// GetNamedParameters name -> upload name (only pos_embd differs), or "" if not a parameter.
std::string upload_name(const std::string &n, int n_layer)
{
    if (n == "pos_embd.weight") return "position_embd.weight";
    for (const std::string &p : parameter_order(n_layer))
        if (p == n && p != "position_embd.weight") return n;
    return "";
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
        if (fd < 0) SQ_FAIL(SMX_EINVAL, "smq: cannot open '%s'", path);
        struct stat st;
        if (fstat(fd, &st) != 0 || st.st_size <= 0) SQ_FAIL(SMX_EINVAL, "smq: cannot stat '%s' or empty file", path);
        n = (uint64_t)st.st_size;
        p = mmap(nullptr, n, PROT_READ, MAP_PRIVATE, fd, 0);
        if (p == MAP_FAILED) SQ_FAIL(SMX_EINVAL, "smq: cannot map '%s'", path);
        return SMX_OK;
    }
};

float code_q4(const uint8_t *data, int64_t i)
{
    const uint32_t nib = (data[i >> 1] >> (4 * (i & 1))) & 15u;
    return (float)(nib < 8 ? (int)nib : (int)nib - 16);   // Q4Tensor.DecodeNibble (Q4Tensor.cs:140-143)
}

}  // namespace

extern "C" {

SMX_API int smx_smq_pack(int type, const void *data, const float *scales, int64_t rows, int64_t cols, int block_size,
                         void *out, size_t out_bytes)
{
    if (type != SMX_TYPE_SMQ_Q8 && type != SMX_TYPE_SMQ_Q4) SQ_FAIL(SMX_EUNSUPPORTED, "smx_smq_pack: type %d", type);
    if (!data || !scales || !out || rows <= 0 || cols <= 0 || block_size <= 0)
        SQ_FAIL(SMX_EINVAL, "smx_smq_pack: bad arguments");
    // every 32-element chunk of a row must lie inside one SMQ block of the flattened tensor
    if (cols % 32 != 0 || block_size % 32 != 0)
        SQ_FAIL(SMX_EUNSUPPORTED, "smx_smq_pack: cols %lld and block size %d must be multiples of 32", (long long)cols,
                block_size);
    if (rows > (INT64_C(1) << 58) / cols)   // the byte counts below stay far inside 64 bits
        SQ_FAIL(SMX_EINVAL, "smx_smq_pack: %lld x %lld elements is too large", (long long)rows, (long long)cols);
    const bool q8 = type == SMX_TYPE_SMQ_Q8;
    const int64_t nchunk = rows * cols / 32;
    const size_t bb = q8 ? 36 : 20;
    if (out_bytes != (size_t)nchunk * bb)
        SQ_FAIL(SMX_EINVAL, "smx_smq_pack: out_bytes %zu, expected %zu", out_bytes, (size_t)nchunk * bb);
    const uint8_t *src = (const uint8_t *)data;
    uint8_t *dst = (uint8_t *)out;
    for (int64_t k = 0; k < nchunk; k++) {
        const int64_t e0 = 32 * k;
        const float sc = scales[e0 / block_size];
        memcpy(dst + k * bb, &sc, 4);
        if (q8) memcpy(dst + k * bb + 4, src + e0, 32);
        else memcpy(dst + k * bb + 4, src + e0 / 2, 16);   // e0 even: whole bytes
    }
    return SMX_OK;
}

SMX_API int smx_smq_read_config(const char *path, smx_model_config *cfg, int64_t *n_tensors)
{
    if (!path || !cfg) SQ_FAIL(SMX_EINVAL, "smx_smq_read_config: null argument");
    Mapping mp;
    int rc = mp.open_file(path);
    if (rc) return rc;
    SmqFile f;
    if ((rc = parse((const uint8_t *)mp.p, mp.n, f))) return rc;
    if ((rc = config_from_meta(f.meta, *cfg))) return rc;
    if (n_tensors) *n_tensors = (int64_t)f.tensors.size();
    return SMX_OK;
}

SMX_API int smx_model_load_smq(smx_context *ctx, const char *path, const smx_model_config *cfg_in, smx_model **out)
{
    if (!ctx || !path || !out) SQ_FAIL(SMX_EINVAL, "smx_model_load_smq: null argument");
    *out = nullptr;
    Mapping mp;
    int rc = mp.open_file(path);
    if (rc) return rc;
    const uint8_t *base = (const uint8_t *)mp.p;
    SmqFile f;
    if ((rc = parse(base, mp.n, f))) return rc;
    smx_model_config cfg;
    if (cfg_in) {
        cfg = *cfg_in;
        if (cfg.arch != SMX_ARCH_GPT2)
            SQ_FAIL(SMX_EUNSUPPORTED, "smx_model_load_smq: SMQ models are SmallMind's GPT-2 style TransformerModel");
    } else if ((rc = config_from_meta(f.meta, cfg))) {
        return rc;
    }
    // names: GetNamedParameters names where any matches, else the parameter order
    std::vector<std::string> names(f.tensors.size());
    bool any_named = false;
    for (size_t i = 0; i < f.tensors.size(); i++) {
        names[i] = upload_name(f.tensors[i].name, cfg.n_layer);
        any_named = any_named || !names[i].empty();
    }
    if (!any_named) {
        const std::vector<std::string> order = parameter_order(cfg.n_layer);
        if (order.size() != f.tensors.size())
            SQ_FAIL(SMX_EINVAL, "smq: %zu tensors carry no parameter names and the model has %zu parameters",
                    f.tensors.size(), order.size());
        names = order;
    }
    smx_model *m = nullptr;
    if ((rc = smx_model_create(ctx, &cfg, &m))) return rc;
    auto fail = [&](int code) {
        const std::string msg = last_error();
        smx_model_destroy(m);
        set_error(msg);
        return code;
    };
    std::vector<uint8_t> buf;
    std::vector<float> vec;
    for (size_t i = 0; i < f.tensors.size(); i++) {
        const SmqEntry &t = f.tensors[i];
        if (names[i].empty()) continue;   // SmqModelLoader skips tensors with no matching parameter
        const int64_t ne = t.elems();
        const uint8_t *data = base + t.data_off;
        const float *scales = (const float *)(base + t.aux_off);
        std::vector<float> sc;
        if (t.type != kSmqF32) {   // the aux data need not be 4-byte aligned in the mapping
            sc.resize((size_t)(t.aux_len / 4));
            memcpy(sc.data(), base + t.aux_off, t.aux_len);
            scales = sc.data();
        }
        // norm weights and biases are 1-D parameters, stored as [1][n] by the SMQ writers
        const std::string &un = names[i];
        const bool one_d = un.find("norm") != std::string::npos ||
                           (un.size() > 5 && un.compare(un.size() - 5, 5, ".bias") == 0);
        if (one_d) {
            // SmqModelLoader.DequantizeTensor: code * scale (Q8Tensor.cs:131-157, Q4Tensor.cs:150-178)
            vec.resize((size_t)ne);
            for (int64_t e = 0; e < ne; e++) {
                if (t.type == kSmqF32) memcpy(&vec[(size_t)e], data + 4 * e, 4);
                else {
                    const float q = t.type == kSmqQ8 ? (float)(int8_t)data[e] : code_q4(data, e);
                    vec[(size_t)e] = q * scales[e / t.block];
                }
            }
            const int64_t dims[1] = {ne};
            rc = smx_model_upload_tensor(m, names[i].c_str(), SMX_TYPE_F32, dims, 1, vec.data(), vec.size() * 4, 0);
        } else {
            if (t.dims.size() != 2) {   // the model is created: release it with the error
                char b[512];
                snprintf(b, sizeof(b), "smq: %s: rank %zu matrix", t.name.c_str(), t.dims.size());
                set_error(b);
                return fail(SMX_EUNSUPPORTED);
            }
            const int64_t rows = t.dims[0], cols = t.dims[1];
            const int64_t gdims[2] = {cols, rows};   // upload dims: ne0 = cols
            if (t.type == kSmqF32) {
                rc = smx_model_upload_tensor(m, names[i].c_str(), SMX_TYPE_F32, gdims, 2, data, (size_t)t.data_len, 0);
            } else {
                const int type = t.type == kSmqQ8 ? SMX_TYPE_SMQ_Q8 : SMX_TYPE_SMQ_Q4;
                buf.resize((size_t)(rows * cols / 32) * (t.type == kSmqQ8 ? 36 : 20));
                rc = smx_smq_pack(type, data, scales, rows, cols, (int)t.block, buf.data(), buf.size());
                if (rc == SMX_OK)
                    rc = smx_model_upload_tensor(m, names[i].c_str(), type, gdims, 2, buf.data(), buf.size(), 0);
            }
        }
        if (rc) return fail(rc);
    }
    if ((rc = smx_model_finalize(m))) return fail(rc);
    *out = m;
    return SMX_OK;
}

}  // extern "C"
