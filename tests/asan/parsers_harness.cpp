// parsers_harness.cpp -- the GGUF and .smq file loaders (smallmind_amd/csrc/gguf.cpp, smq.cpp,
// host_common.cpp) built for the host alone, under AddressSanitizer, LeakSanitizer and UBSan,
// and driven over valid and corrupted files.
//
// The model entry points the loaders call after parsing (smx_model_create / upload_tensor /
// finalize / destroy, which need a GPU in the library) are replaced here by host versions:
// create allocates a heap object (so a failure path that drops a model shows up as a leak),
// upload checks the byte count against the type's block geometry and reads every source byte,
// finalize succeeds.  Everything before them -- the header, metadata and tensor-table cursors,
// the configuration, the SMQ re-layout and host dequantization -- is the library's own code.
//
//   parsers_harness FILE...                 each file through the four loader entry points;
//                                           one line per file: read/load return codes
//   parsers_harness --fuzz BASE N SEED TMP  N corrupted copies of BASE (truncations, byte
//                                           flips, extreme field values, repeated ranges)
//                                           written to TMP and loaded
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "../../include/smx.h"

struct smx_model {
    int64_t tensors = 0, bytes = 0;
};

static int64_t g_size_mismatch = 0;

extern "C" {

SMX_API int smx_model_create(smx_context *, const smx_model_config *cfg, smx_model **out)
{
    if (!cfg || !out) return SMX_EINVAL;
    *out = new smx_model();
    return SMX_OK;
}

SMX_API int smx_model_upload_tensor(smx_model *m, const char *name, int type, const int64_t *dims, int ndims,
                                    const void *bytes, size_t nbytes, int bytes_on_device)
{
    if (!m || !name || !dims || ndims < 1 || ndims > 4 || !bytes || bytes_on_device) return SMX_EINVAL;
    int64_t n = smx_type_row_bytes(type, dims[0]);
    for (int i = 1; i < ndims && n >= 0; i++) n = dims[i] >= 0 ? n * dims[i] : -1;
    if (n < 0 || (size_t)n != nbytes) {
        g_size_mismatch++;
        return SMX_EINVAL;
    }
    const volatile uint8_t *p = (const volatile uint8_t *)bytes;
    uint32_t acc = 0;
    for (size_t i = 0; i < nbytes; i++) acc += p[i];
    m->tensors++;
    m->bytes += (int64_t)nbytes + (acc & 0);
    return SMX_OK;
}

SMX_API int smx_model_finalize(smx_model *m) { return m ? SMX_OK : SMX_EINVAL; }

SMX_API int smx_model_destroy(smx_model *m)
{
    delete m;
    return SMX_OK;
}

}  // extern "C"

// Each entry point on one path; returns the four codes.
static void run_all(const char *path, int rc[4])
{
    smx_context *ctx = reinterpret_cast<smx_context *>(&rc[0]);   // passed through to create only
    smx_model_config cfg;
    int64_t n = 0;
    smx_model *m = nullptr;
    rc[0] = smx_gguf_read_config(path, &cfg, &n);
    rc[1] = smx_model_load_gguf(ctx, path, &m);
    if (rc[1] == SMX_OK) smx_model_destroy(m);
    m = nullptr;
    rc[2] = smx_smq_read_config(path, &cfg, &n);
    rc[3] = smx_model_load_smq(ctx, path, nullptr, &m);
    if (rc[3] == SMX_OK) smx_model_destroy(m);
}

static uint64_t g_rng;
static uint64_t next_u64()
{
    uint64_t z = (g_rng += 0x9E3779B97F4A7C15ull);   // splitmix64
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

static void corrupt(std::vector<uint8_t> &f)
{
    static const uint64_t extremes[] = {0ull, 1ull, 0x7Full, 0xFFull, 0x7FFFFFFFull, 0x80000000ull, 0xFFFFFFFFull,
                                        0x100000000ull, 0x7FFFFFFFFFFFFFFFull, 0xFFFFFFFFFFFFFFFFull};
    // most fields sit in the first bytes: bias edits towards the header, metadata and table
    const size_t span = f.size() < 4096 ? f.size() : (next_u64() % 4 ? 4096 : f.size());
    switch (next_u64() % 5) {
    case 0:   // truncate
        f.resize(next_u64() % (f.size() + 1));
        break;
    case 1: {   // flip 1-4 bytes
        const int k = 1 + (int)(next_u64() % 4);
        for (int i = 0; i < k && span; i++) f[next_u64() % span] ^= (uint8_t)(1 + next_u64() % 255);
        break;
    }
    case 2: {   // an extreme 4- or 8-byte value at any offset
        const size_t w = next_u64() % 2 ? 8 : 4;
        if (span >= w) {
            const uint64_t v = extremes[next_u64() % (sizeof(extremes) / sizeof(extremes[0]))];
            memcpy(f.data() + next_u64() % (span - w + 1), &v, w);
        }
        break;
    }
    case 3: {   // a random byte run
        if (span) {
            const size_t at = next_u64() % span, len = 1 + next_u64() % 64;
            for (size_t i = at; i < at + len && i < f.size(); i++) f[i] = (uint8_t)next_u64();
        }
        break;
    }
    default: {   // repeat a range (shifts every later field)
        if (span > 1) {
            const size_t at = next_u64() % span, len = 1 + next_u64() % 32;
            std::vector<uint8_t> ins(f.begin() + (long)at, f.begin() + (long)std::min(f.size(), at + len));
            f.insert(f.begin() + (long)at, ins.begin(), ins.end());
        }
        break;
    }
    }
}

int main(int argc, char **argv)
{
    if (argc >= 6 && !strcmp(argv[1], "--fuzz")) {
        FILE *in = fopen(argv[2], "rb");
        if (!in) return 2;
        std::vector<uint8_t> base;
        for (int c; (c = fgetc(in)) != EOF;) base.push_back((uint8_t)c);
        fclose(in);
        const long n = atol(argv[3]);
        g_rng = strtoull(argv[4], nullptr, 10);
        const std::string tmp = std::string(argv[5]) + "/fuzz.bin";
        long accepted = 0;
        for (long it = 0; it < n; it++) {
            std::vector<uint8_t> f = base;
            const int edits = 1 + (int)(next_u64() % 3);
            for (int e = 0; e < edits; e++) corrupt(f);
            FILE *o = fopen(tmp.c_str(), "wb");
            if (!o) return 2;
            if (!f.empty() && fwrite(f.data(), 1, f.size(), o) != f.size()) return 2;
            fclose(o);
            int rc[4];
            run_all(tmp.c_str(), rc);
            accepted += rc[1] == SMX_OK || rc[3] == SMX_OK;
        }
        printf("fuzz %s: %ld files, %ld loaded, size mismatches %lld\n", argv[2], n, accepted,
               (long long)g_size_mismatch);
        return 0;
    }
    for (int i = 1; i < argc; i++) {
        int rc[4];
        run_all(argv[i], rc);
        printf("%s %d %d %d %d\n", argv[i], rc[0], rc[1], rc[2], rc[3]);
    }
    printf("size mismatches %lld\n", (long long)g_size_mismatch);
    return 0;
}
