// host_common.cpp -- host-only pieces every part of the library shares: the thread-local error
// message behind smx_last_error and the block geometry of each weight type.  No HIP calls, so
// the file parsers (gguf.cpp, smq.cpp) can also be built on their own with host sanitizers.
#include <cstdint>

#include "smx_internal.h"

namespace smx {

static thread_local std::string g_err;
void set_error(const std::string &msg) { g_err = msg; }
const char *last_error() { return g_err.c_str(); }

int type_block_elems(int type)
{
    switch (type) {
    case SMX_TYPE_F32: case SMX_TYPE_F16: return 1;
    case SMX_TYPE_Q4_0: case SMX_TYPE_Q8_0: case SMX_TYPE_SMQ_Q8: case SMX_TYPE_SMQ_Q4: return 32;
    case SMX_TYPE_Q4_K: case SMX_TYPE_Q5_K: case SMX_TYPE_Q6_K: return 256;
    default: return 0;
    }
}

int type_block_bytes(int type)
{
    switch (type) {
    case SMX_TYPE_F32: return 4;
    case SMX_TYPE_F16: return 2;
    case SMX_TYPE_Q4_0: return 18;
    case SMX_TYPE_Q8_0: return 34;
    case SMX_TYPE_Q4_K: return 144;
    case SMX_TYPE_Q5_K: return 176;
    case SMX_TYPE_Q6_K: return 210;
    case SMX_TYPE_SMQ_Q8: return 36;
    case SMX_TYPE_SMQ_Q4: return 20;
    default: return 0;
    }
}

}  // namespace smx

extern "C" {

SMX_API const char *smx_last_error(void) { return smx::last_error(); }
SMX_API int smx_type_block_elems(int type) { return smx::type_block_elems(type); }
SMX_API int smx_type_block_bytes(int type) { return smx::type_block_bytes(type); }

SMX_API int64_t smx_type_row_bytes(int type, int64_t k)
{
    const int be = smx::type_block_elems(type);
    if (!be || k < 0 || k % be) return -1;
    const int64_t blocks = k / be, bb = smx::type_block_bytes(type);
    if (blocks > INT64_MAX / bb) return -1;   // not representable: no such row
    return blocks * bb;
}

}  // extern "C"
