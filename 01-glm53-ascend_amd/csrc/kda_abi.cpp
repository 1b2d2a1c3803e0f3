// kda_abi.cpp -- the non-kernel half of the C ABI (status text, version).

#include "kda_abi.h"

extern "C" const char *kda_status_string(int status) {
    switch (status) {
        case KDA_OK: return "ok";
        case KDA_ERR_INVALID_ARGUMENT: return "invalid argument (null pointer, size or alignment)";
        case KDA_ERR_UNSUPPORTED: return "unsupported shape, dtype or mode";
        case KDA_ERR_LAUNCH: return "HIP kernel launch failed";
        case KDA_ERR_WORKSPACE: return "workspace missing or too small";
        case KDA_ERR_TOO_LARGE:
            return "arguments need more scratch than kda_chunk_launch_noalloc's static buffer holds";
        default: return "unknown status";
    }
}

extern "C" int kda_abi_version(void) { return KDA_ABI_VERSION; }
