// kda_chunk.hip -- chunked KDA prefill for gfx950 (placeholder until the
// MFMA pipeline lands: the launcher reports the configuration unsupported).

#include <hip/hip_runtime.h>

#include "kda_abi.h"

extern "C" size_t kda_chunk_workspace_bytes(int32_t num_tokens, int32_t num_seqs,
                                            int32_t num_heads, int32_t head_dim) {
    (void)num_tokens;
    (void)num_seqs;
    (void)num_heads;
    (void)head_dim;
    return 0;
}

extern "C" int kda_chunk_launch(const KdaChunkArgs *args, void *workspace,
                                size_t workspace_bytes, void *stream) {
    (void)args;
    (void)workspace;
    (void)workspace_bytes;
    (void)stream;
    return KDA_ERR_UNSUPPORTED;
}
