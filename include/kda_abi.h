/*
 * kda_abi.h -- C ABI of the MI355X (gfx950) KDA operator library.
 *
 * Plain C: POD argument structs, raw device pointers, element strides, and a
 * `void *` HIP stream. No torch, no HIP headers, so the library can be bound
 * from ctypes / cffi / another host language without a C++ toolchain.
 *
 * These entry points replace the reference's host->device launch seam:
 *
 *   kda_recurrent_launch  replaces LaunchKdaDecodeH16/H32/H64 and
 *                         LaunchKdaPrefillH4/H8
 *                         (sgl-glm53-ascend-ops/csrc/kda/recurrent/
 *                          kda_varlen_recurrent.h:94-98), with the argument
 *                         block KdaLaunchArgs (same file, :59-92), and the
 *                         prepared-input kernels behind prepared_recurrent
 *                         (csrc/kda/prepared_recurrent.cpp:592-602,676-708);
 *   kda_chunk_launch      replaces LaunchKdaVarlenChunk (declared at
 *                         csrc/kda/chunk/kda_varlen_chunk.h:143, defined at
 *                         kda_varlen_chunk_kernel.cpp:1641-1662), argument
 *                         block KdaChunkLaunchArgs (kda_varlen_chunk.h:120-141);
 *   kda_chunk_workspace_bytes  sizes the chunk op's scratch, the analogue of
 *                         kWorkspaceFloatsPerBlock (kda_varlen_chunk.h:79-116).
 *
 * Layout contract (same as the reference ops):
 *   token tensors   [T, H, D] contiguous (the leading batch dim of the torch
 *                   op's [1, T, H, D] is 1);
 *   beta / b        [T, H];
 *   state pool      logical [slots, H, K, V], K contiguous: element
 *                   (s, h, k, v) lives at
 *                   state[s*state_stride_slot + h*state_stride_head + v*D + k];
 *   slot 0          the padding row: read as a zero state, never written;
 *   cu_seqlens      int32 [N+1], non-decreasing, cu_seqlens[N] <= T;
 *   indices         int32 [N]; entries outside [0, num_slots) are treated as
 *                   slot 0 (the kernels never address outside the pool).
 *
 * With num_tokens == 0 the token pointers (q, k, v, gate, beta, out) may be
 * null: the requests still run, so a prefix tracked at length 0 receives the
 * request's initial state.
 *
 * All launches are asynchronous on `stream` and never synchronize the host.
 * Every function returns a KdaStatus (0 = success).
 */
#ifndef KDA_ABI_H
#define KDA_ABI_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define KDA_ABI_VERSION 2

typedef enum KdaStatus {
    KDA_OK = 0,
    KDA_ERR_INVALID_ARGUMENT = 1, /* null pointer, bad size, misalignment */
    KDA_ERR_UNSUPPORTED = 2,      /* a shape / dtype / mode with no kernel */
    KDA_ERR_LAUNCH = 3,           /* the HIP runtime refused the launch */
    KDA_ERR_WORKSPACE = 4,        /* workspace missing or too small */
    KDA_ERR_TOO_LARGE = 5         /* needs more scratch than kda_chunk_launch_noalloc holds */
} KdaStatus;

typedef enum KdaDType {
    KDA_BF16 = 0,
    KDA_F32 = 1
} KdaDType;

/* How the per-channel decay and beta arrive.
 *   RAW    gate = bf16 `a` [T,H,D], beta = bf16 logit `b` [T,H]; the kernel
 *          computes g = lower_bound * sigmoid(exp(A_log[h]) * (a + dt_bias)),
 *          beta = sigmoid(b), and L2-normalizes q and k (the sglang schema,
 *          kda_varlen_recurrent.cpp:257-265);
 *   LOG    gate = fp32 log decay g [T,H,D] (<= 0), beta = fp32 [T,H];
 *   DECAY  gate = fp32 multiplicative decay exp(g) [T,H,D], beta = fp32 [T,H]
 *          (the prepared_recurrent schema, prepared_recurrent.cpp:715-720);
 *          `out` is caller-owned and only the rows the requests cover are
 *          written (RAW and LOG also zero the rows no request covers). */
typedef enum KdaGateMode {
    KDA_GATE_RAW = 0,
    KDA_GATE_LOG = 1,
    KDA_GATE_DECAY = 2
} KdaGateMode;

typedef struct KdaRecurrentArgs {
    const void *q;        /* [T,H,D], qk_dtype */
    const void *k;        /* [T,H,D], qk_dtype */
    const void *v;        /* [T,H,D], v_dtype */
    const void *gate;     /* see KdaGateMode */
    const void *beta;     /* see KdaGateMode */
    const float *A_log;   /* [H], RAW only */
    const float *dt_bias; /* [H*D], RAW only */

    float *state;               /* pool base, see layout contract */
    int64_t state_stride_slot;  /* elements */
    int64_t state_stride_head;  /* elements */
    int64_t num_slots;

    const int32_t *state_indices; /* [N] */
    const int32_t *cu_seqlens;    /* [N+1] */
    void *out;                    /* [T,H,D], v_dtype; every token written (DECAY: covered rows only) */

    /* Per-step checkpoints [rows, steps, H, K, V], K contiguous (null = off).
     * Row = the request's position n, step = its local token index; written
     * after each step's update when slot > 0, and the final write-back to
     * the pool is then skipped (decode.h:45-49,683-708,743-751). */
    float *intermediate;
    int64_t mid_stride_req;  /* elements */
    int64_t mid_stride_step; /* elements */
    int64_t mid_stride_head; /* elements */
    int64_t mid_rows;
    int64_t mid_steps;

    /* Prefix tracking (null = off): slot track_indices[n] (> 0) receives the
     * state after track_lens[n] of the request's tokens; 0 = initial state. */
    const int32_t *track_indices; /* [N] */
    const int32_t *track_lens;    /* [N] */

    float scale;       /* multiplies q after the optional L2 norm */
    float lower_bound; /* RAW only */
    int32_t num_seqs;
    int32_t num_tokens;
    int32_t num_heads;   /* H: heads per token row and per pool slot */
    int32_t head_begin;  /* first head processed (0 = all from the start) */
    int32_t head_count;  /* heads processed from head_begin (0 = to H) */
    int32_t head_dim;    /* K == V; 64 or 128 */
    int32_t qk_dtype;  /* KdaDType */
    int32_t v_dtype;   /* KdaDType, also the output dtype */
    int32_t gate_mode; /* KdaGateMode */
    int32_t qk_l2norm; /* LOG mode: normalize q and k in the kernel */
    /* State pool layout: 0 = K contiguous (the layout contract above); 1 =
     * [K,V] contiguous, element (s, h, k, v) at
     * state[s*state_stride_slot + h*state_stride_head + k*D + v] (the
     * prepared_recurrent pool of the reference), read and written in place;
     * KDA_GATE_DECAY only (KDA_ERR_UNSUPPORTED with the other gate modes).
     * Checkpoints (`intermediate`) are K contiguous either way. */
    int32_t state_v_contiguous;
} KdaRecurrentArgs;

/* Fused recurrent (token-by-token) KDA over packed varlen sequences.
 * Alignment (KDA_ERR_INVALID_ARGUMENT otherwise): state and intermediate
 * bases 16 bytes with strides that are multiples of 4 elements; q and k 8
 * bytes (bf16) or 16 (fp32); gate 8 bytes (RAW) or 16. v and out may sit
 * anywhere: aligned ones move as vectors, others element by element. */
int kda_recurrent_launch(const KdaRecurrentArgs *args, void *stream);

typedef struct KdaChunkArgs {
    const void *q;        /* [T,H,D], qk_dtype */
    const void *k;        /* [T,H,D], qk_dtype */
    const void *v;        /* [T,H,D], v_dtype */
    const void *gate;     /* RAW: bf16 a; LOG: fp32 g  (DECAY is unsupported) */
    const void *beta;     /* RAW: bf16 b; LOG: fp32 beta */
    const float *A_log;   /* [H], RAW only */
    const float *dt_bias; /* [H*D], RAW only */

    float *state;
    int64_t state_stride_slot;
    int64_t state_stride_head;
    int64_t num_slots;

    const int32_t *state_indices; /* [N] */
    const int32_t *cu_seqlens;    /* [N+1]; any lengths (no multiple-of-64 rule) */
    void *out;                    /* [T,H,D], v_dtype */

    const int32_t *track_indices; /* [N] or null */
    const int32_t *track_lens;    /* [N] or null */

    float scale;
    float lower_bound;
    int32_t num_seqs;
    int32_t num_tokens;
    int32_t num_heads;
    int32_t head_dim;  /* 128 */
    int32_t qk_dtype;
    int32_t v_dtype;
    int32_t gate_mode;
    int32_t qk_l2norm;
} KdaChunkArgs;

/* Bytes of device scratch kda_chunk_launch needs to run these arguments at
 * full speed. An upper bound that depends only on T, N, H, D and the current
 * device's compute-unit count (no device reads): the chunk records (one per
 * possible chunk and head, or, for a single sequence of at least 16384 tokens
 * on at most 16 heads, a ring of two scan segments' records per head), the
 * tracking records and, when N == 1, the state carried between scan
 * segments. A single sequence that takes the affine form (at most 8 heads on
 * 256 CUs, at least 3 segments of 32 chunks or 2 of 64, at most 1 GiB in all) needs one
 * record per chunk, two fp32 outputs per token-head and 3 (P - 1) + 2 sets of
 * H fp32 128 x 128 states besides; with less than that but at least the other forms'
 * size, kda_chunk_launch runs those. */
size_t kda_chunk_workspace_bytes(int32_t num_tokens, int32_t num_seqs,
                                 int32_t num_heads, int32_t head_dim);

/* Chunked (chunk = 64 tokens) KDA over packed varlen sequences.
 * Decays (g <= 0) of any magnitude: the intra-chunk products factor
 * e^(G_i - G_j) as e^(G_i - a) e^(a - G_j) with the anchor a at the middle of
 * each 16-token block, which holds while any 8 consecutive tokens of a
 * channel decay by less than 2^125 (about 87 nat: always on the RAW path with
 * lower_bound >= -10.9, and for LOG gates g >= -10.9 per token). A chunk
 * with a steeper block forms those products element by element instead
 * (exact, to the same tolerance contract, and slower for that chunk).
 * `workspace`
 * must be 256-byte aligned device memory of kda_chunk_workspace_bytes(...)
 * bytes; its contents need no initialization. A single sequence (N == 1)
 * also runs with less: the scan then goes through windows of as many chunks
 * as the workspace holds records for (at least one chunk per head, else
 * KDA_ERR_WORKSPACE), each window prepared and then scanned on `stream`.
 * With the full workspace, a single sequence of at least 16384 tokens on at
 * most 16 heads runs in segments of about 256 chunks: each next segment is
 * prepared on a library-owned stream while the current one is scanned, forked
 * from and joined back on `stream` by events (graph-capture safe); a single
 * sequence on few heads that takes the affine form scans its P segments at
 * once (segment s > 0 from zero and from the identity) and combines them
 * (S_{s+1} = Phi_s S_s + Z_s, outputs corrected by O_t S_s), all on
 * `stream`. Several sequences with more (sequence, head) pairs than the
 * device's CUs / 4 run their scan on one persistent workgroup per CU, each
 * team of four taking several pairs, longest first (the chunk-index pass
 * orders them); results are those of a workgroup per pair.
 * Alignment
 * (KDA_ERR_INVALID_ARGUMENT otherwise): state 16 bytes with strides in
 * multiples of 4 elements; q, k, v and out 8 bytes; gate 8 (RAW) or 16. */
int kda_chunk_launch(const KdaChunkArgs *args, void *workspace,
                     size_t workspace_bytes, void *stream);

/* Bytes of the static device scratch behind kda_chunk_launch_noalloc. */
#define KDA_NOALLOC_SCRATCH_BYTES (64u * 1024u * 1024u)

/* kda_chunk_launch without a caller workspace and without any device
 * allocation. No counterpart in the reference: for callers that cannot
 * allocate (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc). The workspace is a static device array of
 * KDA_NOALLOC_SCRATCH_BYTES per GPU, held until the process ends; its address
 * on a device is resolved on the first call on that device. The array is part
 * of the chunk kernels' code object: it occupies its 64 MiB on every GPU where
 * this library's kernels are loaded, whether or not this entry point is
 * called. Several sequences
 * whose records do not fit it (at K = V = 128 roughly 1190 (chunk, head)
 * pairs, e.g. 2 x 2048 tokens on 32 heads) return KDA_ERR_TOO_LARGE; a
 * single sequence of any length runs in windows of the chunks it holds (the
 * small-workspace form of kda_chunk_launch: about 1190 / H chunks, 37 on 32
 * heads).
 * Results are those of kda_chunk_launch on the same arguments; no second
 * stream is used. Every call on one GPU shares that GPU's array (its
 * contents need no initialization, the last call's are left behind): calls
 * that overlap on one GPU -- concurrent streams, or host threads -- race, and
 * must be serialized by the caller. */
int kda_chunk_launch_noalloc(const KdaChunkArgs *args, void *stream);

/* Human-readable text of a KdaStatus. */
const char *kda_status_string(int status);

/* KDA_ABI_VERSION of the built library. */
int kda_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* KDA_ABI_H */
