// kda_torch_ops.cpp -- torch operator layer over the KDA C ABI (PyTorch-ROCm).
//
// Registers the reference's operator namespace `sgl_glm53_ascend` with its
// schemas unchanged, implemented on the CUDA dispatch key (HIP devices are
// "cuda" in PyTorch-ROCm):
//
//   kda_varlen_recurrent   schema of csrc/kda/recurrent/kda_varlen_recurrent.cpp:257-265
//   kda_varlen_chunk       schema of csrc/kda/chunk/kda_varlen_chunk.cpp:195-202
//   prepared_recurrent     schema of csrc/kda/prepared_recurrent.cpp:715-720
//   *_v2                   the reference's in-development twins
//                          (recurrent_v2/kda_varlen_recurrent_v2.cpp:226-233,
//                          chunk_v2/kda_varlen_chunk_v2.cpp:183-190), served by
//                          the same kernels
//
// plus the prepared-gate forms the measured configurations use
// (`kda_prepared_varlen_recurrent`, `kda_prepared_varlen_chunk`: q/k/v, fp32
// log decay g and fp32 beta).
//
// Each op validates what the kernels index against, in the reference's
// order and with its message text (callers match substrings, e.g.
// tests/integration/kda_ascendc_dispatch.py:52-58), narrows int64 metadata
// to int32 on the device, allocates the output, and enqueues one launch on the
// current stream. No host synchronization: unlike the reference chunk op
// (kda_varlen_chunk.cpp:130-143), ragged lengths are accepted, so cu_seqlens
// never has to be read back.

#include <ATen/ATen.h>
#include <c10/core/DeviceGuard.h>
#include <c10/hip/HIPStream.h>
#include <torch/library.h>

#include <algorithm>
#include <optional>
#include <string>
#include <utility>

#include "kda_abi.h"

namespace {

using NamedTensor = std::pair<const char *, const at::Tensor &>;

void check_same_device(const at::Tensor &q, const char *name, const at::Tensor &t) {
    TORCH_CHECK(t.device() == q.device(), name, " must be on the same device as q");
}

void check_ok(int status, const char *op) {
    TORCH_CHECK(status == KDA_OK, op, ": ", kda_status_string(status), " (status ", status, ")");
}

void *stream_of(const at::Tensor &t) {
    return static_cast<void *>(c10::hip::getCurrentHIPStream(t.device().index()).stream());
}

at::Tensor as_int32(const at::Tensor &t) {
    return t.scalar_type() == at::kInt ? t.contiguous() : t.to(at::kInt).contiguous();
}

std::optional<at::Tensor> as_int32_opt(const std::optional<at::Tensor> &t) {
    return t.has_value() ? std::optional<at::Tensor>(as_int32(*t)) : std::nullopt;
}

const int32_t *i32_ptr(const at::Tensor &t) { return t.data_ptr<int32_t>(); }

// One packed token batch [1, T, H, D] (the sglang contract; a leading batch
// above one would otherwise be ignored), with T and the request count in the
// kernels' int32 range.
void check_packed(const char *op, const at::Tensor &q, const at::Tensor &indices) {
    TORCH_CHECK(q.size(0) == 1, op, " expects one packed token batch [1, T, H, D], got batch ",
                q.size(0));
    TORCH_CHECK(q.size(1) <= INT32_MAX && indices.numel() < INT32_MAX, op,
                " supports at most 2^31-1 tokens and requests");
}

void check_gate_params(const at::Tensor &q, const at::Tensor &A_log, const at::Tensor &dt_bias,
                       int64_t HV, int64_t D) {
    TORCH_CHECK(A_log.scalar_type() == at::kFloat && A_log.numel() == HV,
                "A_log must be fp32 with HV elements");
    TORCH_CHECK(dt_bias.scalar_type() == at::kFloat && dt_bias.numel() == HV * D,
                "dt_bias must be fp32 with HV*K elements");
    TORCH_CHECK(A_log.is_contiguous() && dt_bias.is_contiguous(),
                "A_log and dt_bias must be contiguous");
    check_same_device(q, "A_log", A_log);
    check_same_device(q, "dt_bias", dt_bias);
}

void check_index_tensors(const char *op, const at::Tensor &q, const at::Tensor &indices,
                         const at::Tensor &cu_seqlens) {
    for (const auto &named : {NamedTensor{"initial_state_indices", indices},
                              NamedTensor{"cu_seqlens", cu_seqlens}}) {
        TORCH_CHECK(named.second.scalar_type() == at::kInt ||
                        named.second.scalar_type() == at::kLong,
                    named.first, " must be int32 or int64");
        TORCH_CHECK(named.second.is_contiguous(), named.first, " must be contiguous");
        TORCH_CHECK(named.second.device() == q.device(), named.first,
                    " must be on the same device as q");
    }
    TORCH_CHECK(cu_seqlens.numel() == indices.numel() + 1, op,
                ": cu_seqlens must have numReq+1 entries, got ", cu_seqlens.numel(), " for ",
                indices.numel(), " requests");
}

void check_track(const at::Tensor &q, const at::Tensor &indices,
                 const std::optional<at::Tensor> &track_indices,
                 const std::optional<at::Tensor> &track_lens) {
    if (!track_indices.has_value()) {
        return;
    }
    TORCH_CHECK(track_lens.has_value(), "track_state_indices requires track_state_lens");
    for (const auto &named : {NamedTensor{"track_state_indices", *track_indices},
                              NamedTensor{"track_state_lens", *track_lens}}) {
        TORCH_CHECK(named.second.scalar_type() == at::kInt ||
                        named.second.scalar_type() == at::kLong,
                    named.first, " must be int32 or int64");
        TORCH_CHECK(named.second.numel() == indices.numel(), named.first,
                    " must have one entry per request");
        TORCH_CHECK(named.second.device() == q.device(), named.first,
                    " must be on the same device as q");
    }
}

// The state pool: 4-D fp32 [slots, H, K, V] with K contiguous
// (kda_varlen_recurrent.cpp:60-74).
void check_pool(const at::Tensor &pool, int64_t H, int64_t D) {
    TORCH_CHECK(pool.dim() == 4 && pool.scalar_type() == at::kFloat,
                "state must be a 4-D fp32 [slots,HV,K,V] pool");
    TORCH_CHECK(pool.size(1) == H && pool.size(2) == D && pool.size(3) == D,
                "state must be [slots,HV,K,V] matching the head and feature dims");
    TORCH_CHECK(pool.stride(2) == 1 && pool.stride(3) == D,
                "state must be K-contiguous (stride(2)==1, stride(3)==", D, "), got strides (",
                pool.stride(2), ", ", pool.stride(3), ")");
}

// The kernels run on a HIP device only; a host tensor is an error, never a
// fallback. Checked after the shape/layout rules so those are testable on a
// machine without a GPU.
void check_on_gpu(const char *name, const at::Tensor &t) {
    TORCH_CHECK(t.device().is_cuda(), name, " must be a CUDA (HIP) tensor");
}

struct PoolRef {
    float *base;
    int64_t stride_slot;
    int64_t stride_head;
    int64_t num_slots;
};

PoolRef pool_ref(at::Tensor &pool) {
    return PoolRef{pool.data_ptr<float>(), pool.stride(0), pool.stride(1), pool.size(0)};
}

at::Tensor run_chunk(const char *op, KdaChunkArgs &args, const at::Tensor &q);

// A prefill of K = V = 128 whose requests average at least this many tokens
// runs in the chunked form (measured: 1024 tokens on 4 heads take ~1 ms
// token by token, a few tens of microseconds in 64-token chunks).
constexpr int64_t kChunkRouteTokensPerRequest = 128;
// ... but only inside the chunk kernels' anchored envelope: with raw gates
// g >= lower_bound per token, so 8 tokens decay by at most 8 |lower_bound|
// nat, below 2^126 (87.3 nat). Beyond it the chunk kernels stay exact but
// form every steep chunk's products element by element, so a lower bound
// under this keeps the token loop.
constexpr double kChunkRouteMinLowerBound = -10.9;
// ... and with a bounded workspace: the token loop allocates nothing beyond
// the output, so the chunked route takes at most this much scratch. A single
// sequence needing more runs in windows of what this holds; several
// sequences needing more, or an allocation that fails, keep the token loop.
constexpr size_t kChunkRouteMaxWorkspace = size_t{512} << 20;

// ---------------------------------------------------------------------------
// kda_varlen_recurrent
// ---------------------------------------------------------------------------

at::Tensor varlen_recurrent_impl(const char *op, const at::Tensor &A_log, const at::Tensor &a,
                                 const at::Tensor &dt_bias, const at::Tensor &q,
                                 const at::Tensor &k, const at::Tensor &v, const at::Tensor &b,
                                 at::Tensor &pool, const at::Tensor &indices,
                                 const at::Tensor &cu_seqlens, double lower_bound, double scale,
                                 const std::optional<at::Tensor> &intermediate, bool prefill,
                                 const std::optional<at::Tensor> &track_indices,
                                 const std::optional<at::Tensor> &track_lens) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, op,
                " expects q, k, v as [1, T, H, D]");
    check_packed(op, q, indices);
    const int64_t H = k.size(2);
    const int64_t D = k.size(3);
    const int64_t HV = v.size(2);
    const int64_t DV = v.size(3);
    const bool save_mid = intermediate.has_value();
    const bool track = track_indices.has_value();

    for (const auto &named : {NamedTensor{"q", q}, NamedTensor{"k", k}, NamedTensor{"v", v},
                              NamedTensor{"a", a}, NamedTensor{"b", b}}) {
        TORCH_CHECK(named.second.scalar_type() == at::kBFloat16, named.first, " must be bf16");
        TORCH_CHECK(named.second.is_contiguous(), named.first, " must be contiguous");
        check_same_device(q, named.first, named.second);
    }
    TORCH_CHECK(H == HV, op, " requires H == HV, got ", H, " and ", HV);
    TORCH_CHECK(D == DV && (D == 64 || D == 128), op, " requires K == V in {64, 128}, got ", D,
                " and ", DV);
    TORCH_CHECK(q.sizes() == k.sizes() && a.sizes() == k.sizes() && v.size(1) == q.size(1),
                op, " expects q, k, a as [1, T, H, K] and v as [1, T, H, V]");
    TORCH_CHECK(b.numel() == q.size(1) * H, op, " expects b as [1, T, H]");
    check_gate_params(q, A_log, dt_bias, HV, D);
    check_pool(pool, HV, D);
    check_same_device(q, "initial_state_source", pool);
    if (save_mid) {
        const auto &mid = *intermediate;
        TORCH_CHECK(mid.dim() == 5 && mid.scalar_type() == at::kFloat,
                    "intermediate_state must be a 5-D fp32 [slots,steps,HV,K,V] buffer");
        TORCH_CHECK(mid.size(2) == HV && mid.size(3) == D && mid.size(4) == D,
                    "intermediate_state must be [slots,steps,HV,K,V] matching the head and "
                    "feature dims");
        TORCH_CHECK(mid.stride(3) == 1 && mid.stride(4) == D,
                    "intermediate_state must be K-contiguous (stride(3)==1, stride(4)==", D,
                    "), got strides (", mid.stride(3), ", ", mid.stride(4), ")");
        check_same_device(q, "intermediate_state", mid);
        TORCH_CHECK(mid.size(0) >= indices.numel(), "intermediate_state needs a row per request, got ",
                    mid.size(0), " for ", indices.numel(), " requests");
        TORCH_CHECK(mid.size(1) * indices.numel() >= q.size(1), "intermediate_state has ",
                    mid.size(1), " step rows, too few for ", q.size(1), " tokens across ",
                    indices.numel(), " requests");
    }
    check_index_tensors(op, q, indices, cu_seqlens);
    check_track(q, indices, track_indices, track_lens);

    const int64_t T = q.size(1);
    const int64_t N = indices.numel();
    // The reference's regime rules that are semantic rather than tied to its
    // Ascend kernels (kda_varlen_recurrent.cpp:219-241). The H limits and the
    // one-packed-sequence prefill limit are not: every H and any number of
    // prefill sequences run here.
    if (prefill) {
        TORCH_CHECK(!save_mid, op, " prefill does not support intermediate_state");
    } else {
        TORCH_CHECK(T >= N, op, " decode expects at least one token per request, got T=", T,
                    " and numReq=", N);
        TORCH_CHECK(!track, op, " tracking is prefill-only");
    }

    check_on_gpu("q", q);
    const c10::DeviceGuard device_guard(q.device());  // launch on q's device
    const at::Tensor idx32 = as_int32(indices);
    const at::Tensor cu32 = as_int32(cu_seqlens);
    const auto ti32 = as_int32_opt(track_indices);
    const auto tl32 = as_int32_opt(track_lens);
    // Every token is written by the kernel (uncovered ones as zero), so the
    // output needs no fill: the reference's zeros_like is kept as a contract,
    // not as a memset.
    at::Tensor out = at::empty_like(v);
    // No request: every token is uncovered, so zero. No tokens but some
    // requests still launch: a prefix tracked at length 0 receives the
    // request's initial state.
    if (N == 0) {
        return out.zero_();
    }
    const PoolRef pr = pool_ref(pool);

    // Long prefill: the chunked form of the same recurrence (64-token chunks
    // on MFMA, within the tolerance contract of the token loop) instead of a
    // serial pass over every token. Same slot, padding, tracking and
    // uncovered-token rules.
    size_t route_ws = 0;
    if (prefill && D == 128 && T >= kChunkRouteTokensPerRequest * N &&
        lower_bound >= kChunkRouteMinLowerBound) {
        route_ws = kda_chunk_workspace_bytes(static_cast<int32_t>(T), static_cast<int32_t>(N),
                                             static_cast<int32_t>(H), static_cast<int32_t>(D));
        if (route_ws > kChunkRouteMaxWorkspace) {
            route_ws = N == 1 ? kChunkRouteMaxWorkspace : 0;
        }
    }
    std::optional<at::Tensor> route_buf;
    if (route_ws > 0) {
        try {
            route_buf = at::empty({static_cast<int64_t>(route_ws)}, q.options().dtype(at::kByte));
        } catch (const c10::OutOfMemoryError &) {
            route_buf.reset();  // the token loop needs no scratch
        }
    }
    if (route_buf.has_value()) {
        KdaChunkArgs cargs{};
        cargs.q = q.data_ptr();
        cargs.k = k.data_ptr();
        cargs.v = v.data_ptr();
        cargs.gate = a.data_ptr();
        cargs.beta = b.data_ptr();
        cargs.A_log = A_log.data_ptr<float>();
        cargs.dt_bias = dt_bias.data_ptr<float>();
        cargs.state = pr.base;
        cargs.state_stride_slot = pr.stride_slot;
        cargs.state_stride_head = pr.stride_head;
        cargs.num_slots = pr.num_slots;
        cargs.state_indices = i32_ptr(idx32);
        cargs.cu_seqlens = i32_ptr(cu32);
        cargs.out = out.data_ptr();
        if (ti32.has_value()) {
            cargs.track_indices = i32_ptr(*ti32);
            cargs.track_lens = i32_ptr(*tl32);
        }
        cargs.scale = static_cast<float>(scale);
        cargs.lower_bound = static_cast<float>(lower_bound);
        cargs.num_seqs = static_cast<int32_t>(N);
        cargs.num_tokens = static_cast<int32_t>(T);
        cargs.num_heads = static_cast<int32_t>(H);
        cargs.head_dim = static_cast<int32_t>(D);
        cargs.qk_dtype = KDA_BF16;
        cargs.v_dtype = KDA_BF16;
        cargs.gate_mode = KDA_GATE_RAW;
        cargs.qk_l2norm = 1;
        check_ok(kda_chunk_launch(&cargs, route_buf->data_ptr(), route_ws, stream_of(q)), op);
        return out;
    }

    KdaRecurrentArgs args{};
    args.q = q.data_ptr();
    args.k = k.data_ptr();
    args.v = v.data_ptr();
    args.gate = a.data_ptr();
    args.beta = b.data_ptr();
    args.A_log = A_log.data_ptr<float>();
    args.dt_bias = dt_bias.data_ptr<float>();
    args.state = pr.base;
    args.state_stride_slot = pr.stride_slot;
    args.state_stride_head = pr.stride_head;
    args.num_slots = pr.num_slots;
    args.state_indices = i32_ptr(idx32);
    args.cu_seqlens = i32_ptr(cu32);
    args.out = out.data_ptr();
    if (save_mid) {
        at::Tensor mid = *intermediate;
        args.intermediate = mid.data_ptr<float>();
        args.mid_stride_req = mid.stride(0);
        args.mid_stride_step = mid.stride(1);
        args.mid_stride_head = mid.stride(2);
        args.mid_rows = mid.size(0);
        args.mid_steps = mid.size(1);
    }
    if (ti32.has_value()) {
        args.track_indices = i32_ptr(*ti32);
        args.track_lens = i32_ptr(*tl32);
    }
    args.scale = static_cast<float>(scale);
    args.lower_bound = static_cast<float>(lower_bound);
    args.num_seqs = static_cast<int32_t>(N);
    args.num_tokens = static_cast<int32_t>(T);
    args.num_heads = static_cast<int32_t>(H);
    args.head_begin = 0;
    args.head_count = static_cast<int32_t>(H);
    args.head_dim = static_cast<int32_t>(D);
    args.qk_dtype = KDA_BF16;
    args.v_dtype = KDA_BF16;
    args.gate_mode = KDA_GATE_RAW;
    args.qk_l2norm = 1;
    check_ok(kda_recurrent_launch(&args, stream_of(q)), op);
    return out;
}

at::Tensor kda_varlen_recurrent(const at::Tensor &A_log, const at::Tensor &a,
                                const at::Tensor &dt_bias, const at::Tensor &q,
                                const at::Tensor &k, const at::Tensor &v, const at::Tensor &b,
                                at::Tensor &initial_state_source,
                                const at::Tensor &initial_state_indices,
                                const at::Tensor &cu_seqlens, double lower_bound, double scale,
                                const std::optional<at::Tensor> &intermediate_state, bool prefill,
                                const std::optional<at::Tensor> &track_state_indices,
                                const std::optional<at::Tensor> &track_state_lens) {
    return varlen_recurrent_impl("kda_varlen_recurrent", A_log, a, dt_bias, q, k, v, b,
                                 initial_state_source, initial_state_indices, cu_seqlens,
                                 lower_bound, scale, intermediate_state, prefill,
                                 track_state_indices, track_state_lens);
}

at::Tensor kda_varlen_recurrent_v2(const at::Tensor &A_log, const at::Tensor &a,
                                   const at::Tensor &dt_bias, const at::Tensor &q,
                                   const at::Tensor &k, const at::Tensor &v, const at::Tensor &b,
                                   at::Tensor &initial_state_source,
                                   const at::Tensor &initial_state_indices,
                                   const at::Tensor &cu_seqlens, double lower_bound,
                                   double scale,
                                   const std::optional<at::Tensor> &intermediate_state,
                                   bool prefill,
                                   const std::optional<at::Tensor> &track_state_indices,
                                   const std::optional<at::Tensor> &track_state_lens) {
    return varlen_recurrent_impl("kda_varlen_recurrent_v2", A_log, a, dt_bias, q, k, v, b,
                                 initial_state_source, initial_state_indices, cu_seqlens,
                                 lower_bound, scale, intermediate_state, prefill,
                                 track_state_indices, track_state_lens);
}

// ---------------------------------------------------------------------------
// kda_varlen_chunk
// ---------------------------------------------------------------------------

at::Tensor run_chunk(const char *op, KdaChunkArgs &args, const at::Tensor &q) {
    const size_t ws = kda_chunk_workspace_bytes(args.num_tokens, args.num_seqs, args.num_heads,
                                                args.head_dim);
    at::Tensor workspace =
        at::empty({static_cast<int64_t>(ws > 0 ? ws : 1)}, q.options().dtype(at::kByte));
    check_ok(kda_chunk_launch(&args, workspace.data_ptr(), ws, stream_of(q)), op);
    return workspace;
}

at::Tensor varlen_chunk_impl(const char *op, const at::Tensor &A_log, const at::Tensor &a,
                             const at::Tensor &dt_bias, const at::Tensor &q, const at::Tensor &k,
                             const at::Tensor &v, const at::Tensor &b, at::Tensor &pool,
                             const at::Tensor &indices, const at::Tensor &cu_seqlens,
                             double lower_bound, double scale,
                             const std::optional<at::Tensor> &track_indices,
                             const std::optional<at::Tensor> &track_lens) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4, op,
                " expects q, k, v as [1, T, H, D]");
    check_packed(op, q, indices);
    const int64_t H = k.size(2);
    const int64_t D = k.size(3);
    const int64_t HV = v.size(2);
    const int64_t DV = v.size(3);
    for (const auto &named : {NamedTensor{"q", q}, NamedTensor{"k", k}, NamedTensor{"v", v},
                              NamedTensor{"a", a}, NamedTensor{"b", b}}) {
        TORCH_CHECK(named.second.scalar_type() == at::kBFloat16, named.first, " must be bf16");
        TORCH_CHECK(named.second.is_contiguous(), named.first, " must be contiguous");
        check_same_device(q, named.first, named.second);
    }
    TORCH_CHECK(H == HV, op, " requires H == HV, got ", H, " and ", HV);
    TORCH_CHECK(D == 128 && DV == 128, op, " requires K == V == 128, got ", D, " and ", DV);
    TORCH_CHECK(q.sizes() == k.sizes() && a.sizes() == k.sizes() && v.size(1) == q.size(1),
                op, " expects q, k, a as [1, T, H, K] and v as [1, T, H, V]");
    TORCH_CHECK(b.numel() == q.size(1) * H, op, " expects b as [1, T, H]");
    check_gate_params(q, A_log, dt_bias, HV, D);
    check_pool(pool, HV, D);
    check_same_device(q, "initial_state_source", pool);
    check_index_tensors(op, q, indices, cu_seqlens);
    check_track(q, indices, track_indices, track_lens);

    const int64_t T = q.size(1);
    const int64_t N = indices.numel();
    check_on_gpu("q", q);
    const c10::DeviceGuard device_guard(q.device());  // launch on q's device
    const at::Tensor idx32 = as_int32(indices);
    const at::Tensor cu32 = as_int32(cu_seqlens);
    const auto ti32 = as_int32_opt(track_indices);
    const auto tl32 = as_int32_opt(track_lens);
    at::Tensor out = at::empty_like(v);
    // No request: every token is uncovered, so zero. No tokens but some
    // requests still launch: a prefix tracked at length 0 receives the
    // request's initial state.
    if (N == 0) {
        return out.zero_();
    }
    const PoolRef pr = pool_ref(pool);
    KdaChunkArgs args{};
    args.q = q.data_ptr();
    args.k = k.data_ptr();
    args.v = v.data_ptr();
    args.gate = a.data_ptr();
    args.beta = b.data_ptr();
    args.A_log = A_log.data_ptr<float>();
    args.dt_bias = dt_bias.data_ptr<float>();
    args.state = pr.base;
    args.state_stride_slot = pr.stride_slot;
    args.state_stride_head = pr.stride_head;
    args.num_slots = pr.num_slots;
    args.state_indices = i32_ptr(idx32);
    args.cu_seqlens = i32_ptr(cu32);
    args.out = out.data_ptr();
    if (ti32.has_value()) {
        args.track_indices = i32_ptr(*ti32);
        args.track_lens = i32_ptr(*tl32);
    }
    args.scale = static_cast<float>(scale);
    args.lower_bound = static_cast<float>(lower_bound);
    args.num_seqs = static_cast<int32_t>(N);
    args.num_tokens = static_cast<int32_t>(T);
    args.num_heads = static_cast<int32_t>(H);
    args.head_dim = static_cast<int32_t>(D);
    args.qk_dtype = KDA_BF16;
    args.v_dtype = KDA_BF16;
    args.gate_mode = KDA_GATE_RAW;
    args.qk_l2norm = 1;
    run_chunk(op, args, q);
    return out;
}

at::Tensor kda_varlen_chunk(const at::Tensor &A_log, const at::Tensor &a,
                            const at::Tensor &dt_bias, const at::Tensor &q, const at::Tensor &k,
                            const at::Tensor &v, const at::Tensor &b,
                            at::Tensor &initial_state_source,
                            const at::Tensor &initial_state_indices,
                            const at::Tensor &cu_seqlens, double lower_bound, double scale,
                            bool prefill, const std::optional<at::Tensor> &track_state_indices,
                            const std::optional<at::Tensor> &track_state_lens) {
    (void)prefill;  // the chunked form is prefill by construction
    return varlen_chunk_impl("kda_varlen_chunk", A_log, a, dt_bias, q, k, v, b,
                             initial_state_source, initial_state_indices, cu_seqlens, lower_bound,
                             scale, track_state_indices, track_state_lens);
}

at::Tensor kda_varlen_chunk_v2(const at::Tensor &A_log, const at::Tensor &a,
                               const at::Tensor &dt_bias, const at::Tensor &q,
                               const at::Tensor &k, const at::Tensor &v, const at::Tensor &b,
                               at::Tensor &initial_state_source,
                               const at::Tensor &initial_state_indices,
                               const at::Tensor &cu_seqlens, double lower_bound, double scale,
                               bool prefill,
                               const std::optional<at::Tensor> &track_state_indices,
                               const std::optional<at::Tensor> &track_state_lens) {
    (void)prefill;
    return varlen_chunk_impl("kda_varlen_chunk_v2", A_log, a, dt_bias, q, k, v, b,
                             initial_state_source, initial_state_indices, cu_seqlens, lower_bound,
                             scale, track_state_indices, track_state_lens);
}

// ---------------------------------------------------------------------------
// prepared-gate forms (q, k, v; fp32 log decay g; fp32 beta)
// ---------------------------------------------------------------------------

struct PreparedInputs {
    int64_t T, H, D;
    int32_t qk_dtype;
};

PreparedInputs check_prepared(const char *op, const at::Tensor &q, const at::Tensor &k,
                              const at::Tensor &v, const at::Tensor &g, const at::Tensor &beta,
                              at::Tensor &pool, const at::Tensor &indices,
                              const at::Tensor &cu_seqlens,
                              const std::optional<at::Tensor> &track_indices,
                              const std::optional<at::Tensor> &track_lens,
                              bool allow_d64) {
    TORCH_CHECK(q.dim() == 4 && k.dim() == 4 && v.dim() == 4 && g.dim() == 4, op,
                " expects q, k, v, g as [1, T, H, D]");
    check_packed(op, q, indices);
    const auto dt = q.scalar_type();
    TORCH_CHECK(dt == at::kBFloat16 || dt == at::kFloat, op, ": q must be bf16 or fp32");
    for (const auto &named : {NamedTensor{"q", q}, NamedTensor{"k", k}, NamedTensor{"v", v}}) {
        TORCH_CHECK(named.second.scalar_type() == dt, named.first, " must have q's dtype");
        TORCH_CHECK(named.second.is_contiguous(), named.first, " must be contiguous");
        check_same_device(q, named.first, named.second);
    }
    for (const auto &named : {NamedTensor{"g", g}, NamedTensor{"beta", beta}}) {
        TORCH_CHECK(named.second.scalar_type() == at::kFloat, named.first, " must be fp32");
        TORCH_CHECK(named.second.is_contiguous(), named.first, " must be contiguous");
        check_same_device(q, named.first, named.second);
    }
    const int64_t H = q.size(2);
    const int64_t D = q.size(3);
    TORCH_CHECK(k.sizes() == q.sizes() && v.sizes() == q.sizes() && g.sizes() == q.sizes(), op,
                " expects q, k, v, g all [1, T, H, D] with H == HV and K == V");
    TORCH_CHECK(D == 128 || (allow_d64 && D == 64), op, " requires K == V in {",
                allow_d64 ? "64, " : "", "128}, got ", D);
    TORCH_CHECK(beta.numel() == q.size(1) * H, op, " expects beta as [1, T, H]");
    check_pool(pool, H, D);
    check_same_device(q, "initial_state_source", pool);
    check_index_tensors(op, q, indices, cu_seqlens);
    check_track(q, indices, track_indices, track_lens);
    return PreparedInputs{q.size(1), H, D, dt == at::kFloat ? KDA_F32 : KDA_BF16};
}

at::Tensor kda_prepared_varlen_recurrent(const at::Tensor &q, const at::Tensor &k,
                                         const at::Tensor &v, const at::Tensor &g,
                                         const at::Tensor &beta,
                                         at::Tensor &initial_state_source,
                                         const at::Tensor &initial_state_indices,
                                         const at::Tensor &cu_seqlens, double scale,
                                         bool use_qk_l2norm,
                                         const std::optional<at::Tensor> &intermediate_state,
                                         const std::optional<at::Tensor> &track_state_indices,
                                         const std::optional<at::Tensor> &track_state_lens) {
    const char *op = "kda_prepared_varlen_recurrent";
    const PreparedInputs p = check_prepared(op, q, k, v, g, beta, initial_state_source,
                                            initial_state_indices, cu_seqlens,
                                            track_state_indices, track_state_lens, true);
    const int64_t N = initial_state_indices.numel();
    if (intermediate_state.has_value()) {
        const auto &mid = *intermediate_state;
        TORCH_CHECK(mid.dim() == 5 && mid.scalar_type() == at::kFloat,
                    "intermediate_state must be a 5-D fp32 [slots,steps,HV,K,V] buffer");
        TORCH_CHECK(mid.size(2) == p.H && mid.size(3) == p.D && mid.size(4) == p.D,
                    "intermediate_state must be [slots,steps,HV,K,V] matching the head and "
                    "feature dims");
        TORCH_CHECK(mid.stride(3) == 1 && mid.stride(4) == p.D,
                    "intermediate_state must be K-contiguous (stride(3)==1, stride(4)==", p.D,
                    "), got strides (", mid.stride(3), ", ", mid.stride(4), ")");
        check_same_device(q, "intermediate_state", mid);
        TORCH_CHECK(mid.size(0) >= N, "intermediate_state needs a row per request, got ",
                    mid.size(0), " for ", N, " requests");
    }
    check_on_gpu("q", q);
    const c10::DeviceGuard device_guard(q.device());  // launch on q's device
    const at::Tensor idx32 = as_int32(initial_state_indices);
    const at::Tensor cu32 = as_int32(cu_seqlens);
    const auto ti32 = as_int32_opt(track_state_indices);
    const auto tl32 = as_int32_opt(track_state_lens);
    at::Tensor out = at::empty_like(v);
    // No request: every token is uncovered, so zero. No tokens but some
    // requests still launch: a prefix tracked at length 0 receives the
    // request's initial state.
    if (N == 0) {
        return out.zero_();
    }
    const PoolRef pr = pool_ref(initial_state_source);
    KdaRecurrentArgs args{};
    args.q = q.data_ptr();
    args.k = k.data_ptr();
    args.v = v.data_ptr();
    args.gate = g.data_ptr();
    args.beta = beta.data_ptr();
    args.state = pr.base;
    args.state_stride_slot = pr.stride_slot;
    args.state_stride_head = pr.stride_head;
    args.num_slots = pr.num_slots;
    args.state_indices = i32_ptr(idx32);
    args.cu_seqlens = i32_ptr(cu32);
    args.out = out.data_ptr();
    if (intermediate_state.has_value()) {
        at::Tensor mid = *intermediate_state;
        args.intermediate = mid.data_ptr<float>();
        args.mid_stride_req = mid.stride(0);
        args.mid_stride_step = mid.stride(1);
        args.mid_stride_head = mid.stride(2);
        args.mid_rows = mid.size(0);
        args.mid_steps = mid.size(1);
    }
    if (ti32.has_value()) {
        args.track_indices = i32_ptr(*ti32);
        args.track_lens = i32_ptr(*tl32);
    }
    args.scale = static_cast<float>(scale);
    args.num_seqs = static_cast<int32_t>(N);
    args.num_tokens = static_cast<int32_t>(p.T);
    args.num_heads = static_cast<int32_t>(p.H);
    args.head_begin = 0;
    args.head_count = static_cast<int32_t>(p.H);
    args.head_dim = static_cast<int32_t>(p.D);
    args.qk_dtype = p.qk_dtype;
    args.v_dtype = p.qk_dtype;
    args.gate_mode = KDA_GATE_LOG;
    args.qk_l2norm = use_qk_l2norm ? 1 : 0;
    check_ok(kda_recurrent_launch(&args, stream_of(q)), op);
    return out;
}

at::Tensor kda_prepared_varlen_chunk(const at::Tensor &q, const at::Tensor &k,
                                     const at::Tensor &v, const at::Tensor &g,
                                     const at::Tensor &beta, at::Tensor &initial_state_source,
                                     const at::Tensor &initial_state_indices,
                                     const at::Tensor &cu_seqlens, double scale,
                                     bool use_qk_l2norm,
                                     const std::optional<at::Tensor> &track_state_indices,
                                     const std::optional<at::Tensor> &track_state_lens) {
    const char *op = "kda_prepared_varlen_chunk";
    const PreparedInputs p = check_prepared(op, q, k, v, g, beta, initial_state_source,
                                            initial_state_indices, cu_seqlens,
                                            track_state_indices, track_state_lens, false);
    TORCH_CHECK(p.qk_dtype == KDA_BF16, op, " takes bf16 q, k, v (bf16 MFMA operands)");
    const int64_t N = initial_state_indices.numel();
    check_on_gpu("q", q);
    const c10::DeviceGuard device_guard(q.device());  // launch on q's device
    const at::Tensor idx32 = as_int32(initial_state_indices);
    const at::Tensor cu32 = as_int32(cu_seqlens);
    const auto ti32 = as_int32_opt(track_state_indices);
    const auto tl32 = as_int32_opt(track_state_lens);
    at::Tensor out = at::empty_like(v);
    // No request: every token is uncovered, so zero. No tokens but some
    // requests still launch: a prefix tracked at length 0 receives the
    // request's initial state.
    if (N == 0) {
        return out.zero_();
    }
    const PoolRef pr = pool_ref(initial_state_source);
    KdaChunkArgs args{};
    args.q = q.data_ptr();
    args.k = k.data_ptr();
    args.v = v.data_ptr();
    args.gate = g.data_ptr();
    args.beta = beta.data_ptr();
    args.state = pr.base;
    args.state_stride_slot = pr.stride_slot;
    args.state_stride_head = pr.stride_head;
    args.num_slots = pr.num_slots;
    args.state_indices = i32_ptr(idx32);
    args.cu_seqlens = i32_ptr(cu32);
    args.out = out.data_ptr();
    if (ti32.has_value()) {
        args.track_indices = i32_ptr(*ti32);
        args.track_lens = i32_ptr(*tl32);
    }
    args.scale = static_cast<float>(scale);
    args.num_seqs = static_cast<int32_t>(N);
    args.num_tokens = static_cast<int32_t>(p.T);
    args.num_heads = static_cast<int32_t>(p.H);
    args.head_dim = static_cast<int32_t>(p.D);
    args.qk_dtype = KDA_BF16;
    args.v_dtype = KDA_BF16;
    args.gate_mode = KDA_GATE_LOG;
    args.qk_l2norm = use_qk_l2norm ? 1 : 0;
    run_chunk(op, args, q);
    return out;
}

// ---------------------------------------------------------------------------
// prepared_recurrent (prepared_recurrent.cpp:610-713)
// ---------------------------------------------------------------------------

void prepared_recurrent(const at::Tensor &qn, const at::Tensor &kn, const at::Tensor &v,
                        const at::Tensor &gdecay, const at::Tensor &beta, at::Tensor &out,
                        at::Tensor &state, const at::Tensor &indices, const at::Tensor &starts,
                        const std::optional<at::Tensor> &track_indices,
                        const std::optional<at::Tensor> &track_lens, bool track_state,
                        int64_t head_offset) {
    const char *op = "prepared_recurrent";
    TORCH_CHECK(state.dim() == 4 && state.scalar_type() == at::kFloat,
                "state must be a 4-D fp32 [slots,H,K,V] pool");
    const int64_t H = state.size(1);
    const int64_t D = state.size(2);
    TORCH_CHECK(state.size(3) == D && (D == 64 || D == 128), op,
                ": state must be [slots,H,D,D] with D in {64, 128}");
    // The reference launches four heads per call, heads [head_offset,
    // head_offset+4) of H (prepared_recurrent.cpp:629-634, 691-707).
    constexpr int64_t kHeadsPerLaunch = 4;
    TORCH_CHECK(head_offset >= 0 && head_offset < H && head_offset % kHeadsPerLaunch == 0,
                "head_offset must be a multiple of 4 below H=", H, ", got ", head_offset);
    for (const auto &named : {NamedTensor{"qn", qn}, NamedTensor{"kn", kn},
                              NamedTensor{"gdecay", gdecay}}) {
        TORCH_CHECK(named.second.scalar_type() == at::kFloat, named.first, " must be fp32");
        TORCH_CHECK(named.second.is_contiguous(), named.first, " must be contiguous");
        TORCH_CHECK(named.second.device() == qn.device(), named.first,
                    " must be on the same device as qn");
    }
    TORCH_CHECK(beta.scalar_type() == at::kFloat && beta.is_contiguous(),
                "beta must be contiguous fp32");
    TORCH_CHECK(v.scalar_type() == out.scalar_type() &&
                    (v.scalar_type() == at::kBFloat16 || v.scalar_type() == at::kFloat),
                "v and out must share a bf16 or fp32 dtype");
    TORCH_CHECK(v.is_contiguous() && out.is_contiguous(), "v and out must be contiguous");
    for (const auto &named : {NamedTensor{"v", v}, NamedTensor{"out", out},
                              NamedTensor{"beta", beta}, NamedTensor{"state", state},
                              NamedTensor{"indices", indices}, NamedTensor{"starts", starts}}) {
        TORCH_CHECK(named.second.device() == qn.device(), named.first,
                    " must be on the same device as qn");
    }
    const int64_t rows = qn.numel() / D;
    TORCH_CHECK(rows % H == 0 && kn.numel() == qn.numel() && v.numel() == qn.numel() &&
                    gdecay.numel() == qn.numel() && out.numel() == qn.numel() &&
                    beta.numel() == rows,
                op, ": qn, kn, v, gdecay, out must hold T*H rows of D, beta T*H values");
    const int64_t T = rows / H;
    TORCH_CHECK(T <= INT32_MAX && starts.numel() <= INT32_MAX, op,
                " supports at most 2^31-1 tokens and requests");
    TORCH_CHECK(starts.scalar_type() == at::kInt || starts.scalar_type() == at::kLong,
                "starts must be int32 or int64");
    TORCH_CHECK(indices.scalar_type() == at::kInt || indices.scalar_type() == at::kLong,
                "indices must be int32 or int64");
    const int64_t N = starts.numel() - 1;
    TORCH_CHECK(N >= 0 && indices.numel() >= N, op,
                ": indices must have an entry per request in starts");
    if (track_state) {
        TORCH_CHECK(track_indices.has_value() && track_indices->defined(),
                    "track_indices is required when track_state=True");
        TORCH_CHECK(track_lens.has_value() && track_lens->defined(),
                    "track_lens is required when track_state=True");
        for (const auto &named : {NamedTensor{"track_indices", *track_indices},
                                  NamedTensor{"track_lens", *track_lens}}) {
            TORCH_CHECK(named.second.device() == qn.device(), named.first,
                        " must be on the same device as qn");
            TORCH_CHECK(named.second.scalar_type() == at::kInt ||
                            named.second.scalar_type() == at::kLong,
                        named.first, " must be int32 or int64");
            TORCH_CHECK(named.second.numel() >= N, named.first, " must contain at least ", N,
                        " elements");
        }
    }
    check_on_gpu("qn", qn);
    check_on_gpu("kn", kn);
    check_on_gpu("v", v);
    const c10::DeviceGuard device_guard(qn.device());  // launch on qn's device
    if (N == 0) {  // no tokens but some requests still launch (tracking at length 0)
        return;
    }
    // The reference pool for this op is [K,V]-contiguous; the native pool of
    // the other ops is K-contiguous. Both are updated in place: the kernel
    // reads and writes either layout (only the touched slots move).
    const bool k_contig = state.stride(2) == 1 && state.stride(3) == D;
    const bool v_contig = state.stride(3) == 1 && state.stride(2) == D;
    TORCH_CHECK(k_contig || v_contig, op,
                ": state must be K-contiguous (stride(2)==1, stride(3)==D) or [K,V]-contiguous "
                "(stride(3)==1, stride(2)==D), got strides (", state.stride(2), ", ", state.stride(3),
                ")");
    const PoolRef pr = pool_ref(state);
    const at::Tensor idx32 = as_int32(indices);
    const at::Tensor cu32 = as_int32(starts);
    std::optional<at::Tensor> ti32, tl32;
    if (track_state) {
        ti32 = as_int32(*track_indices);
        tl32 = as_int32(*track_lens);
    }
    KdaRecurrentArgs args{};
    args.q = qn.data_ptr();
    args.k = kn.data_ptr();
    args.v = v.data_ptr();
    args.gate = gdecay.data_ptr();
    args.beta = beta.data_ptr();
    args.state = pr.base;
    args.state_stride_slot = pr.stride_slot;
    args.state_stride_head = pr.stride_head;
    args.num_slots = pr.num_slots;
    args.state_indices = i32_ptr(idx32);
    args.cu_seqlens = i32_ptr(cu32);
    args.out = out.data_ptr();
    if (ti32.has_value()) {
        args.track_indices = i32_ptr(*ti32);
        args.track_lens = i32_ptr(*tl32);
    }
    args.scale = 1.0f;  // qn arrives with the scale folded in
    args.num_seqs = static_cast<int32_t>(N);
    args.num_tokens = static_cast<int32_t>(T);
    args.num_heads = static_cast<int32_t>(H);
    args.head_begin = static_cast<int32_t>(head_offset);
    args.head_count = static_cast<int32_t>(std::min<int64_t>(kHeadsPerLaunch, H - head_offset));
    args.head_dim = static_cast<int32_t>(D);
    args.qk_dtype = KDA_F32;
    args.v_dtype = v.scalar_type() == at::kFloat ? KDA_F32 : KDA_BF16;
    args.gate_mode = KDA_GATE_DECAY;
    args.qk_l2norm = 0;
    args.state_v_contiguous = k_contig ? 0 : 1;
    check_ok(kda_recurrent_launch(&args, stream_of(qn)), op);
}

}  // namespace

TORCH_LIBRARY(sgl_glm53_ascend, m) {
    m.def(
        "kda_varlen_recurrent(*, Tensor A_log, Tensor a, Tensor dt_bias, "
        "Tensor q, Tensor k, Tensor v, Tensor b, "
        "Tensor(a!) initial_state_source, Tensor initial_state_indices, "
        "Tensor cu_seqlens, float lower_bound, float scale, "
        "Tensor(b!)? intermediate_state=None, bool prefill=False, "
        "Tensor? track_state_indices=None, "
        "Tensor? track_state_lens=None) -> Tensor");
    m.def(
        "kda_varlen_recurrent_v2(*, Tensor A_log, Tensor a, Tensor dt_bias, "
        "Tensor q, Tensor k, Tensor v, Tensor b, "
        "Tensor(a!) initial_state_source, Tensor initial_state_indices, "
        "Tensor cu_seqlens, float lower_bound, float scale, "
        "Tensor(b!)? intermediate_state=None, bool prefill=False, "
        "Tensor? track_state_indices=None, "
        "Tensor? track_state_lens=None) -> Tensor");
    m.def(
        "kda_varlen_chunk(*, Tensor A_log, Tensor a, Tensor dt_bias, "
        "Tensor q, Tensor k, Tensor v, Tensor b, "
        "Tensor(a!) initial_state_source, Tensor initial_state_indices, "
        "Tensor cu_seqlens, float lower_bound, float scale, "
        "bool prefill=False, Tensor? track_state_indices=None, "
        "Tensor? track_state_lens=None) -> Tensor");
    m.def(
        "kda_varlen_chunk_v2(*, Tensor A_log, Tensor a, Tensor dt_bias, "
        "Tensor q, Tensor k, Tensor v, Tensor b, "
        "Tensor(a!) initial_state_source, Tensor initial_state_indices, "
        "Tensor cu_seqlens, float lower_bound, float scale, "
        "bool prefill=False, Tensor? track_state_indices=None, "
        "Tensor? track_state_lens=None) -> Tensor");
    m.def(
        "prepared_recurrent(Tensor qn, Tensor kn, Tensor v, "
        "Tensor gdecay, Tensor beta, Tensor(a!) out, Tensor(b!) state, "
        "Tensor indices, Tensor starts, "
        "Tensor? track_indices=None, Tensor? track_lens=None, "
        "bool track_state=False, int head_offset=0) -> ()");
    m.def(
        "kda_prepared_varlen_recurrent(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, *, "
        "Tensor(a!) initial_state_source, Tensor initial_state_indices, Tensor cu_seqlens, "
        "float scale, bool use_qk_l2norm=False, Tensor(b!)? intermediate_state=None, "
        "Tensor? track_state_indices=None, Tensor? track_state_lens=None) -> Tensor");
    m.def(
        "kda_prepared_varlen_chunk(Tensor q, Tensor k, Tensor v, Tensor g, Tensor beta, *, "
        "Tensor(a!) initial_state_source, Tensor initial_state_indices, Tensor cu_seqlens, "
        "float scale, bool use_qk_l2norm=False, "
        "Tensor? track_state_indices=None, Tensor? track_state_lens=None) -> Tensor");
}

#define KDA_REGISTER_IMPLS(m)                                                   \
    m.impl("kda_varlen_recurrent", &kda_varlen_recurrent);                     \
    m.impl("kda_varlen_recurrent_v2", &kda_varlen_recurrent_v2);               \
    m.impl("kda_varlen_chunk", &kda_varlen_chunk);                             \
    m.impl("kda_varlen_chunk_v2", &kda_varlen_chunk_v2);                       \
    m.impl("prepared_recurrent", &prepared_recurrent);                         \
    m.impl("kda_prepared_varlen_recurrent", &kda_prepared_varlen_recurrent);   \
    m.impl("kda_prepared_varlen_chunk", &kda_prepared_varlen_chunk)

TORCH_LIBRARY_IMPL(sgl_glm53_ascend, CUDA, m) { KDA_REGISTER_IMPLS(m); }

// Host tensors reach the same validation and then fail at the device check:
// there is no CPU implementation of these operators.
TORCH_LIBRARY_IMPL(sgl_glm53_ascend, CPU, m) { KDA_REGISTER_IMPLS(m); }
