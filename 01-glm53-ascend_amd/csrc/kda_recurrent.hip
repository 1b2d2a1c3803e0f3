// kda_recurrent.hip -- fused recurrent KDA (delta rule with per-channel decay)
// over packed varlen sequences, for gfx950.
//
// Semantics follow the reference recurrence (bench/kda_chunk/kda_python.py:
// 253-307; device version sgl-glm53-ascend-ops/csrc/kda/recurrent/
// kda_varlen_recurrent_decode_h32.cpp:289-724): per (sequence, head) with
// state S[k][v] and per token t
//     S   <- exp(g_t)[k] * S
//     d_v  = beta_t * (v_t[v] - sum_k kn_t[k] S[k][v])
//     S   <- S + kn_t[k] d_v
//     o_v  = sum_k qn_t[k] S[k][v]           (readout after the update)
// with slot 0 the zero/padding state, per-step checkpoints and prefix
// tracking as described in kda_abi.h.
//
// MI355X mapping. The update never mixes value rows, so the state splits into
// independent rows S[:, v], each a contiguous 4*D-byte line of the
// K-contiguous pool. A lane owns four consecutive K elements (one 16-byte
// vector) of NP rows; D/4 lanes span one row, so a wave-wide 16-byte load
// covers 64/(D/4) complete rows -- fully coalesced 512 B (D=128) lines. The two
// K-reductions per token (prediction and readout) are group sums over those
// D/4 lanes (DPP + one ds_swizzle), so the state tile lives in VGPRs from the
// first load to the single in-place write-back: HBM sees each state byte
// exactly once in and once out. A workgroup (4 waves) covers NP*RPP value
// rows of one (sequence, head); the host picks NP so small batches still
// launch enough workgroups (V-split), large batches use one workgroup per
// (sequence, head).

#include <hip/hip_runtime.h>

#include "kda_abi.h"
#include "kda_device.h"

namespace kda {
namespace {

constexpr int kThreads = 256;

template <int D, int NP, typename TQK, typename TV, int GATE>
__global__ __launch_bounds__(kThreads) void recurrent_kernel(const KdaRecurrentArgs a) {
    constexpr int L = D / 4;           // lanes per state row
    constexpr int RPW = 64 / L;        // rows per wave per pass
    constexpr int RPP = 4 * RPW;       // rows per workgroup per pass
    constexpr int RB = NP * RPP;       // rows per workgroup
    constexpr int VT = D / RB;         // workgroups per (sequence, head)
    static_assert(D % RB == 0, "a workgroup covers a whole number of row tiles");
    static_assert(NP <= L, "one lane per row writes the output");

    const int H = a.num_heads;
    const int HC = a.head_count;  // heads in this launch, resolved by the host
    // XCD-aware order: consecutive workgroups go to different XCDs (each with
    // its own L2), so the VT row tiles of one (sequence, head), which read the
    // same token rows, are numbered 8 apart and share an XCD.
    const int b = blockIdx.x;
    const int rest = b >> 3;
    const int vt = VT == 1 ? 0 : rest % VT;
    const int pair = VT == 1 ? b : (rest / VT) * 8 + (b & 7);
    const int n = pair / HC;
    const int head = a.head_begin + (pair - n * HC);
    if (n >= a.num_seqs) {
        return;
    }
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int kc = lane % L;
    const int rsub = lane / L;
    const int row0 = vt * RB + wave * RPW + rsub;  // row of pass p: row0 + p*RPP
    const int T = a.num_tokens;

    int bos = a.cu_seqlens[n];
    int eos = a.cu_seqlens[n + 1];
    bos = bos < 0 ? 0 : (bos > T ? T : bos);
    eos = eos < bos ? bos : (eos > T ? T : eos);
    int slot = a.state_indices[n];
    if (slot < 0 || static_cast<int64_t>(slot) >= a.num_slots) {
        slot = 0;
    }

    const int64_t head_off = static_cast<int64_t>(head) * a.state_stride_head;
    float4 S[NP];
    if (slot > 0) {
        const float *src = a.state + slot * a.state_stride_slot + head_off;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            S[p] = load4_stream(src + static_cast<int64_t>(row0 + p * RPP) * D + 4 * kc);
        }
    } else {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            S[p] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }

    // Prefix tracking: the destination slot and the local step after which to
    // store (0 = the initial state, stored right away).
    int track_slot = 0;
    int track_len = -1;
    if (a.track_indices != nullptr) {
        track_slot = a.track_indices[n];
        if (track_slot <= 0 || static_cast<int64_t>(track_slot) >= a.num_slots) {
            track_slot = 0;
        } else {
            track_len = a.track_lens[n];
        }
    }
    // State tiles are touched once per launch: streamed with nontemporal
    // loads and stores so they do not evict the token rows from the caches
    // (measured ~10% more HBM throughput than cached accesses).
    auto store_state = [&](float *dst) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            store4_stream(dst + static_cast<int64_t>(row0 + p * RPP) * D + 4 * kc, S[p]);
        }
    };
    if (track_slot > 0 && track_len == 0) {
        store_state(a.state + track_slot * a.state_stride_slot + head_off);
    }

    // Per-head gate constants (RAW): exp(A_log[h]) and this lane's dt_bias.
    float expA = 0.f;
    float4 dtb = make_float4(0.f, 0.f, 0.f, 0.f);
    if constexpr (GATE == KDA_GATE_RAW) {
        expA = expf(a.A_log[head]);
        dtb = load4(a.dt_bias + static_cast<int64_t>(head) * D + 4 * kc);
    }
    const bool norm = (GATE == KDA_GATE_RAW) || (a.qk_l2norm != 0);
    const bool save_mid = a.intermediate != nullptr && slot > 0 && n < a.mid_rows;

    const TQK *qp = static_cast<const TQK *>(a.q);
    const TQK *kp = static_cast<const TQK *>(a.k);
    const TV *vp = static_cast<const TV *>(a.v);
    TV *op = static_cast<TV *>(a.out);

    // One token's inputs, as loaded (gates are transformed at use). The next
    // token's are loaded while the current one computes: a multi-token
    // sequence (verify, prefill) would otherwise wait a full load latency per
    // token. The branches on `more` are uniform across the workgroup.
    struct TokenIn {
        float4 q, k, g;
        float v[NP];
        float b;
    };
    auto fetch = [&](int t, TokenIn &in) {
        const int64_t base = (static_cast<int64_t>(t) * H + head) * D;
        in.q = load4(qp + base + 4 * kc);
        in.k = load4(kp + base + 4 * kc);
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            in.v[p] = load1(vp + base + row0 + p * RPP);
        }
        const int64_t bi = static_cast<int64_t>(t) * H + head;
        if constexpr (GATE == KDA_GATE_RAW) {
            in.g = load4(static_cast<const uint16_t *>(a.gate) + base + 4 * kc);
            in.b = bf16_to_f32(static_cast<const uint16_t *>(a.beta)[bi]);
        } else {
            in.g = load4(static_cast<const float *>(a.gate) + base + 4 * kc);
            in.b = static_cast<const float *>(a.beta)[bi];
        }
    };
    TokenIn cur, nxt;
    if (bos < eos) {
        fetch(bos, cur);
    }
    for (int t = bos; t < eos; ++t) {
        const bool more = t + 1 < eos;
        if (more) {
            fetch(t + 1, nxt);
        }
        const int64_t base = (static_cast<int64_t>(t) * H + head) * D;
        float4 qv = cur.q;
        float4 kv = cur.k;
        float vr[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            vr[p] = cur.v[p];
        }
        float4 dec;
        float beta;
        if constexpr (GATE == KDA_GATE_RAW) {
            const float4 av = cur.g;
            const float lb = a.lower_bound;
            // g = lower_bound / (1 + exp(-(exp(A_log) * (a + dt_bias)))), decay = exp(g)
            dec.x = expf(lb / (1.0f + expf(-(expA * (av.x + dtb.x)))));
            dec.y = expf(lb / (1.0f + expf(-(expA * (av.y + dtb.y)))));
            dec.z = expf(lb / (1.0f + expf(-(expA * (av.z + dtb.z)))));
            dec.w = expf(lb / (1.0f + expf(-(expA * (av.w + dtb.w)))));
            beta = 1.0f / (1.0f + expf(-cur.b));
        } else if constexpr (GATE == KDA_GATE_LOG) {
            const float4 gv = cur.g;
            dec = make_float4(expf(gv.x), expf(gv.y), expf(gv.z), expf(gv.w));
            beta = cur.b;
        } else {
            dec = cur.g;
            beta = cur.b;
        }
        if (norm) {
            // x / sqrt(sum x^2 + 1e-6), eps inside the sqrt; q then scaled.
            const float qs = group_sum<L>(dot4(qv, qv));
            const float ks = group_sum<L>(dot4(kv, kv));
            const float qd = sqrtf(qs + 1e-6f);
            const float kd = sqrtf(ks + 1e-6f);
            qv = make_float4(qv.x / qd, qv.y / qd, qv.z / qd, qv.w / qd);
            kv = make_float4(kv.x / kd, kv.y / kd, kv.z / kd, kv.w / kd);
        }
        const float sc = a.scale;
        qv = make_float4(qv.x * sc, qv.y * sc, qv.z * sc, qv.w * sc);

        float pred[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            S[p].x *= dec.x;
            S[p].y *= dec.y;
            S[p].z *= dec.z;
            S[p].w *= dec.w;
            pred[p] = dot4(S[p], kv);
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            pred[p] = group_sum<L>(pred[p]);
        }
        float o[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float d = (vr[p] - pred[p]) * beta;
            S[p].x += kv.x * d;
            S[p].y += kv.y * d;
            S[p].z += kv.z * d;
            S[p].w += kv.w * d;
            o[p] = dot4(S[p], qv);
        }
        const int step = t - bos;
        if (save_mid && step < a.mid_steps) {
            store_state(a.intermediate + n * a.mid_stride_req + step * a.mid_stride_step +
                        static_cast<int64_t>(head) * a.mid_stride_head);
        }
        if (track_slot > 0 && step + 1 == track_len) {
            store_state(a.state + track_slot * a.state_stride_slot + head_off);
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            o[p] = group_sum<L>(o[p]);
        }
        // Lane kc < NP writes row row0 + kc*RPP: one store per lane.
        float mine = 0.f;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            mine = (kc == p) ? o[p] : mine;
        }
        if (kc < NP) {
            store1(op + base + row0 + kc * RPP, mine);
        }
        if (more) {
            cur = nxt;
        }
    }

    // Tokens no sequence covers are zero (the reference allocates
    // zeros_like(v), kda_varlen_recurrent.cpp:142): the first request zeroes
    // [0, cu[0]) and the last one [cu[N], T).
    auto zero_rows = [&](int t0, int t1) {
        for (int t = t0; t < t1; ++t) {
            if (kc < NP) {
                store1(op + (static_cast<int64_t>(t) * H + head) * D + row0 + kc * RPP, 0.f);
            }
        }
    };
    if (n == 0) {
        zero_rows(0, bos);
    }
    if (n == a.num_seqs - 1) {
        zero_rows(eos, T);
    }

    if (a.intermediate == nullptr && slot > 0) {
        store_state(a.state + slot * a.state_stride_slot + head_off);
    }
}

using KernelFn = void (*)(const KdaRecurrentArgs);

template <int D, typename TQK, typename TV, int GATE>
KernelFn pick_np(int np) {
    if constexpr (D == 128) {
        switch (np) {
            case 8: return recurrent_kernel<D, 8, TQK, TV, GATE>;
            case 4: return recurrent_kernel<D, 4, TQK, TV, GATE>;
            case 2: return recurrent_kernel<D, 2, TQK, TV, GATE>;
            case 1: return recurrent_kernel<D, 1, TQK, TV, GATE>;
            default: return nullptr;
        }
    } else {
        switch (np) {
            case 4: return recurrent_kernel<D, 4, TQK, TV, GATE>;
            case 1: return recurrent_kernel<D, 1, TQK, TV, GATE>;
            default: return nullptr;
        }
    }
}

template <int D>
KernelFn pick_kernel(int gate, int qk_dtype, int v_dtype, int np) {
    if (gate == KDA_GATE_RAW) {
        if (qk_dtype == KDA_BF16 && v_dtype == KDA_BF16) {
            return pick_np<D, uint16_t, uint16_t, KDA_GATE_RAW>(np);
        }
        return nullptr;
    }
    if (gate == KDA_GATE_LOG) {
        if (qk_dtype == KDA_BF16 && v_dtype == KDA_BF16) {
            return pick_np<D, uint16_t, uint16_t, KDA_GATE_LOG>(np);
        }
        if (qk_dtype == KDA_F32 && v_dtype == KDA_F32) {
            return pick_np<D, float, float, KDA_GATE_LOG>(np);
        }
        return nullptr;
    }
    if (gate == KDA_GATE_DECAY) {
        if (qk_dtype == KDA_F32 && v_dtype == KDA_BF16) {
            return pick_np<D, float, uint16_t, KDA_GATE_DECAY>(np);
        }
        if (qk_dtype == KDA_F32 && v_dtype == KDA_F32) {
            return pick_np<D, float, float, KDA_GATE_DECAY>(np);
        }
        return nullptr;
    }
    return nullptr;
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
bool aligned8(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 7u) == 0; }

}  // namespace
}  // namespace kda

extern "C" int kda_recurrent_launch(const KdaRecurrentArgs *args, void *stream) {
    using namespace kda;
    if (args == nullptr) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    const KdaRecurrentArgs &a = *args;
    const int D = a.head_dim;
    if (D != 64 && D != 128) {
        return KDA_ERR_UNSUPPORTED;
    }
    if (a.num_seqs < 0 || a.num_tokens < 0 || a.num_heads <= 0 || a.num_slots < 0) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    if (a.num_seqs == 0) {
        return KDA_OK;
    }
    if (a.q == nullptr || a.k == nullptr || a.v == nullptr || a.gate == nullptr ||
        a.beta == nullptr || a.state == nullptr || a.state_indices == nullptr ||
        a.cu_seqlens == nullptr || a.out == nullptr) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    if (a.gate_mode == KDA_GATE_RAW && (a.A_log == nullptr || a.dt_bias == nullptr)) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    if ((a.track_indices == nullptr) != (a.track_lens == nullptr)) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    // 16-byte state vectors: pool base and strides must keep rows aligned.
    if (!aligned16(a.state) || (a.state_stride_slot & 3) || (a.state_stride_head & 3)) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    if (a.intermediate != nullptr &&
        (!aligned16(a.intermediate) || (a.mid_stride_req & 3) || (a.mid_stride_step & 3) ||
         (a.mid_stride_head & 3))) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    const bool qk_f32 = a.qk_dtype == KDA_F32;
    if (qk_f32 ? !(aligned16(a.q) && aligned16(a.k)) : !(aligned8(a.q) && aligned8(a.k))) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    if (a.gate_mode == KDA_GATE_RAW ? !aligned8(a.gate) : !aligned16(a.gate)) {
        return KDA_ERR_INVALID_ARGUMENT;
    }

    KdaRecurrentArgs kargs = a;
    if (kargs.head_begin < 0 || kargs.head_begin >= kargs.num_heads || kargs.head_count < 0) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    if (kargs.head_count == 0 || kargs.head_begin + kargs.head_count > kargs.num_heads) {
        kargs.head_count = kargs.num_heads - kargs.head_begin;
    }
    // V-split at D=128, by tokens per sequence (measured on MI355X): one token
    // (decode) -> 16-row tiles, eight workgroups per (sequence, head): 6.3 TB/s
    // at B=256, H=32 against 6.05 with 32-row tiles; two tokens -> 32-row
    // tiles; more (verify, recurrent prefill) -> 64-row tiles, which spread
    // the per-token work (token loads, norms, reductions) over more rows
    // (4 tokens x 1024 sequences, H=16: 456 us against 498 with 32-row tiles).
    // Small batches use 8-row tiles so the launch still fills the GPU.
    const int64_t pairs = static_cast<int64_t>(a.num_seqs) * kargs.head_count;
    int np;
    if (D == 128) {
        const int64_t tokens = a.num_tokens;
        if (pairs < 128) {
            np = 1;
        } else if (tokens <= a.num_seqs) {
            np = 2;
        } else if (tokens <= 2 * static_cast<int64_t>(a.num_seqs)) {
            np = 4;
        } else {
            np = 8;
        }
    } else {
        np = pairs >= 2048 ? 4 : 1;
    }
    KernelFn fn = (D == 128) ? pick_kernel<128>(a.gate_mode, a.qk_dtype, a.v_dtype, np)
                             : pick_kernel<64>(a.gate_mode, a.qk_dtype, a.v_dtype, np);
    if (fn == nullptr) {
        return KDA_ERR_UNSUPPORTED;
    }
    const int rows_per_wg = np * 4 * (64 / (D / 4));
    const int vts = D / rows_per_wg;
    const int64_t blocks = vts == 1 ? pairs : (pairs + 7) / 8 * 8 * vts;
    if (blocks > 0x7fffffff) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    void *params[] = {&kargs};
    const hipError_t err =
        hipLaunchKernel(reinterpret_cast<const void *>(fn), dim3(static_cast<unsigned>(blocks)),
                        dim3(kThreads), params, 0, static_cast<hipStream_t>(stream));
    return err == hipSuccess ? KDA_OK : KDA_ERR_LAUNCH;
}
