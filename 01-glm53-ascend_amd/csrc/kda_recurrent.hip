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
// K-contiguous pool. A row is spread over L lanes (a row group); each lane
// owns E = D/L of its K elements as E/4 16-byte vectors at K offsets
// 4*kc + 4*L*j, so every wave-wide 16-byte load covers whole 4*L-element
// segments of its rows -- complete cache lines. A lane holds the same K
// elements of NP consecutive rows. The two K-reductions per token
// (prediction and readout) are group sums over the L lanes (DPP, plus one
// ds_swizzle when L = 32), so the state tile lives in VGPRs from the first
// load to the single in-place write-back: HBM sees each state byte exactly
// once in and once out. A workgroup (4 waves) covers 4*(64/L)*NP value rows
// of one (sequence, head). The host picks the shape from the tokens per
// sequence: one or two tokens (decode, short verify) use 32-lane rows, one
// token with few rows per lane, so the launch has many small workgroups to
// stream the state; three or more (verify, prefill) use 16-lane rows, whose
// reductions take four DPP steps instead of five plus an LDS swizzle, with
// up to eight rows per lane to share each token's loads, exponentials and
// norms.

#include <hip/hip_runtime.h>

#include <type_traits>

#include "kda_abi.h"
#include "kda_device.h"

namespace kda {
namespace {

constexpr int kThreads = 256;

// e^x as one v_exp_f32 of x*log2(e). The product's rounding puts the
// relative error near |x| * 2^-24 plus the instruction's own ~1 ulp; a
// result below the fp32 normal range may flush to zero.
__device__ __forceinline__ float fexp(float x) {
    return __builtin_amdgcn_exp2f(x * 1.4426950408889634f);
}

// Four consecutive K elements as loaded: 8 bytes of bf16 or 16 of fp32,
// widened to fp32 at use.
template <typename T> struct Raw4;
template <> struct Raw4<uint16_t> {
    uint2 r;
    __device__ __forceinline__ void load(const uint16_t *p) {
        r = *reinterpret_cast<const uint2 *>(p);
    }
    __device__ __forceinline__ float4 get() const {
        return make_float4(__uint_as_float(r.x << 16), __uint_as_float(r.x & 0xffff0000u),
                           __uint_as_float(r.y << 16), __uint_as_float(r.y & 0xffff0000u));
    }
};
template <> struct Raw4<float> {
    float4 r;
    __device__ __forceinline__ void load(const float *p) { r = *reinterpret_cast<const float4 *>(p); }
    __device__ __forceinline__ float4 get() const { return r; }
};

// NP values of one v row, RS elements apart, as loaded (widened at use, so
// the load is not waited for until the value is needed). Consecutive values
// (RS = 1; the host guarantees the segment is aligned to its size) arrive in
// 16-byte or smaller vectors: bf16 pairs packed in words, fp32 as is. Spread
// ones arrive one element per load.
template <typename T, int NP, int RS> struct RowIn;
template <int NP, int RS> struct RowIn<uint16_t, NP, RS> {
    static constexpr int W = RS == 1 ? NP / 2 : NP;
    static_assert(RS != 1 || NP % 2 == 0, "bf16 pairs");
    uint32_t w[W];
    __device__ __forceinline__ void load(const uint16_t *p) {
        if constexpr (RS != 1) {
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                w[i] = p[RS * i];
            }
        } else if constexpr (NP == 2) {
            w[0] = *reinterpret_cast<const uint32_t *>(p);
        } else if constexpr (NP == 4) {
            const uint2 u = *reinterpret_cast<const uint2 *>(p);
            w[0] = u.x;
            w[1] = u.y;
        } else {
#pragma unroll
            for (int i = 0; i < NP / 8; ++i) {
                const uint4 u = reinterpret_cast<const uint4 *>(p)[i];
                w[4 * i + 0] = u.x;
                w[4 * i + 1] = u.y;
                w[4 * i + 2] = u.z;
                w[4 * i + 3] = u.w;
            }
        }
    }
    __device__ __forceinline__ float get(int i) const {
        if constexpr (RS != 1) {
            return __uint_as_float(w[i] << 16);
        } else {
            return __uint_as_float((i & 1) ? (w[i >> 1] & 0xffff0000u) : (w[i >> 1] << 16));
        }
    }
};
template <int NP, int RS> struct RowIn<float, NP, RS> {
    static_assert(RS != 1 || NP % 4 == 0, "whole float4 vectors");
    float x[NP];
    __device__ __forceinline__ void load(const float *p) {
        if constexpr (RS != 1) {
#pragma unroll
            for (int i = 0; i < NP; ++i) {
                x[i] = p[RS * i];
            }
        } else {
#pragma unroll
            for (int i = 0; i < NP / 4; ++i) {
                const float4 u = reinterpret_cast<const float4 *>(p)[i];
                x[4 * i + 0] = u.x;
                x[4 * i + 1] = u.y;
                x[4 * i + 2] = u.z;
                x[4 * i + 3] = u.w;
            }
        }
    }
    __device__ __forceinline__ float get(int i) const { return x[i]; }
};

// NP output values of one row, RS elements apart, written by the row
// group's lanes kc: consecutive ones as one vector by every lane (the same
// bytes to the same address -- a store with no branch around it, so the
// loop's wait for the next token's loads never has to cover a store that
// may or may not have been issued: 8 tokens x 256 sequences, H=32, 245 ->
// 230 us), spread ones value i by lane i.
template <typename T, int NP, int RS>
__device__ __forceinline__ void store_row(T *p, const float (&x)[NP], int kc) {
    if constexpr (RS == 1) {
        if constexpr (sizeof(T) == 2) {
            static_assert(NP % 2 == 0, "bf16 pairs");
            uint32_t w[NP / 2];
#pragma unroll
            for (int i = 0; i < NP / 2; ++i) {
                w[i] = pack_bf16x2(x[2 * i], x[2 * i + 1]);
            }
            if constexpr (NP == 2) {
                *reinterpret_cast<uint32_t *>(p) = w[0];
            } else if constexpr (NP == 4) {
                *reinterpret_cast<uint2 *>(p) = make_uint2(w[0], w[1]);
            } else {
#pragma unroll
                for (int i = 0; i < NP / 8; ++i) {
                    reinterpret_cast<uint4 *>(p)[i] =
                        make_uint4(w[4 * i], w[4 * i + 1], w[4 * i + 2], w[4 * i + 3]);
                }
            }
        } else {
            static_assert(NP % 4 == 0, "whole float4 vectors");
#pragma unroll
            for (int i = 0; i < NP / 4; ++i) {
                reinterpret_cast<float4 *>(p)[i] =
                    make_float4(x[4 * i], x[4 * i + 1], x[4 * i + 2], x[4 * i + 3]);
            }
        }
    } else {
        float mine = 0.f;
#pragma unroll
        for (int i = 0; i < NP; ++i) {
            mine = (kc == i) ? x[i] : mine;
        }
        if (kc < NP) {
            store1(p + RS * kc, mine);
        }
    }
}

template <int D, int L, int NP, bool CONTIG, int TPS, typename TQK, typename TV, int GATE>
__global__ __launch_bounds__(kThreads) void recurrent_kernel(const KdaRecurrentArgs a) {
    constexpr int E = D / L;           // K elements per lane
    constexpr int EV = E / 4;          // 16-byte vectors per lane and row
    constexpr int RPW = 64 / L;        // row groups per wave
    constexpr int RPP = 4 * RPW;       // row groups per workgroup
    constexpr int RB = RPP * NP;       // rows per workgroup
    // A lane's NP rows: consecutive (CONTIG; v and o then move as one vector
    // per row group) or RPP apart (each wave-wide state load then covers
    // RPW adjacent rows, one contiguous span).
    constexpr int RS = CONTIG ? 1 : RPP;
    // TPS: the tokens per sequence a shape is tuned for -- 1 (decode), 2, or
    // 3 and more. With several, the token loop's instruction count matters
    // and the exponentials are one v_exp_f32 each; decode, bound by the
    // state traffic, keeps the correctly rounded expf.
    auto dexp = [](float x) { return TPS > 1 ? fexp(x) : expf(x); };
    constexpr int VT = D / RB;         // workgroups per (sequence, head)
    static_assert(E % 4 == 0 && D % RB == 0, "whole vectors and whole row tiles");

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
    const int rgw = wave * RPW + lane / L;  // row group in the workgroup
    const int row0 = vt * RB + (CONTIG ? rgw * NP : rgw);  // rows row0 + RS*p, p < NP
    const int T = a.num_tokens;

    int bos = a.cu_seqlens[n];
    int eos = a.cu_seqlens[n + 1];
    bos = bos < 0 ? 0 : (bos > T ? T : bos);
    eos = eos < bos ? bos : (eos > T ? T : eos);
    int slot = a.state_indices[n];
    if (slot < 0 || static_cast<int64_t>(slot) >= a.num_slots) {
        slot = 0;
    }

    // Offset of this lane's vector j within a row of D elements.
    auto koff = [&](int j) { return 4 * kc + 4 * L * j; };
    const int64_t head_off = static_cast<int64_t>(head) * a.state_stride_head;
    // A [K,V]-contiguous pool (state_v_contiguous, the prepared_recurrent
    // layout of the reference; DECAY mode only, the launcher rejects it
    // otherwise, so the other modes compile without it) is read and written
    // in place element by element: element (k, v) of a slot and head sits at
    // k*D + v.
    const bool vpool = GATE == KDA_GATE_DECAY && a.state_v_contiguous != 0;
    float4 S[NP][EV];
    if (slot > 0) {
        const float *src = a.state + slot * a.state_stride_slot + head_off;
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int j = 0; j < EV; ++j) {
                if (vpool) {
                    const float *e = src + static_cast<int64_t>(koff(j)) * D + row0 + RS * p;
                    S[p][j] = make_float4(e[0], e[D], e[2 * D], e[3 * D]);
                } else {
                    S[p][j] = load4_stream(src + static_cast<int64_t>(row0 + RS * p) * D + koff(j));
                }
            }
        }
    } else {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int j = 0; j < EV; ++j) {
                S[p][j] = make_float4(0.f, 0.f, 0.f, 0.f);
            }
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
    auto store_state = [&](float *dst, bool vlayout) {
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int j = 0; j < EV; ++j) {
                if (vlayout) {
                    float *e = dst + static_cast<int64_t>(koff(j)) * D + row0 + RS * p;
                    e[0] = S[p][j].x;
                    e[D] = S[p][j].y;
                    e[2 * D] = S[p][j].z;
                    e[3 * D] = S[p][j].w;
                } else {
                    store4_stream(dst + static_cast<int64_t>(row0 + RS * p) * D + koff(j), S[p][j]);
                }
            }
        }
    };
    if (track_slot > 0 && track_len == 0) {
        store_state(a.state + track_slot * a.state_stride_slot + head_off, vpool);
    }

    // Per-head gate constants (RAW): exp(A_log[h]) and this lane's dt_bias.
    float expA = 0.f;
    float4 dtb[EV];
#pragma unroll
    for (int j = 0; j < EV; ++j) {
        dtb[j] = make_float4(0.f, 0.f, 0.f, 0.f);
    }
    if constexpr (GATE == KDA_GATE_RAW) {
        expA = expf(a.A_log[head]);
#pragma unroll
        for (int j = 0; j < EV; ++j) {
            dtb[j] = load4(a.dt_bias + static_cast<int64_t>(head) * D + koff(j));
        }
    }
    const bool norm = (GATE == KDA_GATE_RAW) || (a.qk_l2norm != 0);
    const bool save_mid = a.intermediate != nullptr && slot > 0 && n < a.mid_rows;

    const TQK *qp = static_cast<const TQK *>(a.q);
    const TQK *kp = static_cast<const TQK *>(a.k);
    const TV *vp = static_cast<const TV *>(a.v);
    TV *op = static_cast<TV *>(a.out);
    using TG = typename std::conditional<GATE == KDA_GATE_RAW, uint16_t, float>::type;
    const TG *gp = static_cast<const TG *>(a.gate);

    // One token's inputs, as loaded; widened and transformed before its
    // step. The next token's are loaded while the current one computes: a
    // multi-token sequence (verify, prefill) would otherwise wait a full load
    // latency per token.
    struct TokenIn {
        Raw4<TQK> q[EV], k[EV];
        Raw4<TG> g[EV];
        RowIn<TV, NP, RS> v;
        float b;
    };
    auto fetch = [&](int t, TokenIn &in) {
        const int64_t base = (static_cast<int64_t>(t) * H + head) * D;
#pragma unroll
        for (int j = 0; j < EV; ++j) {
            in.q[j].load(qp + base + koff(j));
            in.k[j].load(kp + base + koff(j));
            in.g[j].load(gp + base + koff(j));
        }
        in.v.load(vp + base + row0);
        const int64_t bi = static_cast<int64_t>(t) * H + head;
        if constexpr (GATE == KDA_GATE_RAW) {
            in.b = bf16_to_f32(static_cast<const uint16_t *>(a.beta)[bi]);
        } else {
            in.b = static_cast<const float *>(a.beta)[bi];
        }
    };
    // A token ready for the update: scaled q, normalized k, decay, beta, v.
    struct Token {
        float4 q[EV], k[EV], dec[EV];
        float beta;
        float v[NP];
    };
    // Every row group of a workgroup needs the same per-channel decays, beta
    // and norms of a token. With one vector per lane and row (EV == 1: the
    // row groups' L lanes cover the D channels four apiece) and one or two
    // tokens per sequence, the workgroup computes them once and shares them
    // through LDS: the row groups of the waves before kNormWave each take one
    // component of their lanes' vectors (rows groups 0-3: channels 4 kc + r),
    // wave kNormWave forms the q norm (its even row groups) and the k norm
    // (odd ones) with the same group sums every row group would use, and the
    // next wave forms beta. Each value is the same expression of the same
    // inputs as in the per-lane form, so the results are bitwise those of
    // every row group computing everything itself; the raw decode's prologue
    // (two expf and a division per channel) then runs once per (token,
    // channel) in the workgroup instead of once per row group (8x fewer).
    // Tokens alternate between two LDS sets, so one barrier per token
    // separates the writes of token t + 2 from the reads of token t.
    constexpr bool kShare = GATE != KDA_GATE_DECAY && TPS <= 2 && EV == 1;
    constexpr int kNormWave = 4 / RPW;
    static_assert(!kShare || (4 * L == D && kNormWave + 1 < 4), "roles of the shared prologue");
    __shared__ float4 sh_dec[kShare ? 2 : 1][kShare ? L : 1];
    __shared__ float sh_tok[kShare ? 2 : 1][4];
    auto widen = [&](const TokenIn &in, Token &w, int t) {
        if constexpr (kShare) {
            const int par = t & 1;
            w.q[0] = in.q[0].get();
            w.k[0] = in.k[0].get();
            const float4 gv = in.g[0].get();
            if (wave < kNormWave) {
                // this row group's channel 4 kc + r, r = rgw < 4
                const int r = rgw;
                const float x = r == 0 ? gv.x : r == 1 ? gv.y : r == 2 ? gv.z : gv.w;
                float d;
                if constexpr (GATE == KDA_GATE_RAW) {
                    const float db = r == 0 ? dtb[0].x : r == 1 ? dtb[0].y : r == 2 ? dtb[0].z : dtb[0].w;
                    d = dexp(a.lower_bound / (1.0f + dexp(-(expA * (x + db)))));
                } else {
                    d = dexp(x);
                }
                reinterpret_cast<float *>(&sh_dec[par][kc])[r] = d;
            } else if (wave == kNormWave) {
                if (norm) {
                    const bool kr_group = (rgw & 1) != 0;
                    float s = 0.f;
                    s += kr_group ? dot4(w.k[0], w.k[0]) : dot4(w.q[0], w.q[0]);
                    s = group_sum<L>(s);
                    const float inv = 1.0f / sqrtf(s + 1e-6f);
                    if (kc == 0 && rgw < 4 + 2) {
                        sh_tok[par][kr_group ? 1 : 0] = kr_group ? inv : inv * a.scale;
                    }
                }
            } else if (wave == kNormWave + 1) {
                if (kc == 0 && (rgw & (RPW - 1)) == 0) {
                    if constexpr (GATE == KDA_GATE_RAW) {
                        sh_tok[par][2] = 1.0f / (1.0f + dexp(-in.b));
                    } else {
                        sh_tok[par][2] = in.b;
                    }
                }
            }
            __syncthreads();
            w.dec[0] = sh_dec[par][kc];
            w.beta = sh_tok[par][2];
#pragma unroll
            for (int p = 0; p < NP; ++p) {
                w.v[p] = in.v.get(p);
            }
            float qsc = a.scale;
            if (norm) {
                qsc = sh_tok[par][0];
                const float kr = sh_tok[par][1];
                w.k[0] = make_float4(w.k[0].x * kr, w.k[0].y * kr, w.k[0].z * kr, w.k[0].w * kr);
            }
            w.q[0] = make_float4(w.q[0].x * qsc, w.q[0].y * qsc, w.q[0].z * qsc, w.q[0].w * qsc);
            return;
        }
#pragma unroll
        for (int j = 0; j < EV; ++j) {
            w.q[j] = in.q[j].get();
            w.k[j] = in.k[j].get();
            const float4 gv = in.g[j].get();
            if constexpr (GATE == KDA_GATE_RAW) {
                // g = lower_bound / (1 + exp(-(exp(A_log) * (a + dt_bias)))), decay = exp(g)
                const float lb = a.lower_bound;
                w.dec[j].x = dexp(lb / (1.0f + dexp(-(expA * (gv.x + dtb[j].x)))));
                w.dec[j].y = dexp(lb / (1.0f + dexp(-(expA * (gv.y + dtb[j].y)))));
                w.dec[j].z = dexp(lb / (1.0f + dexp(-(expA * (gv.z + dtb[j].z)))));
                w.dec[j].w = dexp(lb / (1.0f + dexp(-(expA * (gv.w + dtb[j].w)))));
            } else if constexpr (GATE == KDA_GATE_LOG) {
                w.dec[j] = make_float4(dexp(gv.x), dexp(gv.y), dexp(gv.z), dexp(gv.w));
            } else {
                w.dec[j] = gv;
            }
        }
        if constexpr (GATE == KDA_GATE_RAW) {
            w.beta = 1.0f / (1.0f + dexp(-in.b));
        } else {
            w.beta = in.b;
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            w.v[p] = in.v.get(p);
        }
        float qsc = a.scale;
        if (norm) {
            // x / sqrt(sum x^2 + 1e-6), eps inside the sqrt; q then scaled.
            float qs = 0.f, ks = 0.f;
#pragma unroll
            for (int j = 0; j < EV; ++j) {
                qs += dot4(w.q[j], w.q[j]);
                ks += dot4(w.k[j], w.k[j]);
            }
            qs = group_sum<L>(qs);
            ks = group_sum<L>(ks);
            const float kr = 1.0f / sqrtf(ks + 1e-6f);
            qsc = (1.0f / sqrtf(qs + 1e-6f)) * a.scale;
#pragma unroll
            for (int j = 0; j < EV; ++j) {
                w.k[j] = make_float4(w.k[j].x * kr, w.k[j].y * kr, w.k[j].z * kr, w.k[j].w * kr);
            }
        }
#pragma unroll
        for (int j = 0; j < EV; ++j) {
            w.q[j] = make_float4(w.q[j].x * qsc, w.q[j].y * qsc, w.q[j].z * qsc, w.q[j].w * qsc);
        }
    };
    // sum over the lane's E elements of s * x, one multiply-add chain
    auto dot_lane = [](const float4 (&sv)[EV], const float4 (&xv)[EV]) {
        float acc = dot4(sv[0], xv[0]);
#pragma unroll
        for (int j = 1; j < EV; ++j) {
            acc = fmaf(sv[j].x, xv[j].x, acc);
            acc = fmaf(sv[j].y, xv[j].y, acc);
            acc = fmaf(sv[j].z, xv[j].z, acc);
            acc = fmaf(sv[j].w, xv[j].w, acc);
        }
        return acc;
    };
    auto step = [&](const Token &w, int t) {
        float pred[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
#pragma unroll
            for (int j = 0; j < EV; ++j) {
                S[p][j].x *= w.dec[j].x;
                S[p][j].y *= w.dec[j].y;
                S[p][j].z *= w.dec[j].z;
                S[p][j].w *= w.dec[j].w;
            }
            pred[p] = dot_lane(S[p], w.k);
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            pred[p] = group_sum<L>(pred[p]);
        }
        float o[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            const float d = (w.v[p] - pred[p]) * w.beta;
#pragma unroll
            for (int j = 0; j < EV; ++j) {
                S[p][j].x += w.k[j].x * d;
                S[p][j].y += w.k[j].y * d;
                S[p][j].z += w.k[j].z * d;
                S[p][j].w += w.k[j].w * d;
            }
            o[p] = dot_lane(S[p], w.q);
        }
        const int step_i = t - bos;
        if (save_mid && step_i < a.mid_steps) {
            store_state(a.intermediate + n * a.mid_stride_req + step_i * a.mid_stride_step +
                            static_cast<int64_t>(head) * a.mid_stride_head,
                        false);
        }
        if (track_slot > 0 && step_i + 1 == track_len) {
            store_state(a.state + track_slot * a.state_stride_slot + head_off, vpool);
        }
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            o[p] = group_sum<L>(o[p]);
        }
        // every lane of the row group holds the sums
        store_row<TV, NP, RS>(op + (static_cast<int64_t>(t) * H + head) * D + row0, o, kc);
    };
    if constexpr (TPS > 2) {
        // One buffer: the next token's loads are issued into it right after
        // the current token is widened, unconditionally (the last token
        // reloads itself), so the buffer is always reloaded, never kept --
        // keeping it would cost register copies and a wait for every
        // outstanding store on the way back to the loop's top.
        if (bos < eos) {
            TokenIn in;
            fetch(bos, in);
            for (int t = bos; t < eos; ++t) {
                Token w;
                widen(in, w, t);
                fetch(t + 1 < eos ? t + 1 : t, in);
                step(w, t);
            }
        }
    } else {
        // One or two tokens per sequence: a second buffer, loaded only when
        // a next token exists (an unconditional reload would be a third of
        // the token loads at two tokens, all of them at one).
        TokenIn cur, nxt;
        if (bos < eos) {
            fetch(bos, cur);
        }
        for (int t = bos; t < eos; ++t) {
            if (t + 1 < eos) {
                fetch(t + 1, nxt);
            }
            Token w;
            widen(cur, w, t);
            step(w, t);
            cur = nxt;
        }
    }

    // Tokens no sequence covers are zero (the reference allocates
    // zeros_like(v), kda_varlen_recurrent.cpp:142): the first request zeroes
    // [0, cu[0]) and the last one [cu[N], T). The DECAY form writes a
    // caller-owned output and touches only the rows its requests cover, as
    // the reference's prepared kernels do (prepared_recurrent.cpp:386-560),
    // so a caller may launch request by request into one buffer.
    auto zero_rows = [&](int t0, int t1) {
        float z[NP];
#pragma unroll
        for (int p = 0; p < NP; ++p) {
            z[p] = 0.f;
        }
        for (int t = t0; t < t1; ++t) {
            store_row<TV, NP, RS>(op + (static_cast<int64_t>(t) * H + head) * D + row0, z, kc);
        }
    };
    if constexpr (GATE != KDA_GATE_DECAY) {
        if (n == 0) {
            zero_rows(0, bos);
        }
        if (n == a.num_seqs - 1) {
            zero_rows(eos, T);
        }
    }

    if (a.intermediate == nullptr && slot > 0) {
        store_state(a.state + slot * a.state_stride_slot + head_off, vpool);
    }
}

using KernelFn = void (*)(const KdaRecurrentArgs);

// Tile shapes: (lanes per row L, rows per lane NP).
enum Shape { kDecode16, kDecode8, kVerify16, kMulti32, kMulti64, kMulti128, kD64Small, kD64Large };

template <int D, typename TQK, typename TV, int GATE>
KernelFn pick_shape(Shape shape) {
    if constexpr (D == 128) {
        switch (shape) {
            case kDecode16: return recurrent_kernel<D, 32, 2, false, 1, TQK, TV, GATE>;
            case kDecode8: return recurrent_kernel<D, 32, 1, false, 1, TQK, TV, GATE>;
            case kVerify16: return recurrent_kernel<D, 16, 1, false, 3, TQK, TV, GATE>;
            case kMulti32: return recurrent_kernel<D, 32, 4, false, 2, TQK, TV, GATE>;
            case kMulti64: return recurrent_kernel<D, 16, 4, true, 3, TQK, TV, GATE>;
            case kMulti128: return recurrent_kernel<D, 16, 8, true, 3, TQK, TV, GATE>;
            default: return nullptr;
        }
    } else {
        switch (shape) {
            case kD64Large: return recurrent_kernel<D, 16, 4, false, 1, TQK, TV, GATE>;
            case kD64Small: return recurrent_kernel<D, 16, 1, false, 1, TQK, TV, GATE>;
            default: return nullptr;
        }
    }
}

template <int D>
KernelFn pick_kernel(int gate, int qk_dtype, int v_dtype, Shape shape) {
    if (gate == KDA_GATE_RAW) {
        if (qk_dtype == KDA_BF16 && v_dtype == KDA_BF16) {
            return pick_shape<D, uint16_t, uint16_t, KDA_GATE_RAW>(shape);
        }
        return nullptr;
    }
    if (gate == KDA_GATE_LOG) {
        if (qk_dtype == KDA_BF16 && v_dtype == KDA_BF16) {
            return pick_shape<D, uint16_t, uint16_t, KDA_GATE_LOG>(shape);
        }
        if (qk_dtype == KDA_F32 && v_dtype == KDA_F32) {
            return pick_shape<D, float, float, KDA_GATE_LOG>(shape);
        }
        return nullptr;
    }
    if (gate == KDA_GATE_DECAY) {
        if (qk_dtype == KDA_F32 && v_dtype == KDA_BF16) {
            return pick_shape<D, float, uint16_t, KDA_GATE_DECAY>(shape);
        }
        if (qk_dtype == KDA_F32 && v_dtype == KDA_F32) {
            return pick_shape<D, float, float, KDA_GATE_DECAY>(shape);
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
    if (a.state_v_contiguous != 0 && a.gate_mode != KDA_GATE_DECAY) {
        return KDA_ERR_UNSUPPORTED;  // the [K,V] pool is the prepared (DECAY) layout
    }
    if (a.num_seqs < 0 || a.num_tokens < 0 || a.num_heads <= 0 || a.num_slots < 0) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    if (a.num_seqs == 0) {
        return KDA_OK;
    }
    // token tensors are never read or written when there are no tokens
    const bool tokens = a.num_tokens > 0;
    if ((tokens && (a.q == nullptr || a.k == nullptr || a.v == nullptr || a.gate == nullptr ||
                    a.beta == nullptr || a.out == nullptr)) ||
        a.state == nullptr || a.state_indices == nullptr || a.cu_seqlens == nullptr) {
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
    // Tile shape at D=128, by tokens per sequence (measured on MI355X,
    // interleaved A/B on one box): one token (decode) -> 32-lane rows, 2 rows
    // per lane: 16-row tiles, eight workgroups per (sequence, head), which
    // stream the state fastest (B=256, H=32: 173 us, against 182 with
    // 32-row tiles); two tokens -> 32-lane rows, 4 rows per lane (32-row
    // tiles: 361 us at 512 x 2 tokens, H=32, against 367 with 16-lane
    // rows); more (verify, recurrent prefill) -> 16-lane rows, whose
    // reductions take four DPP steps instead of five plus a swizzle, with 8
    // consecutive rows per lane (the whole state of a (sequence, head) in one
    // workgroup) so each token's loads and exponentials serve more rows:
    // 1024 x 4 tokens, H=16: 382 us, against 406 with 4 rows per lane, 464
    // with 2 and 432 with 32-lane rows; 256 x 8 tokens, H=32: 265 against
    // 284 and 351. The 8-row-per-lane shape runs three workgroups per CU, so
    // below 1024 pairs the 4-row one (two workgroups per pair) fills the GPU
    // instead. Fewer than 128 pairs: one token per request uses 8-row tiles,
    // 32 lanes per row; several (speculative verify) use 16-row tiles of
    // 16-lane rows with the multi-token loop (2 requests x 4 tokens, H=32:
    // 8.7 us against 12.8 with the decode shape).
    const int64_t pairs = static_cast<int64_t>(a.num_seqs) * kargs.head_count;
    Shape shape;
    int rows_per_wg;
    if (D == 128) {
        const int64_t tokens = a.num_tokens;
        if (pairs < 128) {
            shape = tokens <= a.num_seqs ? kDecode8 : kVerify16;
        } else if (tokens <= a.num_seqs) {
            shape = kDecode16;
        } else if (tokens <= 2 * static_cast<int64_t>(a.num_seqs)) {
            shape = kMulti32;
        } else if (pairs < 1024) {
            shape = kMulti64;
        } else {
            shape = kMulti128;
        }
        // The 16-lane shapes move a lane's consecutive v and o values as one
        // vector of up to 16 bytes; v or out not aligned for that take the
        // 32-row shape, which moves them one element at a time.
        if (shape == kMulti64 || shape == kMulti128) {
            const size_t vbytes = static_cast<size_t>(shape == kMulti128 ? 8 : 4) *
                                  (a.v_dtype == KDA_F32 ? 4 : 2);
            const uintptr_t mis = (reinterpret_cast<uintptr_t>(a.v) |
                                   reinterpret_cast<uintptr_t>(a.out)) &
                                  ((vbytes > 16 ? 16 : vbytes) - 1);
            if (mis != 0) {
                shape = kMulti32;
            }
        }
        rows_per_wg = shape == kDecode8    ? 8
                      : shape == kVerify16 ? 16
                      : shape == kDecode16 ? 16
                      : shape == kMulti32  ? 32
                      : shape == kMulti64  ? 64
                                           : 128;
    } else {
        shape = pairs >= 2048 ? kD64Large : kD64Small;
        rows_per_wg = shape == kD64Large ? 64 : 16;
    }
    KernelFn fn = (D == 128) ? pick_kernel<128>(a.gate_mode, a.qk_dtype, a.v_dtype, shape)
                             : pick_kernel<64>(a.gate_mode, a.qk_dtype, a.v_dtype, shape);
    if (fn == nullptr) {
        return KDA_ERR_UNSUPPORTED;
    }
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
