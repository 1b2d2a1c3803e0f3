// kda_chunk.hip -- chunked KDA prefill (64-token chunks) for gfx950.
//
// Semantics: the chunked WY/UT form of the delta rule with per-channel decay,
// as in the reference's fp32 torch anchor (bench/kda_chunk/kda_python.py:121-186,
// per head at tests/ops/test_kda_chunk.py:140-173) and its Ascend kernel
// (sgl-glm53-ascend-ops/csrc/kda/chunk/kda_varlen_chunk_kernel.cpp). Per chunk
// with G = in-chunk cumsum of the log decay g:
//     Akk[i,j] = sum_k k_i k_j e^(G_i-G_j)  (j<i),   Aqk likewise with q (j<=i)
//     T  = (I + diag(beta) Akk)^-1 diag(beta)
//     w  = T (e^G * k),   u = T v
//     vnew = u - w S,     o = (q e^G) S + Aqk vnew
//     S  <- e^(G_last) * S + (e^(G_last - G) * k)^T vnew
// Sequences of any length are accepted: a short last chunk is zero-padded
// (k = q = v = 0, g = 0, beta = 0), which leaves every equation above exact.
//
// MI355X structure (three launches, one stream, no host synchronization):
//   K0 chunk_index_kernel   prefix sums of ceil(len/64) per sequence, so the
//                           chunk grid is sized on the host from T and N alone;
//   K1 chunk_prepare_kernel one workgroup per (chunk, head), all chunks in
//                           parallel: cumsum, Akk / Aqk on MFMA with exponents
//                           anchored at each 16-row block start (all off-diagonal
//                           factors e^(<=0)), the blocked triangular inverse in
//                           fp32, w and u on MFMA; writes the scan's operands as
//                           ready MFMA fragments;
//   K2 chunk_scan_kernel    one workgroup per (sequence, head, 16 value
//                           columns), the serial chunk recurrence: four waves
//                           split the rows of each product and exchange S and
//                           vnew through LDS; S stays fp32 in registers.
//
// MFMA: v_mfma_f32_16x16x32_bf16 with fp32 accumulation. Operands whose
// rounding would break the tolerance contract are carried as bf16 hi + lo
// pairs (x = hi + lo to ~2^-17) and multiplied in three passes
// (hi*hi + hi*lo + lo*hi): u = T v (T split, v exact), Aqk, q e^G, Aqk vnew and
// the state update; Akk, w and w S run single-pass.
//
// Fragment conventions (lane l, r = l % 16, g = l / 16), shared by A and B so
// that C-layout accumulators can be fed back as B operands without moving
// data. Within a 32-wide K slice, lane group g carries the K indices
//     kperm(g, e) = 4g + e (e < 4),  16 + 4g + (e - 4) (e >= 4);
//   A fragment (16 x 32): lane l holds A[r][kperm(g, e)], e = 0..7;
//   B fragment (32 x 16): lane l holds B[kperm(g, e)][r];
//   C tile (16 x 16):     lane l holds C[4g + i][r], i = 0..3.
// Any assignment of K indices works as long as A and B agree, so the
// hardware's own K order does not matter; this one makes the two C tiles
// covering K rows [32s, 32s+16) and [32s+16, 32s+32) exactly the B fragment
// of slice s.

#include <hip/hip_runtime.h>

#include "kda_abi.h"
#include "kda_device.h"

namespace kda {
namespace chunk {

constexpr int BT = 64;   // tokens per chunk
constexpr int DK = 128;  // K == V
constexpr int kThreads = 256;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Workspace record of one (chunk, head), in 16-byte-per-lane fragments
// (a fragment is 64 lanes x 16 B = 1 KiB).
constexpr int kFrag = 1024;
constexpr int kOffW = 0;                          // w hi: A (mt 0..3, s 0..3)
constexpr int kOffQgH = kOffW + 16 * kFrag;       // q e^G hi: A (mt, s)
constexpr int kOffQgL = kOffQgH + 16 * kFrag;     // q e^G lo
constexpr int kOffAqH = kOffQgL + 16 * kFrag;     // Aqk hi: A (mt 0..3, s 0..1)
constexpr int kOffAqL = kOffAqH + 8 * kFrag;      // Aqk lo
constexpr int kOffKdH = kOffAqL + 8 * kFrag;      // kd^T hi: A (mk 0..7, s 0..1)
constexpr int kOffKdL = kOffKdH + 16 * kFrag;     // kd^T lo
constexpr int kOffU = kOffKdL + 16 * kFrag;       // u fp32: C (mt 0..3, vt 0..7)
constexpr int kOffGl = kOffU + 32 * kFrag;        // e^(G_last) fp32 [128]
constexpr int kRecBytes = kOffGl + DK * 4;        // 131584
// Track record of one (sequence, head): operands of the state after r < len
// tokens of the chunk holding the tracked position.
constexpr int kTrOffKdH = 0;
constexpr int kTrOffKdL = kTrOffKdH + 16 * kFrag;
constexpr int kTrOffGl = kTrOffKdL + 16 * kFrag;
constexpr int kTrBytes = kTrOffGl + DK * 4;       // 33280
static_assert(kRecBytes % 256 == 0 && kTrBytes % 256 == 0, "records stay 256-B aligned");

struct Layout {
    size_t chunk_start;  // int32 [N+1]
    size_t recs;         // kRecBytes x (max_chunks x H)
    size_t tracks;       // kTrBytes x (N x H)
    size_t total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline int max_chunks(int T, int N) { return (T + BT - 1) / BT + N; }

__host__ __device__ inline Layout layout(int T, int N, int H) {
    Layout L;
    L.chunk_start = 0;
    L.recs = align256(static_cast<size_t>(N + 1) * 4);
    L.tracks = L.recs + static_cast<size_t>(kRecBytes) * max_chunks(T, N) * H;
    L.total = L.tracks + static_cast<size_t>(kTrBytes) * N * H;
    return L;
}

__device__ __forceinline__ int kperm(int g, int e) { return e < 4 ? 4 * g + e : 12 + 4 * g + e; }

__device__ __forceinline__ f32x4 mfma(bf16x8 a, bf16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ uint32_t pack2(uint16_t lo, uint16_t hi) {
    return static_cast<uint32_t>(lo) | (static_cast<uint32_t>(hi) << 16);
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(bf16x8 v) { return __builtin_bit_cast(u32x4, v); }

// x[8] -> bf16 hi (+ lo) fragments.
__device__ __forceinline__ bf16x8 to_bf16x8(const float x[8]) {
    u32x4 h;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        h[p] = pack2(f32_to_bf16(x[2 * p]), f32_to_bf16(x[2 * p + 1]));
    }
    return as_bf16x8(h);
}
__device__ __forceinline__ void split_bf16x8(const float x[8], bf16x8 &hi, bf16x8 &lo) {
    u32x4 h, l;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint16_t h0 = f32_to_bf16(x[2 * p]);
        const uint16_t h1 = f32_to_bf16(x[2 * p + 1]);
        const uint16_t l0 = f32_to_bf16(x[2 * p] - bf16_to_f32(h0));
        const uint16_t l1 = f32_to_bf16(x[2 * p + 1] - bf16_to_f32(h1));
        h[p] = pack2(h0, h1);
        l[p] = pack2(l0, l1);
    }
    hi = as_bf16x8(h);
    lo = as_bf16x8(l);
}

__device__ __forceinline__ void store_frag(char *base, int off, int idx, int lane, bf16x8 v) {
    reinterpret_cast<u32x4 *>(base + off)[idx * 64 + lane] = as_u32x4(v);
}
__device__ __forceinline__ bf16x8 load_frag(const char *base, int off, int idx, int lane) {
    return as_bf16x8(reinterpret_cast<const u32x4 *>(base + off)[idx * 64 + lane]);
}

__device__ __forceinline__ void seq_bounds(const KdaChunkArgs &a, int n, int &bos, int &eos) {
    const int T = a.num_tokens;
    bos = a.cu_seqlens[n];
    eos = a.cu_seqlens[n + 1];
    bos = bos < 0 ? 0 : (bos > T ? T : bos);
    eos = eos < bos ? bos : (eos > T ? T : eos);
}

// ---------------------------------------------------------------------------
// K0: chunk_start[n] = sum_{m<n} ceil(len_m / 64), chunk_start[N] = total.
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(1024) void chunk_index_kernel(const KdaChunkArgs a, int *cs) {
    __shared__ int part[1024];
    const int N = a.num_seqs;
    const int tid = threadIdx.x;
    const int per = (N + 1023) / 1024;
    const int begin = tid * per;
    const int end = begin + per < N ? begin + per : N;
    int sum = 0;
    for (int n = begin; n < end; ++n) {
        int bos, eos;
        seq_bounds(a, n, bos, eos);
        sum += (eos - bos + BT - 1) / BT;
    }
    part[tid] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int add = tid >= off ? part[tid - off] : 0;
        __syncthreads();
        part[tid] += add;
        __syncthreads();
    }
    int run = tid == 0 ? 0 : part[tid - 1];
    for (int n = begin; n < end; ++n) {
        cs[n] = run;
        int bos, eos;
        seq_bounds(a, n, bos, eos);
        run += (eos - bos + BT - 1) / BT;
    }
    if (tid == 1023) {
        cs[N] = part[1023];
    }
}

// ---------------------------------------------------------------------------
// K1: per (chunk, head) intra-chunk work.
// ---------------------------------------------------------------------------

constexpr int kPadF = 132;  // fp32 row stride of [64][128] tiles (bank spread)
constexpr int kPadV = 72;   // u16 row stride of [128][64] transposed tiles
constexpr int kPadX = 68;   // fp32 row stride of [64][64] tiles

struct PrepShared {
    float G[BT][kPadF];         // cumsum of the log decay
    float K[BT][kPadF];         // normalized k
    float Q[BT][kPadF];         // normalized, scaled q; later e^G k (bf16, [k][t])
    uint16_t Vt[DK][kPadV];     // v^T, bf16 bits
    float L[BT][BT + 1];        // diag(beta) strict-lower Akk
    float X[BT][kPadX];         // (I + L)^-1, then T = X diag(beta)
    float beta[BT];
    float carry[DK];
};

template <typename TIn, int GATE>
__global__ __launch_bounds__(kThreads) void chunk_prepare_kernel(const KdaChunkArgs a, char *ws,
                                                                 int nrec) {
    __shared__ PrepShared sm;
    const int c = blockIdx.x;
    const int h = blockIdx.y;
    const int H = a.num_heads;
    const int N = a.num_seqs;
    const Layout LY = layout(a.num_tokens, N, H);
    const int *cs = reinterpret_cast<const int *>(ws + LY.chunk_start);
    if (c >= cs[N] || c >= nrec) {
        return;
    }
    int lo = 0, hi = N - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (cs[mid] <= c) {
            lo = mid;
        } else {
            hi = mid - 1;
        }
    }
    const int n = lo;
    const int jc = c - cs[n];
    int bos, eos;
    seq_bounds(a, n, bos, eos);
    const int t0 = bos + BT * jc;
    const int len = eos - t0 < BT ? eos - t0 : BT;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int gq = lane >> 4;
    char *rec = ws + LY.recs + (static_cast<size_t>(c) * H + h) * kRecBytes;

    // ---- S1: load rows (zero-padded), gates, norms -------------------------
    {
        const int kc = tid & 31;
        const int rg = tid >> 5;
        const TIn *qp = static_cast<const TIn *>(a.q);
        const TIn *kp = static_cast<const TIn *>(a.k);
        const uint16_t *vp = static_cast<const uint16_t *>(a.v);
        const bool norm = GATE == KDA_GATE_RAW || a.qk_l2norm != 0;
        float expA = 0.f;
        float4 dtb = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (GATE == KDA_GATE_RAW) {
            expA = expf(a.A_log[h]);
            dtb = load4(a.dt_bias + static_cast<int64_t>(h) * DK + 4 * kc);
        }
#pragma unroll 2
        for (int i = 0; i < 8; ++i) {
            const int t = rg + 8 * i;
            const bool valid = t < len;
            const int64_t base = (static_cast<int64_t>(t0 + t) * H + h) * DK + 4 * kc;
            float4 q4 = make_float4(0.f, 0.f, 0.f, 0.f), k4 = q4, g4 = q4;
            uint2 vraw = make_uint2(0u, 0u);
            if (valid) {
                q4 = load4(qp + base);
                k4 = load4(kp + base);
                vraw = *reinterpret_cast<const uint2 *>(vp + base);
                if constexpr (GATE == KDA_GATE_RAW) {
                    const float4 av = load4(static_cast<const uint16_t *>(a.gate) + base);
                    const float lb = a.lower_bound;
                    g4.x = lb / (1.0f + expf(-(expA * (av.x + dtb.x))));
                    g4.y = lb / (1.0f + expf(-(expA * (av.y + dtb.y))));
                    g4.z = lb / (1.0f + expf(-(expA * (av.z + dtb.z))));
                    g4.w = lb / (1.0f + expf(-(expA * (av.w + dtb.w))));
                } else {
                    g4 = load4(static_cast<const float *>(a.gate) + base);
                }
            }
            if (norm) {
                const float qd = sqrtf(group_sum32(dot4(q4, q4)) + 1e-6f);
                const float kd = sqrtf(group_sum32(dot4(k4, k4)) + 1e-6f);
                q4 = make_float4(q4.x / qd, q4.y / qd, q4.z / qd, q4.w / qd);
                k4 = make_float4(k4.x / kd, k4.y / kd, k4.z / kd, k4.w / kd);
            }
            const float sc = a.scale;
            float *Qr = &sm.Q[t][4 * kc];
            Qr[0] = q4.x * sc;
            Qr[1] = q4.y * sc;
            Qr[2] = q4.z * sc;
            Qr[3] = q4.w * sc;
            float *Kr = &sm.K[t][4 * kc];
            Kr[0] = k4.x;
            Kr[1] = k4.y;
            Kr[2] = k4.z;
            Kr[3] = k4.w;
            float *Gr = &sm.G[t][4 * kc];
            Gr[0] = g4.x;
            Gr[1] = g4.y;
            Gr[2] = g4.z;
            Gr[3] = g4.w;
            sm.Vt[4 * kc + 0][t] = static_cast<uint16_t>(vraw.x & 0xffffu);
            sm.Vt[4 * kc + 1][t] = static_cast<uint16_t>(vraw.x >> 16);
            sm.Vt[4 * kc + 2][t] = static_cast<uint16_t>(vraw.y & 0xffffu);
            sm.Vt[4 * kc + 3][t] = static_cast<uint16_t>(vraw.y >> 16);
        }
        if (tid < BT) {
            float b = 0.f;
            if (tid < len) {
                const int64_t bi = static_cast<int64_t>(t0 + tid) * H + h;
                if constexpr (GATE == KDA_GATE_RAW) {
                    b = 1.0f / (1.0f + expf(-bf16_to_f32(static_cast<const uint16_t *>(a.beta)[bi])));
                } else {
                    b = static_cast<const float *>(a.beta)[bi];
                }
            }
            sm.beta[tid] = b;
        }
    }
    __syncthreads();

    // ---- S2: in-chunk cumsum of g, per channel ------------------------------
    {
        const int ch = tid & 127;
        const int half = tid >> 7;
        float vals[32];
        float run = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            run += sm.G[half * 32 + i][ch];
            vals[i] = run;
        }
        if (half == 0) {
            sm.carry[ch] = run;
        }
        __syncthreads();
        const float add = half ? sm.carry[ch] : 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            sm.G[half * 32 + i][ch] = vals[i] + add;
        }
    }
    __syncthreads();

    // ---- S3: Akk (-> LDS) and Aqk (-> fragments), wave = 16-row block I ----
    {
        const int I = wave;
        const int ri = 16 * I + r;
        bf16x8 Rh[4], Qh[4], Ql[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            float rv[8], qv[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int k = 32 * s + kperm(gq, e);
                const float ex = expf(sm.G[ri][k] - sm.G[16 * I][k]);
                rv[e] = sm.K[ri][k] * ex;
                qv[e] = sm.Q[ri][k] * ex;
            }
            Rh[s] = to_bf16x8(rv);
            split_bf16x8(qv, Qh[s], Ql[s]);
        }
        float aq[4][4];
#pragma unroll
        for (int J = 0; J < 4; ++J) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                aq[J][e] = 0.f;
            }
            if (J > I) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    sm.L[16 * I + 4 * gq + e][16 * J + r] = 0.f;
                }
                continue;
            }
            const int rj = 16 * J + r;
            f32x4 akk = {0.f, 0.f, 0.f, 0.f};
            f32x4 aqt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                float cv[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int k = 32 * s + kperm(gq, e);
                    cv[e] = sm.K[rj][k] * expf(sm.G[16 * I][k] - sm.G[rj][k]);
                }
                bf16x8 Ch, Cl;
                split_bf16x8(cv, Ch, Cl);
                akk = mfma(Rh[s], Ch, akk);  // Akk[i][j]: rows i of block I
                aqt = mfma(Ch, Qh[s], aqt);  // Aqk^T[j][i]
                aqt = mfma(Ch, Ql[s], aqt);
                aqt = mfma(Cl, Qh[s], aqt);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 16 * I + 4 * gq + e;
                const int j = 16 * J + r;
                sm.L[i][j] = j < i ? akk[e] * sm.beta[i] : 0.f;
                // aqt holds Aqk[16I + r][16J + 4gq + e]
                aq[J][e] = (16 * J + 4 * gq + e) <= ri ? aqt[e] : 0.f;
            }
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                x[e] = aq[2 * s][e];
                x[4 + e] = aq[2 * s + 1][e];
            }
            bf16x8 fh, fl;
            split_bf16x8(x, fh, fl);
            store_frag(rec, kOffAqH, I * 2 + s, lane, fh);
            store_frag(rec, kOffAqL, I * 2 + s, lane, fl);
        }
    }
    __syncthreads();

    // ---- S4: q e^G, kd^T, e^(G_last), tracking operands ---------------------
    {
        // q e^G: fragments (mt = wave, s)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int t = 16 * wave + r;
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int k = 32 * s + kperm(gq, e);
                x[e] = sm.Q[t][k] * expf(sm.G[t][k]);
            }
            bf16x8 fh, fl;
            split_bf16x8(x, fh, fl);
            store_frag(rec, kOffQgH, wave * 4 + s, lane, fh);
            store_frag(rec, kOffQgL, wave * 4 + s, lane, fl);
        }
        // kd^T[k][t] = k_t e^(G_last - G_t): fragments (mk = 2*wave + tt, s)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int mk = 2 * wave + tt;
            const int k = 16 * mk + r;
            const float gl = sm.G[BT - 1][k];
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                float x[8];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int t = 32 * s + kperm(gq, e);
                    x[e] = sm.K[t][k] * expf(gl - sm.G[t][k]);
                }
                bf16x8 fh, fl;
                split_bf16x8(x, fh, fl);
                store_frag(rec, kOffKdH, mk * 2 + s, lane, fh);
                store_frag(rec, kOffKdL, mk * 2 + s, lane, fl);
            }
        }
        if (tid < DK) {
            reinterpret_cast<float *>(rec + kOffGl)[tid] = expf(sm.G[BT - 1][tid]);
        }
        // The tracked prefix inside this chunk (0 < rr < len): its state is
        // e^(G_{rr-1}) S + (e^(G_{rr-1} - G_t) k_t)_{t<rr}^T vnew.
        if (a.track_indices != nullptr) {
            const int ts = a.track_indices[n];
            const int tl = a.track_lens[n];
            const int rr = tl - BT * jc;
            if (ts > 0 && static_cast<int64_t>(ts) < a.num_slots && rr > 0 && rr < len) {
                char *tr = ws + LY.tracks + (static_cast<size_t>(n) * H + h) * kTrBytes;
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    const int mk = 2 * wave + tt;
                    const int k = 16 * mk + r;
                    const float gr = sm.G[rr - 1][k];
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        float x[8];
#pragma unroll
                        for (int e = 0; e < 8; ++e) {
                            const int t = 32 * s + kperm(gq, e);
                            x[e] = t < rr ? sm.K[t][k] * expf(gr - sm.G[t][k]) : 0.f;
                        }
                        bf16x8 fh, fl;
                        split_bf16x8(x, fh, fl);
                        store_frag(tr, kTrOffKdH, mk * 2 + s, lane, fh);
                        store_frag(tr, kTrOffKdL, mk * 2 + s, lane, fl);
                    }
                }
                if (tid < DK) {
                    reinterpret_cast<float *>(tr + kTrOffGl)[tid] = expf(sm.G[rr - 1][tid]);
                }
            }
        }
    }
    __syncthreads();
    // e^G k as bf16, transposed [k][t], over the q tile (no longer needed).
    uint16_t(*KE)[kPadV] = reinterpret_cast<uint16_t(*)[kPadV]>(&sm.Q[0][0]);
    {
        const int k = tid & 127;
        const int half = tid >> 7;
#pragma unroll 8
        for (int i = 0; i < 32; ++i) {
            const int t = half * 32 + i;
            KE[k][t] = f32_to_bf16(sm.K[t][k] * expf(sm.G[t][k]));
        }
    }

    // ---- S5: X = (I + L)^-1 (blocked, fp32), then T = X diag(beta) ----------
    {
        // upper blocks of X are zero; diagonal blocks by forward substitution
        for (int idx = tid; idx < BT * BT; idx += kThreads) {
            const int i = idx >> 6;
            const int j = idx & 63;
            if ((j >> 4) > (i >> 4)) {
                sm.X[i][j] = 0.f;
            }
        }
        if (lane < 16) {
            const int b0 = 16 * wave;
            const int col = lane;
            float x[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                float acc = i == col ? 1.f : 0.f;
#pragma unroll
                for (int jj = 0; jj < i; ++jj) {
                    acc -= sm.L[b0 + i][b0 + jj] * x[jj];
                }
                x[i] = acc;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                sm.X[b0 + i][b0 + col] = x[i];
            }
        }
    }
    __syncthreads();
    // Off-diagonal blocks by level d = I - J:
    //   M_IJ = sum_{K=J}^{I-1} L_IK X_KJ,  X_IJ = -X_II M_IJ.
    // M_IJ is parked in the (still zero) upper block (J, I) of X.
    for (int d = 1; d < 4; ++d) {
        const int nb = 4 - d;
        for (int idx = tid; idx < nb * 256; idx += kThreads) {
            const int J = idx >> 8;
            const int I = J + d;
            const int i = (idx >> 4) & 15;
            const int jj = idx & 15;
            float acc = 0.f;
            for (int kk = 16 * J; kk < 16 * I; ++kk) {
                acc += sm.L[16 * I + i][kk] * sm.X[kk][16 * J + jj];
            }
            sm.X[16 * J + jj][16 * I + i] = acc;  // M_IJ[i][jj], transposed into (J, I)
        }
        __syncthreads();
        for (int idx = tid; idx < nb * 256; idx += kThreads) {
            const int J = idx >> 8;
            const int I = J + d;
            const int i = (idx >> 4) & 15;
            const int jj = idx & 15;
            float acc = 0.f;
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                acc += sm.X[16 * I + i][16 * I + kk] * sm.X[16 * J + jj][16 * I + kk];
            }
            sm.X[16 * I + i][16 * J + jj] = -acc;
        }
        __syncthreads();
        for (int idx = tid; idx < nb * 256; idx += kThreads) {
            const int J = idx >> 8;
            const int I = J + d;
            const int i = (idx >> 4) & 15;
            const int jj = idx & 15;
            sm.X[16 * J + jj][16 * I + i] = 0.f;
        }
        __syncthreads();
    }
    for (int idx = tid; idx < BT * BT; idx += kThreads) {
        const int i = idx >> 6;
        const int j = idx & 63;
        sm.X[i][j] *= sm.beta[j];
    }
    __syncthreads();

    // ---- S6: u = T v (T split) and w^T = (e^G k)^T T^T (single) --------------
    {
        const int t = 16 * wave + r;
        const int nS = wave >= 2 ? 2 : 1;  // T is lower triangular
        bf16x8 Th[2], Tl[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                x[e] = sm.X[t][32 * s + kperm(gq, e)];
            }
            split_bf16x8(x, Th[s], Tl[s]);
        }
        // u tiles (mt = wave, vt): A = T rows, B = v (K = j)
        for (int vt = 0; vt < 8; ++vt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            for (int s = 0; s < nS; ++s) {
                const uint16_t *vr = &sm.Vt[16 * vt + r][32 * s];
                const uint2 v0 = *reinterpret_cast<const uint2 *>(vr + 4 * gq);
                const uint2 v1 = *reinterpret_cast<const uint2 *>(vr + 16 + 4 * gq);
                const bf16x8 vb = as_bf16x8(u32x4{v0.x, v0.y, v1.x, v1.y});
                acc = mfma(Th[s], vb, acc);
                acc = mfma(Tl[s], vb, acc);
            }
            reinterpret_cast<f32x4 *>(rec + kOffU)[(wave * 8 + vt) * 64 + lane] = acc;
        }
        // w^T tiles (mk, nt = wave): A = (e^G k)^T rows k, B = T^T (K = j)
        for (int sp = 0; sp < 4; ++sp) {
            float x[8];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int mk = 2 * sp + half;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
                for (int s = 0; s < nS; ++s) {
                    const uint16_t *kr = &KE[16 * mk + r][32 * s];
                    const uint2 k0 = *reinterpret_cast<const uint2 *>(kr + 4 * gq);
                    const uint2 k1 = *reinterpret_cast<const uint2 *>(kr + 16 + 4 * gq);
                    const bf16x8 kb = as_bf16x8(u32x4{k0.x, k0.y, k1.x, k1.y});
                    acc = mfma(kb, Th[s], acc);
                }
                // acc[i] = w[16*wave + r][16*mk + 4gq + i]
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    x[4 * half + i] = acc[i];
                }
            }
            store_frag(rec, kOffW, wave * 4 + sp, lane, to_bf16x8(x));
        }
    }
}

// ---------------------------------------------------------------------------
// K2: the serial chunk scan per (sequence, head, 16 value columns).
// ---------------------------------------------------------------------------

__global__ __launch_bounds__(kThreads) void chunk_scan_kernel(const KdaChunkArgs a, const char *ws) {
    __shared__ u32x4 sfrag[4][2][64];     // S as B fragments, slice s = k rows [32s, 32s+32)
    __shared__ uint32_t vfrag[2][2][64][4];  // vnew as B fragments, slice s = tokens [32s, 32s+32)

    const int H = a.num_heads;
    const int N = a.num_seqs;
    const int pairs = N * H;
    // XCD-aware order: the 8 column tiles of one (sequence, head) share an XCD
    // (and its L2), since they read the same chunk records.
    const int b = blockIdx.x;
    const int xcd = b & 7;
    const int rest = b >> 3;
    const int vt = rest & 7;
    const int pair = (rest >> 3) * 8 + xcd;
    if (pair >= pairs) {
        return;
    }
    const int n = pair / H;
    const int h = pair - n * H;
    const Layout LY = layout(a.num_tokens, N, H);
    const int *cs = reinterpret_cast<const int *>(ws + LY.chunk_start);
    int bos, eos;
    seq_bounds(a, n, bos, eos);
    const int c0 = cs[n];
    const int nch = cs[n + 1] - c0;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int gq = lane >> 4;
    const int vcol = 16 * vt + r;

    int slot = a.state_indices[n];
    if (slot < 0 || static_cast<int64_t>(slot) >= a.num_slots) {
        slot = 0;
    }
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
    const int64_t head_off = static_cast<int64_t>(h) * a.state_stride_head;

    // S rows k in [32w, 32w+32): tiles kt = 2w + tt, lane holds S[16kt + 4gq + i][vcol].
    f32x4 S[2];
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        if (slot > 0) {
            const float *src = a.state + slot * a.state_stride_slot + head_off +
                               static_cast<int64_t>(vcol) * DK + 16 * (2 * w + tt) + 4 * gq;
            const float4 s4 = load4(src);
            S[tt] = f32x4{s4.x, s4.y, s4.z, s4.w};
        } else {
            S[tt] = f32x4{0.f, 0.f, 0.f, 0.f};
        }
    }
    auto store_S = [&](int dst_slot, const f32x4 *val) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            float *dst = a.state + dst_slot * a.state_stride_slot + head_off +
                         static_cast<int64_t>(vcol) * DK + 16 * (2 * w + tt) + 4 * gq;
            *reinterpret_cast<float4 *>(dst) = make_float4(val[tt][0], val[tt][1], val[tt][2], val[tt][3]);
        }
    };
    if (track_slot > 0 && track_len == 0) {
        store_S(track_slot, S);
    }

    uint16_t *out = static_cast<uint16_t *>(a.out);
    const char *tr = ws + LY.tracks + (static_cast<size_t>(n) * H + h) * kTrBytes;

    for (int j = 0; j < nch; ++j) {
        const char *rec = ws + LY.recs + (static_cast<size_t>(c0 + j) * H + h) * kRecBytes;
        const int t0 = bos + BT * j;
        const int len = eos - t0 < BT ? eos - t0 : BT;

        // operands of this chunk
        bf16x8 Wf[4], Qh[4], Ql[4], Ah[2], Al[2], Kh[2][2], Kl[2][2];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            Wf[s] = load_frag(rec, kOffW, w * 4 + s, lane);
            Qh[s] = load_frag(rec, kOffQgH, w * 4 + s, lane);
            Ql[s] = load_frag(rec, kOffQgL, w * 4 + s, lane);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            Ah[s] = load_frag(rec, kOffAqH, w * 2 + s, lane);
            Al[s] = load_frag(rec, kOffAqL, w * 2 + s, lane);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                Kh[tt][s] = load_frag(rec, kOffKdH, (2 * w + tt) * 2 + s, lane);
                Kl[tt][s] = load_frag(rec, kOffKdL, (2 * w + tt) * 2 + s, lane);
            }
        }
        const f32x4 u = reinterpret_cast<const f32x4 *>(rec + kOffU)[(w * 8 + vt) * 64 + lane];
        f32x4 gl[2];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            gl[tt] = *reinterpret_cast<const f32x4 *>(rec + kOffGl + 4 * (16 * (2 * w + tt) + 4 * gq));
        }

        // 1. publish S (slice s = w) as hi/lo B fragments
        {
            float x[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[i] = S[0][i];
                x[4 + i] = S[1][i];
            }
            bf16x8 hi, lo;
            split_bf16x8(x, hi, lo);
            sfrag[w][0][lane] = as_u32x4(hi);
            sfrag[w][1][lane] = as_u32x4(lo);
        }
        __syncthreads();

        // 2. vnew rows [16w, 16w+16) = u - w S ; 3. o = (q e^G) S (3-pass)
        f32x4 ws_acc = {0.f, 0.f, 0.f, 0.f};
        f32x4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8 sh = as_bf16x8(sfrag[s][0][lane]);
            const bf16x8 sl = as_bf16x8(sfrag[s][1][lane]);
            ws_acc = mfma(Wf[s], sh, ws_acc);
            o = mfma(Qh[s], sh, o);
            o = mfma(Qh[s], sl, o);
            o = mfma(Ql[s], sh, o);
        }
        f32x4 vn;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vn[i] = u[i] - ws_acc[i];
        }
        // 4. publish vnew (tile mt = w is half w%2 of slice w/2)
        {
            uint32_t hp[2], lp[2];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                const uint16_t h0 = f32_to_bf16(vn[2 * p]);
                const uint16_t h1 = f32_to_bf16(vn[2 * p + 1]);
                const uint16_t l0 = f32_to_bf16(vn[2 * p] - bf16_to_f32(h0));
                const uint16_t l1 = f32_to_bf16(vn[2 * p + 1] - bf16_to_f32(h1));
                hp[p] = pack2(h0, h1);
                lp[p] = pack2(l0, l1);
            }
            const int sl = w >> 1;
            const int hf = (w & 1) * 2;
            vfrag[sl][0][lane][hf] = hp[0];
            vfrag[sl][0][lane][hf + 1] = hp[1];
            vfrag[sl][1][lane][hf] = lp[0];
            vfrag[sl][1][lane][hf + 1] = lp[1];
        }
        __syncthreads();

        bf16x8 vh[2], vl[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            vh[s] = as_bf16x8(u32x4{vfrag[s][0][lane][0], vfrag[s][0][lane][1], vfrag[s][0][lane][2],
                                    vfrag[s][0][lane][3]});
            vl[s] = as_bf16x8(u32x4{vfrag[s][1][lane][0], vfrag[s][1][lane][1], vfrag[s][1][lane][2],
                                    vfrag[s][1][lane][3]});
        }
        // 5. o += Aqk vnew (3-pass) and store rows t < len
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            o = mfma(Ah[s], vh[s], o);
            o = mfma(Ah[s], vl[s], o);
            o = mfma(Al[s], vh[s], o);
        }
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int t = 16 * w + 4 * gq + i;
            if (t < len) {
                out[(static_cast<int64_t>(t0 + t) * H + h) * DK + vcol] = f32_to_bf16(o[i]);
            }
        }
        // tracked prefix strictly inside this chunk
        const int rr = track_len - BT * j;
        if (track_slot > 0 && rr > 0 && rr < len) {
            f32x4 St[2];
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const f32x4 g2 = *reinterpret_cast<const f32x4 *>(tr + kTrOffGl +
                                                                  4 * (16 * (2 * w + tt) + 4 * gq));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    St[tt][i] = S[tt][i] * g2[i];
                }
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const bf16x8 th = load_frag(tr, kTrOffKdH, (2 * w + tt) * 2 + s, lane);
                    const bf16x8 tl = load_frag(tr, kTrOffKdL, (2 * w + tt) * 2 + s, lane);
                    St[tt] = mfma(th, vh[s], St[tt]);
                    St[tt] = mfma(th, vl[s], St[tt]);
                    St[tt] = mfma(tl, vh[s], St[tt]);
                }
            }
            store_S(track_slot, St);
        }
        // 6. S <- e^(G_last) S + kd^T vnew (3-pass)
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                S[tt][i] *= gl[tt][i];
            }
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                S[tt] = mfma(Kh[tt][s], vh[s], S[tt]);
                S[tt] = mfma(Kh[tt][s], vl[s], S[tt]);
                S[tt] = mfma(Kl[tt][s], vh[s], S[tt]);
            }
        }
        if (track_slot > 0 && rr == len) {
            store_S(track_slot, S);
        }
    }

    // Tokens outside every sequence are written as zero.
    auto zero_rows = [&](int ta, int tb) {
        for (int t = ta + tid / 16; t < tb; t += kThreads / 16) {
            if ((tid & 15) == 0) {
                // one thread per token row writes this tile's 16 columns
                for (int cidx = 0; cidx < 16; ++cidx) {
                    out[(static_cast<int64_t>(t) * H + h) * DK + 16 * vt + cidx] = 0;
                }
            }
        }
    };
    if (n == 0) {
        zero_rows(0, bos);
    }
    if (n == N - 1) {
        zero_rows(eos, a.num_tokens);
    }
    if (slot > 0) {
        store_S(slot, S);
    }
}

bool aligned(const void *p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; }

}  // namespace chunk
}  // namespace kda

extern "C" size_t kda_chunk_workspace_bytes(int32_t num_tokens, int32_t num_seqs,
                                            int32_t num_heads, int32_t head_dim) {
    if (num_tokens < 0 || num_seqs < 0 || num_heads <= 0 || head_dim != kda::chunk::DK) {
        return 0;
    }
    return kda::chunk::layout(num_tokens, num_seqs, num_heads).total;
}

extern "C" int kda_chunk_launch(const KdaChunkArgs *args, void *workspace, size_t workspace_bytes,
                                void *stream) {
    using namespace kda::chunk;
    if (args == nullptr) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    const KdaChunkArgs &a = *args;
    if (a.head_dim != DK) {
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
    if (a.qk_dtype != KDA_BF16 || a.v_dtype != KDA_BF16 ||
        (a.gate_mode != KDA_GATE_RAW && a.gate_mode != KDA_GATE_LOG)) {
        return KDA_ERR_UNSUPPORTED;
    }
    if (!aligned(a.state, 16) || (a.state_stride_slot & 3) || (a.state_stride_head & 3) ||
        !aligned(a.q, 8) || !aligned(a.k, 8) || !aligned(a.v, 8) ||
        !aligned(a.gate, a.gate_mode == KDA_GATE_RAW ? 8 : 16)) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    const Layout LY = layout(a.num_tokens, a.num_seqs, a.num_heads);
    if (workspace == nullptr || workspace_bytes < LY.total || !aligned(workspace, 256)) {
        return KDA_ERR_WORKSPACE;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
    KdaChunkArgs kargs = a;
    int *cs = reinterpret_cast<int *>(ws + LY.chunk_start);
    {
        void *params[] = {&kargs, &cs};
        if (hipLaunchKernel(reinterpret_cast<const void *>(chunk_index_kernel), dim3(1), dim3(1024),
                            params, 0, st) != hipSuccess) {
            return KDA_ERR_LAUNCH;
        }
    }
    const int nrec = max_chunks(a.num_tokens, a.num_seqs);
    {
        const void *fn = a.gate_mode == KDA_GATE_RAW
                             ? reinterpret_cast<const void *>(chunk_prepare_kernel<uint16_t, KDA_GATE_RAW>)
                             : reinterpret_cast<const void *>(chunk_prepare_kernel<uint16_t, KDA_GATE_LOG>);
        int nr = nrec;
        void *params[] = {&kargs, &ws, &nr};
        if (hipLaunchKernel(fn, dim3(static_cast<unsigned>(nrec), static_cast<unsigned>(a.num_heads)),
                            dim3(kThreads), params, 0, st) != hipSuccess) {
            return KDA_ERR_LAUNCH;
        }
    }
    {
        const int64_t pairs = static_cast<int64_t>(a.num_seqs) * a.num_heads;
        const int64_t blocks = (pairs + 7) / 8 * 64;
        if (blocks > 0x7fffffff) {
            return KDA_ERR_INVALID_ARGUMENT;
        }
        const char *cws = ws;
        void *params[] = {&kargs, &cws};
        if (hipLaunchKernel(reinterpret_cast<const void *>(chunk_scan_kernel),
                            dim3(static_cast<unsigned>(blocks)), dim3(kThreads), params, 0,
                            st) != hipSuccess) {
            return KDA_ERR_LAUNCH;
        }
    }
    return KDA_OK;
}
