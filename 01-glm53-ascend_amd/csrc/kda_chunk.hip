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

// x[8] -> bf16 hi (+ lo) fragments; lo = bf16(x - hi), so x = hi + lo to
// about 2^-17 relative.
__device__ __forceinline__ bf16x8 to_bf16x8(const float x[8]) {
    u32x4 h;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        h[p] = pack_bf16x2(x[2 * p], x[2 * p + 1]);
    }
    return as_bf16x8(h);
}
__device__ __forceinline__ void split_bf16x8(const float x[8], bf16x8 &hi, bf16x8 &lo) {
    u32x4 h, l;
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        const uint32_t hp = pack_bf16x2(x[2 * p], x[2 * p + 1]);
        const float h0 = __uint_as_float(hp << 16);
        const float h1 = __uint_as_float(hp & 0xffff0000u);
        h[p] = hp;
        l[p] = pack_bf16x2(x[2 * p] - h0, x[2 * p + 1] - h1);
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

// Workgroup barrier for LDS hand-offs only: waits for this wave's LDS
// accesses, not for its outstanding global loads (a full __syncthreads() also
// drains vmcnt, which would stall the scan's prefetch of the next chunk).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
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
//
// 68 KiB of LDS, so two workgroups share a CU and one's loads overlap the
// other's math. k is kept as its bf16 input plus a per-row inverse norm, q
// never enters LDS (each wave loads its own rows into registers), and the
// solve's X and v^T reuse the cumsum tile once it is dead.
// ---------------------------------------------------------------------------

constexpr int kPadF = 132;  // fp32 row stride of [64][128] tiles (bank spread)
constexpr int kPadK = 136;  // bf16 row stride of the k tile
constexpr int kPadX = 68;   // fp32 row stride of [64][64] tiles (16-B rows)

// [128][64] bf16 tiles stored with 8-element groups XOR-swizzled by the row,
// so the 16 rows a wave reads at one column land in different banks.
__device__ __forceinline__ int swz(int row, int col) {
    return row * 64 + ((((col >> 3) ^ (row & 7)) << 3) | (col & 7));
}

struct PrepShared {
    union {
        float G[BT][kPadF];  // cumsum of the log decay (S1-S4)
        struct {
            float X[BT][kPadX];       // (I + L)^-1, then T = X diag(beta) (S5-S6)
            uint16_t Vt[DK * BT];     // v^T, bf16 bits, swizzled (S5-S6)
        } late;
    } r0;
    union {
        uint16_t K[BT][kPadK];   // k, bf16 input bits (S1-S4)
        uint16_t KE[DK * BT];    // (e^G k)^T as bf16, swizzled (S4-S6)
    } r1;
    float LT[BT][kPadX];  // L^T: LT[j][i] = beta_i Akk[i][j] (j < i)
    float beta[BT];
    float rnk[BT];        // k row scale (1 / norm, or 1)
    float carry[DK];
};
static_assert(sizeof(PrepShared) <= 80 * 1024, "two prepare workgroups per CU");

template <int GATE>
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
    const bool norm = GATE == KDA_GATE_RAW || a.qk_l2norm != 0;
    const uint16_t *qp = static_cast<const uint16_t *>(a.q);

    // Row blocks I this wave builds Akk/Aqk pairs for (balanced over waves):
    //   wave 0: (0,0) (1,0) (1,1)   wave 1: (2,0) (2,1) (2,2)
    //   wave 2: (3,0) (3,1)         wave 3: (3,2) (3,3)
    const int nI = wave == 0 ? 2 : 1;
    const int I0 = wave == 0 ? 0 : (wave == 1 ? 2 : 3);
    // Its q rows, loaded now so the loads overlap S1/S2: lane (r, gq) holds
    // q[16I + r][32s + kperm(gq, e)] as 4 x (4 bf16) per slice pair.
    uint2 qraw[2][4][2];
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int t = 16 * (I0 + ii) + r;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            qraw[ii][s][0] = make_uint2(0u, 0u);
            qraw[ii][s][1] = make_uint2(0u, 0u);
            if (ii < nI && t < len) {
                const uint16_t *row = qp + (static_cast<int64_t>(t0 + t) * H + h) * DK + 32 * s;
                qraw[ii][s][0] = *reinterpret_cast<const uint2 *>(row + 4 * gq);
                qraw[ii][s][1] = *reinterpret_cast<const uint2 *>(row + 16 + 4 * gq);
            }
        }
    }

    // ---- S1: k rows, log decay, beta (zero-padded); L^T cleared -------------
    {
        const int kc = tid & 31;
        const int rg = tid >> 5;
        const uint16_t *kp = static_cast<const uint16_t *>(a.k);
        float expA = 0.f;
        float4 dtb = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (GATE == KDA_GATE_RAW) {
            expA = expf(a.A_log[h]);
            dtb = load4(a.dt_bias + static_cast<int64_t>(h) * DK + 4 * kc);
        }
        uint2 kraw[8];
        float4 g4[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int t = rg + 8 * i;
            const int64_t base = (static_cast<int64_t>(t0 + t) * H + h) * DK + 4 * kc;
            kraw[i] = make_uint2(0u, 0u);
            g4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (t < len) {
                kraw[i] = *reinterpret_cast<const uint2 *>(kp + base);
                if constexpr (GATE == KDA_GATE_RAW) {
                    const float4 av = load4(static_cast<const uint16_t *>(a.gate) + base);
                    const float lb = a.lower_bound;
                    g4[i].x = lb / (1.0f + __expf(-(expA * (av.x + dtb.x))));
                    g4[i].y = lb / (1.0f + __expf(-(expA * (av.y + dtb.y))));
                    g4[i].z = lb / (1.0f + __expf(-(expA * (av.z + dtb.z))));
                    g4[i].w = lb / (1.0f + __expf(-(expA * (av.w + dtb.w))));
                } else {
                    g4[i] = load4(static_cast<const float *>(a.gate) + base);
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int t = rg + 8 * i;
            if (norm) {
                const float4 k4 = make_float4(__uint_as_float(kraw[i].x << 16),
                                              __uint_as_float(kraw[i].x & 0xffff0000u),
                                              __uint_as_float(kraw[i].y << 16),
                                              __uint_as_float(kraw[i].y & 0xffff0000u));
                const float ks = group_sum32(dot4(k4, k4));
                if (kc == 0) {
                    sm.rnk[t] = 1.0f / sqrtf(ks + 1e-6f);
                }
            } else if (kc == 0) {
                sm.rnk[t] = 1.0f;
            }
            *reinterpret_cast<uint2 *>(&sm.r1.K[t][4 * kc]) = kraw[i];
            *reinterpret_cast<float4 *>(&sm.r0.G[t][4 * kc]) = g4[i];
        }
        if (tid < BT) {
            float b = 0.f;
            if (tid < len) {
                const int64_t bi = static_cast<int64_t>(t0 + tid) * H + h;
                if constexpr (GATE == KDA_GATE_RAW) {
                    b = 1.0f / (1.0f + __expf(-bf16_to_f32(static_cast<const uint16_t *>(a.beta)[bi])));
                } else {
                    b = static_cast<const float *>(a.beta)[bi];
                }
            }
            sm.beta[tid] = b;
        }
        for (int idx = tid; idx < BT * BT; idx += kThreads) {
            sm.LT[idx >> 6][idx & 63] = 0.f;
        }
    }
    lds_barrier();

    // ---- S2: in-chunk cumsum of g, per channel ------------------------------
    {
        const int ch = tid & 127;
        const int half = tid >> 7;
        float vals[32];
        float run = 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            run += sm.r0.G[half * 32 + i][ch];
            vals[i] = run;
        }
        if (half == 0) {
            sm.carry[ch] = run;
        }
        lds_barrier();
        const float add = half ? sm.carry[ch] : 0.f;
#pragma unroll
        for (int i = 0; i < 32; ++i) {
            sm.r0.G[half * 32 + i][ch] = vals[i] + add;
        }
    }
    lds_barrier();

    auto kval = [&](int t, int k) {
        return bf16_to_f32(sm.r1.K[t][k]) * sm.rnk[t];
    };
    // 8 channels {32s + kperm(gq, e)} of one row: two 8-byte k reads, two
    // 16-byte G reads (vector LDS accesses instead of per-element ones).
    auto load_k8 = [&](int row, int s, float x[8]) {
        const uint2 k0 = *reinterpret_cast<const uint2 *>(&sm.r1.K[row][32 * s + 4 * gq]);
        const uint2 k1 = *reinterpret_cast<const uint2 *>(&sm.r1.K[row][32 * s + 16 + 4 * gq]);
        x[0] = __uint_as_float(k0.x << 16);
        x[1] = __uint_as_float(k0.x & 0xffff0000u);
        x[2] = __uint_as_float(k0.y << 16);
        x[3] = __uint_as_float(k0.y & 0xffff0000u);
        x[4] = __uint_as_float(k1.x << 16);
        x[5] = __uint_as_float(k1.x & 0xffff0000u);
        x[6] = __uint_as_float(k1.y << 16);
        x[7] = __uint_as_float(k1.y & 0xffff0000u);
    };
    auto load_g8 = [&](int row, int s, float x[8]) {
        const float4 g0 = *reinterpret_cast<const float4 *>(&sm.r0.G[row][32 * s + 4 * gq]);
        const float4 g1 = *reinterpret_cast<const float4 *>(&sm.r0.G[row][32 * s + 16 + 4 * gq]);
        x[0] = g0.x;
        x[1] = g0.y;
        x[2] = g0.z;
        x[3] = g0.w;
        x[4] = g1.x;
        x[5] = g1.y;
        x[6] = g1.z;
        x[7] = g1.w;
    };

    // ---- S3: Akk (-> L^T in LDS), Aqk and q e^G (-> fragments) --------------
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        if (ii >= nI) {
            break;
        }
        const int I = I0 + ii;
        const int ri = 16 * I + r;
        // q row: widen, norm over all 128 channels (4 lane groups), scale
        float qv[4][8];
        float qss = 0.f;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const uint2 q0 = qraw[ii][s][0];
            const uint2 q1 = qraw[ii][s][1];
            qv[s][0] = __uint_as_float(q0.x << 16);
            qv[s][1] = __uint_as_float(q0.x & 0xffff0000u);
            qv[s][2] = __uint_as_float(q0.y << 16);
            qv[s][3] = __uint_as_float(q0.y & 0xffff0000u);
            qv[s][4] = __uint_as_float(q1.x << 16);
            qv[s][5] = __uint_as_float(q1.x & 0xffff0000u);
            qv[s][6] = __uint_as_float(q1.y << 16);
            qv[s][7] = __uint_as_float(q1.y & 0xffff0000u);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                qss += qv[s][e] * qv[s][e];
            }
        }
        float qscale = a.scale;
        if (norm) {
            qss += __shfl_xor(qss, 16);
            qss += __shfl_xor(qss, 32);
            qscale = a.scale / sqrtf(qss + 1e-6f);
        }
        // the block's anchor row G[16I][.], kept for every column block
        float anc[4][8];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            load_g8(16 * I, s, anc[s]);
        }
        const float rki = sm.rnk[ri];
        bf16x8 Rh[4], Qh[4], Ql[4];
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            float kk[8], gg[8], rv[8], qa[8], qg[8];
            load_k8(ri, s, kk);
            load_g8(ri, s, gg);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float ex = __expf(gg[e] - anc[s][e]);
                const float qn = qv[s][e] * qscale;
                rv[e] = kk[e] * rki * ex;
                qa[e] = qn * ex;
                qg[e] = qn * __expf(gg[e]);
            }
            Rh[s] = to_bf16x8(rv);
            split_bf16x8(qa, Qh[s], Ql[s]);
            // q e^G fragment (mt = I, s); for I = 3 only wave 2 writes it
            if (!(I == 3 && wave == 3)) {
                bf16x8 fh, fl;
                split_bf16x8(qg, fh, fl);
                store_frag(rec, kOffQgH, I * 4 + s, lane, fh);
                store_frag(rec, kOffQgL, I * 4 + s, lane, fl);
            }
        }
        // this wave's column blocks J of row block I
        const int J0 = wave == 3 ? 2 : 0;
        const int J1 = wave == 2 ? 1 : I;
        float aq[4][4];
#pragma unroll
        for (int J = 0; J < 4; ++J) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                aq[J][e] = 0.f;
            }
        }
#pragma unroll
        for (int J = 0; J < 4; ++J) {
            if (J < J0 || J > J1) {
                continue;
            }
            const int rj = 16 * J + r;
            const float rkj = sm.rnk[rj];
            const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
            f32x4 akk2[2] = {z4, z4};
            f32x4 aq3[3] = {z4, z4, z4};
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                float kk[8], gg[8], cv[8];
                load_k8(rj, s, kk);
                load_g8(rj, s, gg);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    cv[e] = kk[e] * rkj * __expf(anc[s][e] - gg[e]);
                }
                bf16x8 Ch, Cl;
                split_bf16x8(cv, Ch, Cl);
                akk2[s & 1] = mfma(Rh[s], Ch, akk2[s & 1]);  // Akk[i][j], rows i of block I
                aq3[0] = mfma(Ch, Qh[s], aq3[0]);            // Aqk^T[j][i]
                aq3[1] = mfma(Ch, Ql[s], aq3[1]);
                aq3[2] = mfma(Cl, Qh[s], aq3[2]);
            }
            f32x4 akk, aqt;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                akk[e] = akk2[0][e] + akk2[1][e];
                aqt[e] = (aq3[0][e] + aq3[1][e]) + aq3[2][e];
            }
            float4 lt;
            float *ltp = &lt.x;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int i = 16 * I + 4 * gq + e;
                const int j = 16 * J + r;
                ltp[e] = j < i ? akk[e] * sm.beta[i] : 0.f;
                // aqt holds Aqk[16I + r][16J + 4gq + e]
                aq[J][e] = (16 * J + 4 * gq + e) <= ri ? aqt[e] : 0.f;
            }
            *reinterpret_cast<float4 *>(&sm.LT[16 * J + r][16 * I + 4 * gq]) = lt;
        }
        // Aqk fragments (mt = I, s): s covers column blocks 2s and 2s+1
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const bool mine = (2 * s >= J0 && 2 * s <= (J1 | 1)) || (I < 3 && s * 2 > I);
            if (!mine) {
                continue;
            }
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

    // ---- S4: kd^T fragments, e^(G_last), tracking operands, (e^G k)^T -------
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int mk = 2 * wave + tt;
        const int k = 16 * mk + r;
        const float gl = sm.r0.G[BT - 1][k];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            float x[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int t = 32 * s + kperm(gq, e);
                x[e] = kval(t, k) * __expf(gl - sm.r0.G[t][k]);
            }
            bf16x8 fh, fl;
            split_bf16x8(x, fh, fl);
            store_frag(rec, kOffKdH, mk * 2 + s, lane, fh);
            store_frag(rec, kOffKdL, mk * 2 + s, lane, fl);
        }
    }
    if (tid < DK) {
        reinterpret_cast<float *>(rec + kOffGl)[tid] = __expf(sm.r0.G[BT - 1][tid]);
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
                const float gr = sm.r0.G[rr - 1][k];
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    float x[8];
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int t = 32 * s + kperm(gq, e);
                        x[e] = t < rr ? kval(t, k) * __expf(gr - sm.r0.G[t][k]) : 0.f;
                    }
                    bf16x8 fh, fl;
                    split_bf16x8(x, fh, fl);
                    store_frag(tr, kTrOffKdH, mk * 2 + s, lane, fh);
                    store_frag(tr, kTrOffKdL, mk * 2 + s, lane, fl);
                }
            }
            if (tid < DK) {
                reinterpret_cast<float *>(tr + kTrOffGl)[tid] = __expf(sm.r0.G[rr - 1][tid]);
            }
        }
    }
    uint32_t kep[16];
    {
        const int k = tid & 127;
        const int half = tid >> 7;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            const int t = half * 32 + 2 * i;
            const uint16_t e0 = f32_to_bf16(kval(t, k) * __expf(sm.r0.G[t][k]));
            const uint16_t e1 = f32_to_bf16(kval(t + 1, k) * __expf(sm.r0.G[t + 1][k]));
            kep[i] = pack2(e0, e1);
        }
    }
    lds_barrier();  // G and K are dead from here on
    {
        const int k = tid & 127;
        const int half = tid >> 7;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            *reinterpret_cast<uint32_t *>(&sm.r1.KE[swz(k, half * 32 + 2 * i)]) = kep[i];
        }
        // v^T (bf16, swizzled), rows zero-padded
        const int kc = tid & 31;
        const int rg = tid >> 5;
        const uint16_t *vp = static_cast<const uint16_t *>(a.v);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int t = rg + 8 * i;
            uint2 vr = make_uint2(0u, 0u);
            if (t < len) {
                vr = *reinterpret_cast<const uint2 *>(vp + (static_cast<int64_t>(t0 + t) * H + h) * DK + 4 * kc);
            }
            sm.r0.late.Vt[swz(4 * kc + 0, t)] = static_cast<uint16_t>(vr.x & 0xffffu);
            sm.r0.late.Vt[swz(4 * kc + 1, t)] = static_cast<uint16_t>(vr.x >> 16);
            sm.r0.late.Vt[swz(4 * kc + 2, t)] = static_cast<uint16_t>(vr.y & 0xffffu);
            sm.r0.late.Vt[swz(4 * kc + 3, t)] = static_cast<uint16_t>(vr.y >> 16);
        }
        // X: upper blocks zero
        for (int idx = tid; idx < BT * BT; idx += kThreads) {
            const int i = idx >> 6;
            const int j = idx & 63;
            if ((j >> 4) > (i >> 4)) {
                sm.r0.late.X[i][j] = 0.f;
            }
        }
    }

    // ---- S5: X = (I + L)^-1 (blocked, fp32), then T = X diag(beta) ----------
    // Diagonal 16x16 blocks, right-looking: column c of block w per lane c.
    if (lane < 16) {
        const int b0 = 16 * wave;
        const int col = lane;
        // Constant loop bounds with a compile-time i > j mask: every acc[]
        // index is static, so the array stays in registers (a bound that
        // depends on j leaves the inner loop rolled and turns acc[] into a
        // runtime-indexed select chain).
        float acc[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            acc[i] = i == col ? 1.f : 0.f;
        }
#pragma unroll
        for (int j = 0; j < 15; ++j) {
            const float xj = acc[j];
            float lrow[16];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const float4 t4 = *reinterpret_cast<const float4 *>(&sm.LT[b0 + j][b0 + 4 * q]);
                lrow[4 * q + 0] = t4.x;
                lrow[4 * q + 1] = t4.y;
                lrow[4 * q + 2] = t4.z;
                lrow[4 * q + 3] = t4.w;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (i > j) {
                    acc[i] -= lrow[i] * xj;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
            sm.r0.late.X[b0 + i][b0 + col] = acc[i];
        }
    }
    lds_barrier();
    // Off-diagonal blocks by level d = I - J:
    //   M_IJ = sum_{K=J}^{I-1} L_IK X_KJ,  X_IJ = -X_II M_IJ;
    // M_IJ is parked (transposed) in the still-zero upper block (J, I).
    for (int d = 1; d < 4; ++d) {
        const int nb = 4 - d;
        for (int idx = tid; idx < nb * 256; idx += kThreads) {
            const int J = idx >> 8;
            const int I = J + d;
            const int i = (idx >> 4) & 15;
            const int jj = idx & 15;
            float acc = 0.f;
#pragma unroll 16
            for (int kk = 16 * J; kk < 16 * I; ++kk) {
                acc += sm.LT[kk][16 * I + i] * sm.r0.late.X[kk][16 * J + jj];
            }
            sm.r0.late.X[16 * J + jj][16 * I + i] = acc;
        }
        lds_barrier();
        for (int idx = tid; idx < nb * 256; idx += kThreads) {
            const int J = idx >> 8;
            const int I = J + d;
            const int i = (idx >> 4) & 15;
            const int jj = idx & 15;
            float acc = 0.f;
#pragma unroll
            for (int kk = 0; kk < 16; ++kk) {
                acc += sm.r0.late.X[16 * I + i][16 * I + kk] * sm.r0.late.X[16 * J + jj][16 * I + kk];
            }
            sm.r0.late.X[16 * I + i][16 * J + jj] = -acc;
        }
        lds_barrier();
        for (int idx = tid; idx < nb * 256; idx += kThreads) {
            const int J = idx >> 8;
            const int I = J + d;
            const int i = (idx >> 4) & 15;
            const int jj = idx & 15;
            sm.r0.late.X[16 * J + jj][16 * I + i] = 0.f;
        }
        lds_barrier();
    }
    for (int idx = tid; idx < BT * BT; idx += kThreads) {
        const int i = idx >> 6;
        const int j = idx & 63;
        sm.r0.late.X[i][j] *= sm.beta[j];
    }
    lds_barrier();

    // ---- S6: u = T v (T split) and w^T = (e^G k)^T T^T (single) --------------
    {
        const int t = 16 * wave + r;
        const int nS = wave >= 2 ? 2 : 1;  // T is lower triangular
        bf16x8 Th[2], Tl[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float4 x0 = *reinterpret_cast<const float4 *>(&sm.r0.late.X[t][32 * s + 4 * gq]);
            const float4 x1 = *reinterpret_cast<const float4 *>(&sm.r0.late.X[t][32 * s + 16 + 4 * gq]);
            const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
            split_bf16x8(x, Th[s], Tl[s]);
        }
        // u tiles (mt = wave, vt): A = T rows, B = v (K = j)
#pragma unroll
        for (int vt = 0; vt < 8; ++vt) {
            const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
            f32x4 acc[2] = {z4, z4};
#pragma unroll
            for (int s = 0; s < 2; ++s) {
                if (s >= nS) {
                    break;  // uniform per wave; keeps s (and Th[s]) static
                }
                const int row = 16 * vt + r;
                const uint2 v0 = *reinterpret_cast<const uint2 *>(&sm.r0.late.Vt[swz(row, 32 * s + 4 * gq)]);
                const uint2 v1 = *reinterpret_cast<const uint2 *>(&sm.r0.late.Vt[swz(row, 32 * s + 16 + 4 * gq)]);
                const bf16x8 vb = as_bf16x8(u32x4{v0.x, v0.y, v1.x, v1.y});
                acc[0] = mfma(Th[s], vb, acc[0]);
                acc[1] = mfma(Tl[s], vb, acc[1]);
            }
            f32x4 uo;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                uo[i] = acc[0][i] + acc[1][i];
            }
            reinterpret_cast<f32x4 *>(rec + kOffU)[(wave * 8 + vt) * 64 + lane] = uo;
        }
        // w^T tiles (mk, nt = wave): A = (e^G k)^T rows k, B = T^T (K = j)
        for (int sp = 0; sp < 4; ++sp) {
            float x[8];
#pragma unroll
            for (int half = 0; half < 2; ++half) {
                const int mk = 2 * sp + half;
                f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    if (s >= nS) {
                        break;
                    }
                    const int row = 16 * mk + r;
                    const uint2 k0 = *reinterpret_cast<const uint2 *>(&sm.r1.KE[swz(row, 32 * s + 4 * gq)]);
                    const uint2 k1 = *reinterpret_cast<const uint2 *>(&sm.r1.KE[swz(row, 32 * s + 16 + 4 * gq)]);
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
    __shared__ uint32_t otile[4][16][8];     // per wave: its 16 output rows x 16 bf16 columns

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

    // One chunk's operands, held in registers. Two sets alternate so the
    // next chunk's fragments are in flight while this chunk computes.
    struct Ops {
        bf16x8 Wf[4], Qh[4], Ql[4], Ah[2], Al[2], Kh[2][2], Kl[2][2];
        f32x4 u, gl[2];
    };
    auto load_ops = [&](Ops &op, int j) {
        const char *rec = ws + LY.recs + (static_cast<size_t>(c0 + j) * H + h) * kRecBytes;
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            op.Wf[s] = load_frag(rec, kOffW, w * 4 + s, lane);
            op.Qh[s] = load_frag(rec, kOffQgH, w * 4 + s, lane);
            op.Ql[s] = load_frag(rec, kOffQgL, w * 4 + s, lane);
        }
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            op.Ah[s] = load_frag(rec, kOffAqH, w * 2 + s, lane);
            op.Al[s] = load_frag(rec, kOffAqL, w * 2 + s, lane);
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                op.Kh[tt][s] = load_frag(rec, kOffKdH, (2 * w + tt) * 2 + s, lane);
                op.Kl[tt][s] = load_frag(rec, kOffKdL, (2 * w + tt) * 2 + s, lane);
            }
        }
        op.u = reinterpret_cast<const f32x4 *>(rec + kOffU)[(w * 8 + vt) * 64 + lane];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            op.gl[tt] = *reinterpret_cast<const f32x4 *>(rec + kOffGl + 4 * (16 * (2 * w + tt) + 4 * gq));
        }
    };

    auto step = [&](const Ops &op, int j) {
        const int t0 = bos + BT * j;
        const int len = eos - t0 < BT ? eos - t0 : BT;

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
        lds_barrier();

        // 2. vnew rows [16w, 16w+16) = u - w S ; 3. o = (q e^G) S (3-pass).
        // Independent accumulators (per pass, per slice parity) keep several
        // MFMA chains in flight: with one wave per SIMD a single dependent
        // chain would pay the full MFMA latency on every link.
        const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
        f32x4 wsa[2] = {z4, z4};
        f32x4 oq[3] = {z4, z4, z4};
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const bf16x8 sh = as_bf16x8(sfrag[s][0][lane]);
            const bf16x8 sl = as_bf16x8(sfrag[s][1][lane]);
            wsa[s & 1] = mfma(op.Wf[s], sh, wsa[s & 1]);
            oq[0] = mfma(op.Qh[s], sh, oq[0]);
            oq[1] = mfma(op.Qh[s], sl, oq[1]);
            oq[2] = mfma(op.Ql[s], sh, oq[2]);
        }
        f32x4 vn;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            vn[i] = op.u[i] - (wsa[0][i] + wsa[1][i]);
        }
        // 4. publish vnew (tile mt = w is half w%2 of slice w/2)
        {
            uint32_t hp[2], lp[2];
#pragma unroll
            for (int p = 0; p < 2; ++p) {
                hp[p] = pack_bf16x2(vn[2 * p], vn[2 * p + 1]);
                lp[p] = pack_bf16x2(vn[2 * p] - __uint_as_float(hp[p] << 16),
                                    vn[2 * p + 1] - __uint_as_float(hp[p] & 0xffff0000u));
            }
            const int sl = w >> 1;
            const int hf = (w & 1) * 2;
            vfrag[sl][0][lane][hf] = hp[0];
            vfrag[sl][0][lane][hf + 1] = hp[1];
            vfrag[sl][1][lane][hf] = lp[0];
            vfrag[sl][1][lane][hf + 1] = lp[1];
        }
        lds_barrier();

        bf16x8 vh[2], vl[2];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            vh[s] = as_bf16x8(u32x4{vfrag[s][0][lane][0], vfrag[s][0][lane][1], vfrag[s][0][lane][2],
                                    vfrag[s][0][lane][3]});
            vl[s] = as_bf16x8(u32x4{vfrag[s][1][lane][0], vfrag[s][1][lane][1], vfrag[s][1][lane][2],
                                    vfrag[s][1][lane][3]});
        }
        // 5. o += Aqk vnew (3-pass) and store rows t < len
        f32x4 oa[3] = {z4, z4, z4};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            oa[0] = mfma(op.Ah[s], vh[s], oa[0]);
            oa[1] = mfma(op.Ah[s], vl[s], oa[1]);
            oa[2] = mfma(op.Al[s], vh[s], oa[2]);
        }
        f32x4 o;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            o[i] = ((oq[0][i] + oq[1][i]) + oq[2][i]) + ((oa[0][i] + oa[1][i]) + oa[2][i]);
        }
        // Output rows [16w, 16w+16) x 16 columns: transposed through this
        // wave's own LDS tile so each lane stores 4 consecutive columns of one
        // row (one 8-byte nontemporal store per lane instead of four 2-byte
        // stores; no workgroup barrier -- the tile is private to the wave).
        {
            uint16_t *ot = reinterpret_cast<uint16_t *>(&otile[w][0][0]);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ot[(4 * gq + i) * 16 + r] = f32_to_bf16(o[i]);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            const int row = lane >> 2;
            const int cq = lane & 3;
            typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
            const u32x2 val = *reinterpret_cast<const u32x2 *>(&otile[w][row][2 * cq]);
            const int t = 16 * w + row;
            if (t < len) {
                __builtin_nontemporal_store(
                    val, reinterpret_cast<u32x2 *>(out + (static_cast<int64_t>(t0 + t) * H + h) * DK +
                                                   16 * vt + 4 * cq));
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
                f32x4 tu[3] = {z4, z4, z4};
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    const bf16x8 th = load_frag(tr, kTrOffKdH, (2 * w + tt) * 2 + s, lane);
                    const bf16x8 tl = load_frag(tr, kTrOffKdL, (2 * w + tt) * 2 + s, lane);
                    tu[0] = mfma(th, vh[s], tu[0]);
                    tu[1] = mfma(th, vl[s], tu[1]);
                    tu[2] = mfma(tl, vh[s], tu[2]);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    St[tt][i] += (tu[0][i] + tu[1][i]) + tu[2][i];
                }
            }
            store_S(track_slot, St);
        }
        // 6. S <- e^(G_last) S + kd^T vnew (3-pass, independent chains)
        f32x4 su[2][3] = {{z4, z4, z4}, {z4, z4, z4}};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                su[tt][0] = mfma(op.Kh[tt][s], vh[s], su[tt][0]);
                su[tt][1] = mfma(op.Kh[tt][s], vl[s], su[tt][1]);
                su[tt][2] = mfma(op.Kl[tt][s], vh[s], su[tt][2]);
            }
        }
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                S[tt][i] = S[tt][i] * op.gl[tt][i] + ((su[tt][0][i] + su[tt][1][i]) + su[tt][2][i]);
            }
        }
        if (track_slot > 0 && rr == len) {
            store_S(track_slot, S);
        }
    };

    // The prefetches are unconditional (clamped to the last chunk) so the
    // compiler's wait counts stay exact on every path through the loop.
    Ops opA, opB;
    if (nch > 0) {
        load_ops(opA, 0);
    }
    for (int j = 0; j < nch; j += 2) {
        load_ops(opB, j + 1 < nch ? j + 1 : nch - 1);
        step(opA, j);
        if (j + 1 >= nch) {
            break;
        }
        load_ops(opA, j + 2 < nch ? j + 2 : nch - 1);
        step(opB, j + 1);
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
                             ? reinterpret_cast<const void *>(chunk_prepare_kernel<KDA_GATE_RAW>)
                             : reinterpret_cast<const void *>(chunk_prepare_kernel<KDA_GATE_LOG>);
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
