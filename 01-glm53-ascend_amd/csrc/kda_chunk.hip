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
// Since vnew = T (v - (e^G k) S), this file computes, with y = v - (e^G k) S,
//     o = (q e^G) S + (Aqk T) y,   S <- e^(G_last) * S + (T^T kd)^T y
// (kd = e^(G_last - G) * k): u, w and vnew are never formed.
//
// MI355X structure (three launches, one stream, no host synchronization):
//   K0 chunk_index_kernel   prefix sums of ceil(len/64) per sequence, so the
//                           chunk grid is sized on the host from T and N alone;
//   K1 chunk_prepare_kernel one workgroup per (chunk, head), all chunks in
//                           parallel: cumsum, Akk / Aqk on MFMA with exponents
//                           anchored at each 16-row block's midpoint row (no
//                           factor spans more than 8 tokens of decay, all
//                           column factors of earlier blocks e^(<=0)), the
//                           blocked triangular inverse in
//                           fp32, T^T kd and Aqk T on MFMA; writes the scan's
//                           operands as ready MFMA fragments;
//   K2 chunk_scan_kernel    one workgroup per (sequence, head, 16 or 32 value
//                           columns), the serial chunk recurrence: four chain
//                           waves carry S (fp32, registers) and y, four
//                           output waves compute o one phase behind, four
//                           loader waves stage the chain's operands and v in
//                           LDS; S and y are exchanged through LDS.
// A single long sequence on few heads, whose one scan would leave most CUs
// idle, takes the affine form instead (chunk_affine_combine_kernel): K1 for
// every chunk, then segment 0 scanned as usual while every later segment is
// scanned from zero and from the identity at once, then a serial combine of
// the segments' transitions and a parallel correction of their outputs.
//
// MFMA: v_mfma_f32_16x16x32_bf16 / _f16 with fp32 accumulation. Inside K1,
// operands whose rounding would break the tolerance contract are carried as
// bf16 hi + lo pairs (x = hi + lo to ~2^-17) and multiplied in three passes
// (hi hi, hi lo, lo hi): Akk and Aqk; T^T kd and Aqk T take T, kd and Aqk
// as fp16 hi + lo pairs (~2^-22) in three passes.
// The record the scan reads holds every matrix operand as fp16 (11-bit
// significands) with a power-of-two scale per fragment or row tile: e^G k,
// q e^G, (T^T kd)^T and Aqk T. The scan meets them with S_j as fp16 (scaled
// per 32-row slice; S itself stays fp32) for (e^G k) S and (q e^G) S, and
// with y as fp16 hi + lo (~2^-22) for (T^T kd)^T y and (Aqk T) y.
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

#include <atomic>
#include <mutex>

#include "kda_abi.h"
#include "kda_device.h"

namespace kda {
namespace chunk {

constexpr int BT = 64;   // tokens per chunk
constexpr int DK = 128;  // K == V
constexpr int kThreads = 256;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

// Workspace record of one (chunk, head), in 16-byte-per-lane fragments
// (a fragment is 64 lanes x 16 B = 1 KiB). With T = (I + diag(beta) Akk)^-1
// diag(beta) the chunk's UT transform, the scan forms y = v - (e^G k) S
// from the input v and never vnew = T y itself: the record holds the
// operands of y, of the state update (T^T kd)^T y and of the output
// (q e^G) S + (Aqk T) y. Every matrix operand is fp16 with a power-of-two
// scale (held in the scale block); the first 38 fragments are the chain's
// operands that every column group of a (sequence, head) reads whole, in
// the order the scan stages them.
constexpr int kFrag = 1024;
constexpr int kOffKe = 0;                         // e^G k fp16: A (mt 0..3, s 0..3)
constexpr int kOffKd = kOffKe + 16 * kFrag;       // (T^T kd)^T fp16: A (mk 0..7, s 0..1)
constexpr int kOffAq = kOffKd + 16 * kFrag;       // Aqk T fp16: A (mt, s), see aq_frag
constexpr int kOffQg = kOffAq + 6 * kFrag;        // q e^G fp16: A (mt, s)
constexpr int kOffGl = kOffQg + 16 * kFrag;       // e^(G_last) fp32 [128]
constexpr int kOffSc = kOffGl + DK * 4;           // fp32 scale block [128], indices below
constexpr int kRecBytes = kOffSc + 512;           // 56320
// Scale block: 2^-shift of each fp16 fragment group, and the bound the scan
// derives y's scale from (|y| <= max|v| + kel1 max|S|).
constexpr int kScKe = 0;     // [16] e^G k fragment (mt, s): mt * 4 + s (equal within s = 0, 1 and s = 2, 3)
constexpr int kScQg = 16;    // [16] q e^G fragment (mt, s) (equal within s = 0, 1 and s = 2, 3)
constexpr int kScKd = 32;    // [8]  (T^T kd)^T row tile mk (both token slices)
constexpr int kScAq = 40;    // [4]  Aqk T row tile mt (both token slices)
constexpr int kScKel1 = 48;  // [8]  4 h + mt: max over the rows t of tile mt of the sum of
                             //      |(e^G k)[t][k]| over channel half h (k in [64h, 64h + 64))
// Largest of four nonnegative values (magnitudes), compared as their bit
// patterns: no quieting of the operands as fmaxf needs for values it did not
// produce itself.
__device__ __forceinline__ float max4_mag(float a, float b, float c, float d) {
    return __uint_as_float(max(max(__float_as_uint(a), __float_as_uint(b)),
                               max(__float_as_uint(c), __float_as_uint(d))));
}
__device__ __forceinline__ float max4_mag(float4 v) { return max4_mag(v.x, v.y, v.z, v.w); }

// max over a chunk's rows t of sum_k |(e^G k)[t][k]|, bounded from above by
// the two channel halves' maxima of each row tile
__device__ __forceinline__ float kel1_bound(const float *sc) {
    const float4 h0 = *reinterpret_cast<const float4 *>(sc + kScKel1);
    const float4 h1 = *reinterpret_cast<const float4 *>(sc + kScKel1 + 4);
    return max4_mag(h0.x + h1.x, h0.y + h1.y, h0.z + h1.z, h0.w + h1.w);
}

// Track record of one (sequence, head): operands of the state after r < len
// tokens of the chunk holding the tracked position.
constexpr int kTrOffKd = 0;                       // (T^T kd_r)^T fp16, scaled per row tile mk
constexpr int kTrOffGl = kTrOffKd + 16 * kFrag;
constexpr int kTrOffSc = kTrOffGl + DK * 4;       // fp32 [8]
constexpr int kTrBytes = kTrOffSc + 256;          // 17152
static_assert(kRecBytes % 256 == 0 && kTrBytes % 256 == 0, "records stay 256-B aligned");

struct Layout {
    size_t chunk_start;  // int32 [N+1]
    size_t sched;        // several sequences: int4 [2N+1], see chunk_index_kernel
    size_t recs;         // kRecBytes x (ring x H): chunk c's record in ring slot c % ring
    size_t tracks;       // kTrBytes x (N x H)
    size_t carry;        // one sequence: fp32 [H][V][K], the state between scan segments
    size_t total;
};

__host__ __device__ inline size_t align256(size_t x) { return (x + 255) & ~size_t(255); }

__host__ __device__ inline int max_chunks(int T, int N) { return (T + BT - 1) / BT + N; }

// Aqk is lower triangular: its fragments (mt, s = 1) for mt < 2 (rows < 32,
// columns >= 32) are zero and not stored, leaving six per record.
__host__ __device__ constexpr int aq_frag(int mt, int s) { return mt < 2 ? mt : 2 * mt - 2 + s; }

// ring: record slots per head; every chunk has its own slot when ring >=
// max_chunks (the one-pass layout), a window ring of 2W slots otherwise.
__host__ __device__ inline Layout layout(int T, int N, int H, int ring) {
    Layout L;
    L.chunk_start = 0;
    L.sched = align256(static_cast<size_t>(N + 1) * 4);
    L.recs = N > 1 ? L.sched + align256(static_cast<size_t>(2 * N + 1) * 16) : L.sched;
    L.tracks = L.recs + static_cast<size_t>(kRecBytes) * ring * H;
    L.carry = L.tracks + static_cast<size_t>(kTrBytes) * N * H;
    L.total = L.carry + (N == 1 ? static_cast<size_t>(DK) * DK * 4 * H : 0);
    return L;
}
__host__ __device__ inline Layout layout(int T, int N, int H) { return layout(T, N, H, max_chunks(T, N)); }

// The affine form of one sequence (P segments; see chunk_affine_combine_kernel)
// keeps every chunk's record (the one-pass layout) and adds: the fp32
// outputs of the later segments' zero-start and identity-start scans
// ([T][H][V] each, indexed by token), the two scans' final states per later
// segment and the true state at each later segment's start ([P-1][H][V][K]
// each, K contiguous), and the two scans' tracked states ([H][V][K] each).
struct AffLayout {
    size_t out_zero, out_phi, fin_zero, fin_phi, start, trk_zero, trk_phi, total;
};
__host__ __device__ inline AffLayout aff_layout(int T, int H, int P) {
    const size_t st = static_cast<size_t>(H) * DK * DK * 4;
    const size_t ob = align256(static_cast<size_t>(T) * H * DK * 4);
    AffLayout A;
    A.out_zero = layout(T, 1, H).total;
    A.out_phi = A.out_zero + ob;
    A.fin_zero = A.out_phi + ob;
    A.fin_phi = A.fin_zero + st * (P - 1);
    A.start = A.fin_phi + st * (P - 1);
    A.trk_zero = A.start + st * (P - 1);
    A.trk_phi = A.trk_zero + st;
    A.total = A.trk_phi + st;
    return A;
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

// fp16 fragments carry x * 2^sh, with sh chosen per fragment (or per S
// slice) from its largest magnitude m so that m * 2^sh lies in [2^13, 2^14):
// well inside fp16's range, full 11-bit significands down to 2^-27 m.
__device__ __forceinline__ int f16_shift(float m) {
    if (!(m > 0.f)) {
        return 0;
    }
    int e;
    (void)frexpf(m, &e);  // m = f 2^e, f in [0.5, 1)
    const int sh = 14 - e;
    return sh < -120 ? -120 : (sh > 120 ? 120 : sh);
}
__device__ __forceinline__ f16x8 to_f16x8(const float x[8], int sh) {
    f16x8 h;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        h[e] = static_cast<_Float16>(ldexpf(x[e], sh));
    }
    return h;
}
// (x0, x1) * 2^sh = hi + lo to about 2^-22 relative, as packed fp16 pairs
// (round to nearest even; bits of x0 in the low half): one packed conversion
// for the high parts, the exact residuals xs - hi with hi read as fp16 from
// its half of the packed pair (v_fma_mix_f32), one packed conversion for the
// low parts.
__device__ __forceinline__ void split_f16x2(float x0, float x1, int sh, uint32_t &hi, uint32_t &lo) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    const f32x2_t xs = {ldexpf(x0, sh), ldexpf(x1, sh)};
    const f16x2_t h = __builtin_convertvector(xs, f16x2_t);
    const uint32_t hp = __builtin_bit_cast(uint32_t, h);
    float d0, d1;
    asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,0] op_sel_hi:[0,0,1]" : "=v"(d0) : "v"(xs[0]), "v"(hp));
    asm("v_fma_mix_f32 %0, %1, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[0,0,1]" : "=v"(d1) : "v"(xs[1]), "v"(hp));
    const f32x2_t ds = {d0, d1};
    hi = hp;
    lo = __builtin_bit_cast(uint32_t, __builtin_convertvector(ds, f16x2_t));
}
// the same for eight values
__device__ __forceinline__ void split_f16x8(const float x[8], int sh, f16x8 &hi, f16x8 &lo) {
    uint32_t h[4], l[4];
#pragma unroll
    for (int p = 0; p < 4; ++p) {
        split_f16x2(x[2 * p], x[2 * p + 1], sh, h[p], l[p]);
    }
    hi = __builtin_bit_cast(f16x8, u32x4{h[0], h[1], h[2], h[3]});
    lo = __builtin_bit_cast(f16x8, u32x4{l[0], l[1], l[2], l[3]});
}
__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(f16x8 v) { return __builtin_bit_cast(u32x4, v); }

__device__ __forceinline__ f32x4 mfma(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Largest value over the wave for nonnegative x (magnitudes and sums of
// magnitudes): their bit patterns order as the values do, so the reduction runs
// on them as unsigned integers (zero, what a lane without a source would
// read, is the identity), each DPP step one fused max and the cross-row tail
// on scalars.
__device__ __forceinline__ float wave_max_mag(float x) {
    uint32_t u = __float_as_uint(x);
    u = max(u, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(u), kDppQuadXor1, 0xf, 0xf, true)));
    u = max(u, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(u), kDppQuadXor2, 0xf, 0xf, true)));
    u = max(u, static_cast<uint32_t>(
                   __builtin_amdgcn_mov_dpp(static_cast<int>(u), kDppRowHalfMirror, 0xf, 0xf, true)));
    u = max(u, static_cast<uint32_t>(__builtin_amdgcn_mov_dpp(static_cast<int>(u), kDppRowMirror, 0xf, 0xf, true)));
    const uint32_t a = max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 0)),
                           static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 16)));
    const uint32_t b = max(static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 32)),
                           static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(u), 48)));
    return __uint_as_float(max(a, b));
}

// One wave stores NF consecutive fp16 fragments with one shared scale, and
// writes the inverse scale to sc[0 .. nsc).
template <int NF>
__device__ __forceinline__ void store_frags_f16(char *base, int off, int idx, float *sc, int lane,
                                                const float (&x)[NF][8], int nsc = 1) {
    float m = 0.f;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            m = fmaxf(m, fabsf(x[f][e]));
        }
    }
    const int sh = f16_shift(wave_max_mag(m));
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        reinterpret_cast<u32x4 *>(base + off)[(idx + f) * 64 + lane] = as_u32x4(to_f16x8(x[f], sh));
    }
    if (lane < nsc) {
        sc[lane] = ldexpf(1.f, -sh);
    }
}

// store_frags_f16 for values given as x * 2^ex[t], with t = 2f + (e >= 4) the
// 16-row tile of element e of fragment f: the exponents join the fragment's
// own shift (one ldexp per value; power-of-two factors change no bits).
template <int NF>
__device__ __forceinline__ void store_frags_f16_exp(char *base, int off, int idx, float *sc, int lane,
                                                    const float (&x)[NF][8], const int (&ex)[2 * NF]) {
    float m = 0.f;
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        float m0 = 0.f, m1 = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            m0 = fmaxf(m0, fabsf(x[f][e]));
            m1 = fmaxf(m1, fabsf(x[f][4 + e]));
        }
        m = fmaxf(m, fmaxf(ldexpf(m0, ex[2 * f]), ldexpf(m1, ex[2 * f + 1])));
    }
    const int sh = f16_shift(wave_max_mag(m));
#pragma unroll
    for (int f = 0; f < NF; ++f) {
        f16x8 h;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            h[e] = static_cast<_Float16>(ldexpf(x[f][e], sh + ex[2 * f + (e >> 2)]));
        }
        reinterpret_cast<u32x4 *>(base + off)[(idx + f) * 64 + lane] = as_u32x4(h);
    }
    if (lane == 0) {
        sc[0] = ldexpf(1.f, -sh);
    }
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
// K0 (several sequences): chunk_start[n] = sum_{m<n} ceil(len_m / 64),
// chunk_start[N] = total; with `sort` (the persistent scan runs next), also
// the sequences ordered by chunk count, longest first (ties by index): for
// rank r < N, sched[2r] = (n, chunk_start[n], bos_n, eos_n) and sched[2r+1]
// = (pool slot, tracked slot, tracked length, 0) with the slots' range rules
// applied (0: none; length -1: no tracking), and sched[2N].x = the number of
// nonempty sequences (a prefix of that order).
// ---------------------------------------------------------------------------

// Sequences the schedule sorts (in LDS) at most, and items per persistent
// team at most; beyond either the scan runs a workgroup per item.
constexpr int kPersMaxSeqs = 4096;
constexpr int kPersMaxItems = 256;

__global__ __launch_bounds__(1024) void chunk_index_kernel(const KdaChunkArgs a, int *cs, int4 *sched, int sort) {
    // With the schedule, every per-sequence value is loaded once, up front,
    // into LDS, so the sort and the table wait on no global round trip.
    __shared__ int part[16];                            // each wave's chunk total
    __shared__ unsigned long long key[kPersMaxSeqs];    // (chunks + 1, ~n)
    __shared__ int4 info[kPersMaxSeqs];                 // (bos, eos, chunk start, pool slot)
    __shared__ int2 tinfo[kPersMaxSeqs];                // (tracked slot, tracked length)
    const int N = a.num_seqs;
    const bool dosort = sort != 0 && N <= kPersMaxSeqs;
    const bool track = a.track_indices != nullptr;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int per = (N + 1023) / 1024;
    const int begin = tid * per;
    const int end = begin + per < N ? begin + per : N;
    int sum = 0;
    for (int n = begin; n < end; ++n) {
        int bos, eos;
        seq_bounds(a, n, bos, eos);
        const int c = (eos - bos + BT - 1) / BT;
        sum += c;
        if (dosort) {
            int slot = a.state_indices[n];
            if (slot < 0 || static_cast<int64_t>(slot) >= a.num_slots) {
                slot = 0;
            }
            int tslot = 0;
            int tlen = -1;
            if (track) {
                tslot = a.track_indices[n];
                const int tl = a.track_lens[n];
                if (tslot <= 0 || static_cast<int64_t>(tslot) >= a.num_slots) {
                    tslot = 0;
                } else {
                    tlen = tl;
                }
            }
            info[n] = make_int4(bos, eos, 0, slot);
            tinfo[n] = make_int2(tslot, tlen);
            key[n] = (static_cast<unsigned long long>(c + 1) << 32) | (0xffffffffu - static_cast<unsigned>(n));
        }
    }
    // exclusive prefix of the per-thread sums: within the wave by lane
    // shuffles, across the 16 waves through LDS
    int inc = sum;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int o = __shfl_up(inc, off);
        inc += lane >= off ? o : 0;
    }
    if (lane == 63) {
        part[wave] = inc;
    }
    __syncthreads();
    int run = inc - sum;
    int total = 0;
#pragma unroll
    for (int w = 0; w < 16; ++w) {
        const int p = part[w];
        run += w < wave ? p : 0;
        total += p;
    }
    for (int n = begin; n < end; ++n) {
        cs[n] = run;
        int bos, eos;
        if (dosort) {
            const int4 in = info[n];
            info[n].z = run;
            bos = in.x;
            eos = in.y;
        } else {
            seq_bounds(a, n, bos, eos);
        }
        run += (eos - bos + BT - 1) / BT;
    }
    if (tid == 1023) {
        cs[N] = total;
    }
    if (!dosort) {
        return;
    }
    // Sort descending by (chunks + 1, ~n): padding (zero) sorts after every
    // sequence, empty ones included. Up to 64 sequences: one wave, bitonic
    // through lane exchanges; beyond, bitonic in LDS.
    int npad = 1;
    while (npad < N) {
        npad <<= 1;
    }
    if (npad <= 64) {
        __syncthreads();  // info, tinfo and key complete
        if (wave != 0) {
            return;
        }
        unsigned long long x = lane < N ? key[lane] : 0ull;
#pragma unroll
        for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
            for (int stride = size >> 1; stride > 0; stride >>= 1) {
                const unsigned lo = __shfl_xor(static_cast<unsigned>(x), stride);
                const unsigned hi = __shfl_xor(static_cast<unsigned>(x >> 32), stride);
                const unsigned long long y = (static_cast<unsigned long long>(hi) << 32) | lo;
                const bool lower = (lane & stride) == 0;
                const bool desc = (lane & size) == 0;
                x = lower == desc ? (x > y ? x : y) : (x < y ? x : y);
            }
        }
        const unsigned nlo = __shfl_down(static_cast<unsigned>(x), 1);
        const unsigned nhi = __shfl_down(static_cast<unsigned>(x >> 32), 1);
        const unsigned long long xn = (static_cast<unsigned long long>(nhi) << 32) | nlo;
        if (lane < N) {
            const int n = static_cast<int>(0xffffffffu - static_cast<unsigned>(x & 0xffffffffu));
            const int4 in = info[n];
            const int2 ti = tinfo[n];
            sched[2 * lane] = make_int4(n, in.z, in.x, in.y);
            sched[2 * lane + 1] = make_int4(in.w, ti.x, ti.y, 0);
            const bool nonempty = (x >> 32) > 1;
            const bool next_empty = lane + 1 == N || (xn >> 32) <= 1;
            if ((nonempty && next_empty) || (lane == 0 && !nonempty)) {
                sched[2 * N] = make_int4(nonempty ? lane + 1 : 0, 0, 0, 0);
            }
        }
        return;
    }
    for (int i = N + tid; i < npad; i += 1024) {
        key[i] = 0ull;
    }
    __syncthreads();
    for (int size = 2; size <= npad; size <<= 1) {
        for (int stride = size >> 1; stride > 0; stride >>= 1) {
            for (int i = tid; i < npad; i += 1024) {
                const int pj = i ^ stride;
                if (pj > i) {
                    const bool desc = (i & size) == 0;
                    const unsigned long long x = key[i];
                    const unsigned long long y = key[pj];
                    if (desc ? x < y : x > y) {
                        key[i] = y;
                        key[pj] = x;
                    }
                }
            }
            __syncthreads();
        }
    }
    for (int r = tid; r < N; r += 1024) {
        const unsigned long long x = key[r];
        const int n = static_cast<int>(0xffffffffu - static_cast<unsigned>(x & 0xffffffffu));
        const int4 in = info[n];
        const int2 ti = tinfo[n];
        sched[2 * r] = make_int4(n, in.z, in.x, in.y);
        sched[2 * r + 1] = make_int4(in.w, ti.x, ti.y, 0);
        const bool nonempty = (x >> 32) > 1;
        const bool next_empty = r + 1 == N || (key[r + 1] >> 32) <= 1;
        if ((nonempty && next_empty) || (r == 0 && !nonempty)) {
            sched[2 * N] = make_int4(nonempty ? r + 1 : 0, 0, 0, 0);
        }
    }
}

// ---------------------------------------------------------------------------
// K1: per (chunk, head) intra-chunk work.
//
// 69 KiB of LDS (two workgroups per CU, which its registers allow; at three,
// forced, it ran no faster). The chunk's k, g, beta and each wave's q rows
// are loaded up front (v is not read here). k is normalized once and kept
// in fp32, so every operand built from it reads ready values; the decay is
// accumulated in log2 units, so each exponential is one v_exp_f32. X, LT and
// the T^T fragments lie over the cumsum and k tiles once those are dead.
// ---------------------------------------------------------------------------

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kPadF = 132;  // fp32 row stride of [64][128] tiles (16-lane float4 reads)
constexpr int kPadX = 68;   // fp32 row stride of [64][64] tiles (16-B rows)

__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }

// Akk / Aqk exponent anchor: row 7 of each 16-row block, and the largest
// exponent (log2 units) a factor may take before it is clamped. A chunk in
// which some block's factors would span more than kExactExp2 (the margin
// covers the rounding of the cumsum) takes the exact form instead.
constexpr int kAnchorRow = 7;
constexpr float kMaxExp2 = 126.f;
constexpr float kExactExp2 = 125.f;

// All-ones if `keep`, else zero, opaque to the optimizer: a value masked with
// it is used unconditionally, so its load cannot be sunk into a branch (a
// load under a per-lane branch is waited for before the next one issues).
__device__ __forceinline__ uint32_t keep_mask(bool keep) {
    uint32_t m = keep ? 0xffffffffu : 0u;
    asm volatile("" : "+v"(m));
    return m;
}

// gfx950's transposing LDS read ds_read_b64_tr_b16: within each group of 16
// lanes, lane 16G + i receives as element m the (i % 4)-th 16-bit value of
// the 8-byte word addressed by lane 16G + 4m + i / 4.
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4;

struct PrepShared {
    union {
        struct {
            float G[BT][kPadF];     // cumsum of the log2 decay (S1-S4)
            float K[BT][kPadF];     // k normalized (or as is), fp32 (S1-S4)
            float qss[2][BT];       // sum of q^2 over each channel half, per row (S1-S3)
        } early;
        struct {
            float X[BT][kPadX];  // (I + L)^-1; T = X diag(beta) (S5-S6)
            // Strict upper triangle: L^T, LT[j][i] = beta_i Akk[i][j] (j < i).
            // Lower triangle with the diagonal: Aqk[i][j] (j <= i).
            float LT[BT][kPadX];
            u32x4 TT[4][2][2][64];  // T^T A fragments (row tile, token slice, hi / lo) (S6)
            int ttsh[4];            // their power-of-two shift per row tile
        } mid;
    } u;
    float beta[BT];
    float gsum[4][DK];  // each wave's two row groups' decay sums (the cumsum's carries)
    alignas(16) int far[4];  // per wave: some anchor factor of its rows spans > kExactExp2
};
static_assert(sizeof(PrepShared) <= 80 * 1024, "two prepare workgroups per CU");

// Chunks [c_lo, c_hi) of the launch (global chunk indices: one sequence's
// own chunks, or all sequences' through the chunk index); chunk c's record
// goes to ring slot c % ring. Two workgroups per CU is what the LDS allows,
// so the register budget is that of two waves per SIMD (256 per lane): the
// compiler then keeps S3's MFMA results in VGPRs instead of AGPRs.
// seg_w > 0 (the affine form of one sequence): the chunks are numbered in
// segments of seg_w and every segment's first chunks are written last,
// since the affine form's first pass scans all segments at once.
template <int GATE>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(2, 2))) void chunk_prepare_kernel(
    const KdaChunkArgs a, char *ws, int ring, int c_lo, int c_hi, int seg_w) {
    __shared__ PrepShared sm;
    // Workgroups run chunk-descending, heads fastest: the scan starts with the
    // first chunk of every sequence and head, so those records are written
    // last and are still in the memory-side cache when it reads them (plain
    // write-back stores; with this order they beat nontemporal ones by 2%).
    const int H = a.num_heads;
    int c = (c_hi - 1) - static_cast<int>(blockIdx.x) / H;
    if (seg_w > 0) {
        const int segs = (c_hi + seg_w - 1) / seg_w;
        const int i = static_cast<int>(blockIdx.x) / H;
        c = (i % segs) * seg_w + (seg_w - 1 - i / segs);
        if (c >= c_hi) {
            return;
        }
    }
    const int h = static_cast<int>(blockIdx.x) % H;
    const int N = a.num_seqs;
    const Layout LY = layout(a.num_tokens, N, H, ring);
    int n = 0;
    int jc = c;
    int bos, eos;
    if (c < c_lo) {
        return;
    }
    if (N == 1) {
        // one sequence: chunk c is its c-th (no chunk-index pass ran)
        seq_bounds(a, 0, bos, eos);
        const int nch = (eos - bos + BT - 1) / BT;
        if (c >= nch) {
            return;
        }
    } else {
        const int *cs = reinterpret_cast<const int *>(ws + LY.chunk_start);
        if (c >= cs[N]) {
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
        n = lo;
        jc = c - cs[n];
        seq_bounds(a, n, bos, eos);
    }
    const int t0 = bos + BT * jc;
    const int len = eos - t0 < BT ? eos - t0 : BT;

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int r = lane & 15;
    const int gq = lane >> 4;
    char *rec = ws + LY.recs + (static_cast<size_t>(c % ring) * H + h) * kRecBytes;
    const bool norm = GATE == KDA_GATE_RAW || a.qk_l2norm != 0;
    const uint16_t *qp = static_cast<const uint16_t *>(a.q);

    // S3 work units: (row block I, channel half sh = slices 2sh and 2sh+1),
    // each with its pairs (I, J <= I); the two halves of every product are
    // summed through LDS (half 1 stores, half 0 adds after a barrier). Five
    // half-pairs and two half-blocks per wave:  wave 0: (3,0) (0,0)   wave 1: (3,1) (0,1)
    //        wave 2: (2,0) (1,0)   wave 3: (2,1) (1,1)
    const int sh = wave & 1;
    const int IA = wave < 2 ? 3 : 2;
    // q rows of both blocks in this wave's channel half (loaded in S1, after
    // k, g and beta, which S1 needs first): lane (r, gq) holds
    // q[16I + r][32s + kperm(gq, e)] as 2 x (4 bf16) for slices s = 2 sh + q2
    uint2 qraw[2][2][2];
    // widened q: 8 channels {32s + kperm(gq, e)} of slice s = 2 sh + q2, the
    // padding rows zeroed (loaded from a row clamped into the chunk)
    auto q8 = [&](int ii, int q2, float x[8]) {
        uint2 q0 = qraw[ii][q2][0];
        uint2 q1 = qraw[ii][q2][1];
        if (len < BT) {
            const uint32_t keep = keep_mask(16 * (ii == 0 ? IA : 3 - IA) + r < len);
            q0 = make_uint2(q0.x & keep, q0.y & keep);
            q1 = make_uint2(q1.x & keep, q1.y & keep);
        }
        x[0] = __uint_as_float(q0.x << 16);
        x[1] = __uint_as_float(q0.x & 0xffff0000u);
        x[2] = __uint_as_float(q0.y << 16);
        x[3] = __uint_as_float(q0.y & 0xffff0000u);
        x[4] = __uint_as_float(q1.x << 16);
        x[5] = __uint_as_float(q1.x & 0xffff0000u);
        x[6] = __uint_as_float(q1.y << 16);
        x[7] = __uint_as_float(q1.y & 0xffff0000u);
    };

    // ---- S1: k rows, log2 decay, beta (zero-padded); the q rows' loads ------
    const int kc = tid & 31;
    const int rg = tid >> 5;
    float4 gcum[8];  // the in-chunk prefix of this lane's rows, then the cumsum
    float4 gprev;    // the partner row group's sum (odd rg) or zero
    {
        const uint16_t *kp = static_cast<const uint16_t *>(a.k);
        float expA = 0.f;
        float4 dtb = make_float4(0.f, 0.f, 0.f, 0.f);
        if constexpr (GATE == KDA_GATE_RAW) {
            expA = expf(a.A_log[h]);
            dtb = load4(a.dt_bias + static_cast<int64_t>(h) * DK + 4 * kc);
        }
        // Loads are unconditional, from a row clamped into the chunk (a chunk
        // holds at least one token); padding rows are zeroed afterwards.
        // beta of row (tid & 63), used by the first wave
        const int tb = (tid & 63) < len ? (tid & 63) : len - 1;
        float braw;
        if constexpr (GATE == KDA_GATE_RAW) {
            braw = bf16_to_f32(static_cast<const uint16_t *>(a.beta)[static_cast<int64_t>(t0 + tb) * H + h]);
        } else {
            braw = static_cast<const float *>(a.beta)[static_cast<int64_t>(t0 + tb) * H + h];
        }
        // lane (rg, kc) carries rows 8 rg .. 8 rg + 7, channels 4 kc .. 4 kc + 3
        uint2 kraw[8];
        float4 g4[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int t = 8 * rg + i;
            const int tc = t < len ? t : len - 1;
            const int64_t base = (static_cast<int64_t>(t0 + tc) * H + h) * DK + 4 * kc;
            kraw[i] = *reinterpret_cast<const uint2 *>(kp + base);
            if constexpr (GATE == KDA_GATE_RAW) {
                g4[i] = load4(static_cast<const uint16_t *>(a.gate) + base);
            } else {
                g4[i] = load4(static_cast<const float *>(a.gate) + base);
            }
        }
        // the q rows, behind them
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int t = 16 * (ii == 0 ? IA : 3 - IA) + r;
#pragma unroll
            for (int q2 = 0; q2 < 2; ++q2) {
                const int s = 2 * sh + q2;
                const int tc = t < len ? t : len - 1;
                const uint16_t *row = qp + (static_cast<int64_t>(t0 + tc) * H + h) * DK + 32 * s;
                qraw[ii][q2][0] = *reinterpret_cast<const uint2 *>(row + 4 * gq);
                qraw[ii][q2][1] = *reinterpret_cast<const uint2 *>(row + 16 + 4 * gq);
            }
        }
        if constexpr (GATE == KDA_GATE_RAW) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const float4 av = g4[i];
                const float lb = a.lower_bound;
                // lb * sigmoid(x), the reciprocal as v_rcp_f32 (within 1 ulp)
                g4[i].x = lb * __builtin_amdgcn_rcpf(1.0f + __expf(-(expA * (av.x + dtb.x))));
                g4[i].y = lb * __builtin_amdgcn_rcpf(1.0f + __expf(-(expA * (av.y + dtb.y))));
                g4[i].z = lb * __builtin_amdgcn_rcpf(1.0f + __expf(-(expA * (av.z + dtb.z))));
                g4[i].w = lb * __builtin_amdgcn_rcpf(1.0f + __expf(-(expA * (av.w + dtb.w))));
            }
        }
        if (len < BT) {  // a partial chunk: its padding rows' k and g become zero
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const uint32_t keep = keep_mask(8 * rg + i < len);
                kraw[i].x &= keep;
                kraw[i].y &= keep;
                g4[i].x = __uint_as_float(__float_as_uint(g4[i].x) & keep);
                g4[i].y = __uint_as_float(__float_as_uint(g4[i].y) & keep);
                g4[i].z = __uint_as_float(__float_as_uint(g4[i].z) & keep);
                g4[i].w = __uint_as_float(__float_as_uint(g4[i].w) & keep);
            }
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int t = 8 * rg + i;
            const float4 k4 = make_float4(__uint_as_float(kraw[i].x << 16), __uint_as_float(kraw[i].x & 0xffff0000u),
                                          __uint_as_float(kraw[i].y << 16), __uint_as_float(kraw[i].y & 0xffff0000u));
            // the row's 1 / norm (every lane of the 32-lane row group holds it;
            // v_rsq_f32, within 1 ulp, where 1 / sqrtf takes ~30 instructions)
            const float rn = norm ? __builtin_amdgcn_rsqf(group_sum32(dot4(k4, k4)) + 1e-6f) : 1.0f;
            *reinterpret_cast<float4 *>(&sm.u.early.K[t][4 * kc]) =
                make_float4(k4.x * rn, k4.y * rn, k4.z * rn, k4.w * rn);
        }
        // S2, the in-chunk cumsum of the log2 decay: this lane's eight rows in
        // registers, then the row groups before it: its half-wave partner
        // (rg - 1, for odd rg) by a lane exchange, earlier waves' pairs
        // through LDS
        float4 run = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            run.x += g4[i].x * kLog2e;
            run.y += g4[i].y * kLog2e;
            run.z += g4[i].z * kLog2e;
            run.w += g4[i].w * kLog2e;
            gcum[i] = run;
        }
        const float4 other = make_float4(__shfl_xor(run.x, 32), __shfl_xor(run.y, 32), __shfl_xor(run.z, 32),
                                         __shfl_xor(run.w, 32));
        const bool odd = (rg & 1) != 0;
        if (odd) {
            *reinterpret_cast<float4 *>(&sm.gsum[wave][4 * kc]) =
                make_float4(other.x + run.x, other.y + run.y, other.z + run.z, other.w + run.w);
        }
        // The anchor factors' largest exponents in this lane's rows: rows
        // 16I .. 16I + 7 (even rg) end at the anchor, so e^(G_16I - anchor)
        // is their row factor; rows 16I + 8 .. 16I + 15 (odd rg) start after
        // it, so e^(anchor - G_16I+15) is their column factor (decays g <= 0)
        {
            const float4 d = odd ? make_float4(-run.x, -run.y, -run.z, -run.w)
                                 : make_float4(gcum[0].x - run.x, gcum[0].y - run.y, gcum[0].z - run.z,
                                               gcum[0].w - run.w);
            const bool far = fmaxf(fmaxf(d.x, d.y), fmaxf(d.z, d.w)) > kExactExp2;
            // every lane stores the wave's same value (no branch)
            sm.far[wave] = __ballot(far) != 0ull;
        }
        gprev = odd ? other : make_float4(0.f, 0.f, 0.f, 0.f);
        if (tid < BT) {
            float b = braw;
            if constexpr (GATE == KDA_GATE_RAW) {
                b = __builtin_amdgcn_rcpf(1.0f + __expf(-b));
            }
            sm.beta[tid] = tid < len ? b : 0.f;
        }
    }
    lds_barrier();
    {
        // the cumsum rows of this lane: its own prefix, the earlier waves'
        // pair totals, and its partner's total
        float4 add = gprev;
        for (int w2 = 0; w2 < wave; ++w2) {
            const float4 p4 = *reinterpret_cast<const float4 *>(&sm.gsum[w2][4 * kc]);
            add.x += p4.x;
            add.y += p4.y;
            add.z += p4.z;
            add.w += p4.w;
        }
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            *reinterpret_cast<float4 *>(&sm.u.early.G[8 * rg + i][4 * kc]) =
                make_float4(gcum[i].x + add.x, gcum[i].y + add.y, gcum[i].z + add.z, gcum[i].w + add.w);
        }
    }
    if (norm) {
        // this wave's half of each q row's sum of squares (4 lane groups x
        // 2 slices), one lane per row writes it
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            float x[8];
            float ss = 0.f;
#pragma unroll
            for (int q2 = 0; q2 < 2; ++q2) {
                q8(ii, q2, x);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    ss += x[e] * x[e];
                }
            }
            ss += __shfl_xor(ss, 16);
            ss += __shfl_xor(ss, 32);
            if (gq == 0) {
                sm.u.early.qss[sh][16 * (ii == 0 ? IA : 3 - IA) + r] = ss;
            }
        }
    }
    lds_barrier();

    // 8 channels {32s + kperm(gq, e)} of one row: two 16-byte reads each
    // from the (normalized) k and the cumsum tiles.
    auto load_k8 = [&](int row, int s, float x[8]) {
        const float4 k0 = *reinterpret_cast<const float4 *>(&sm.u.early.K[row][32 * s + 4 * gq]);
        const float4 k1 = *reinterpret_cast<const float4 *>(&sm.u.early.K[row][32 * s + 16 + 4 * gq]);
        x[0] = k0.x;
        x[1] = k0.y;
        x[2] = k0.z;
        x[3] = k0.w;
        x[4] = k1.x;
        x[5] = k1.y;
        x[6] = k1.z;
        x[7] = k1.w;
    };
    auto load_g8 = [&](int row, int s, float x[8]) {
        const float4 g0 = *reinterpret_cast<const float4 *>(&sm.u.early.G[row][32 * s + 4 * gq]);
        const float4 g1 = *reinterpret_cast<const float4 *>(&sm.u.early.G[row][32 * s + 16 + 4 * gq]);
        x[0] = g0.x;
        x[1] = g0.y;
        x[2] = g0.z;
        x[3] = g0.w;
        x[4] = g1.x;
        x[5] = g1.y;
        x[6] = g1.z;
        x[7] = g1.w;
    };

    // The exact form of pair (I, J) over this wave's channel half, for a
    // chunk whose anchor factors would be clamped: every element's own
    // e^(G_i - G_j) (<= 1 for j <= i under decay; the entries above the
    // diagonal, which nothing reads, are clamped), in fp32. For each row x
    // of the block, lane (r, gq) sums its 16 channels of Akk[16I + x][16J + r]
    // and Aqk[16I + r][16J + x]; the four lanes of each r add their channels,
    // and the lane whose MFMA layout holds the entry keeps it.
    auto exact_pair = [&](int I, int J, int ri, const float (&qv)[2][8], float qscale, f32x4 &akk, f32x4 &aqt) {
#pragma unroll 1
        for (int x = 0; x < 16; ++x) {
            float a = 0.f, b = 0.f;
#pragma unroll 1
            for (int sl = 0; sl < 2; ++sl) {
                const int s = 2 * sh + sl;
                float kj[8], gj[8], gi[8], kx[8], gx[8], ky[8], gy[8];
                load_k8(16 * J + r, s, kj);
                load_g8(16 * J + r, s, gj);
                load_g8(ri, s, gi);
                load_k8(16 * I + x, s, kx);
                load_g8(16 * I + x, s, gx);
                load_k8(16 * J + x, s, ky);
                load_g8(16 * J + x, s, gy);
                const float *q = sl == 0 ? qv[0] : qv[1];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    a = fmaf(kx[e] * kj[e], ex2(fminf(gx[e] - gj[e], kMaxExp2)), a);
                    b = fmaf(q[e] * ky[e], ex2(fminf(gi[e] - gy[e], kMaxExp2)), b);
                }
            }
            a += __shfl_xor(a, 16);
            a += __shfl_xor(a, 32);
            b += __shfl_xor(b, 16);
            b += __shfl_xor(b, 32);
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (x == 4 * gq + e) {
                    akk[e] = a;
                    aqt[e] = b * qscale;
                }
            }
        }
    };

    // ---- S3: Akk (-> L^T), Aqk (-> LT's lower triangle), q e^G fragments ----
    // Each wave sums its pairs over its channel half; the partial products
    // stay in registers until the k and cumsum tiles are dead (after S4), and
    // the halves are then summed in LT.
    f32x4 pk[2][4], pq[2][4];  // this half's partials of pair (I, J): Akk, Aqk
#pragma unroll
    for (int ii = 0; ii < 2; ++ii) {
        const int I = ii == 0 ? IA : 3 - IA;
        const int ri = 16 * I + r;
        // q row: this half's channels, scaled by the norm over all 128
        // (the two halves' sums of squares meet in LDS during S1)
        float qv[2][8];
        q8(ii, 0, qv[0]);
        q8(ii, 1, qv[1]);
        float qscale = a.scale;
        if (norm) {
            qscale = a.scale * __builtin_amdgcn_rsqf(sm.u.early.qss[0][ri] + sm.u.early.qss[1][ri] + 1e-6f);
        }
        // The block's anchor row G[16I + 7][.]: a row factor e^(G_i - anchor)
        // of the block spans at most 7 tokens of decay above 1, a column
        // factor e^(anchor - G_j) at most 8 (diagonal block, j > anchor) and
        // is e^(<=0) for every earlier block, so fp32 and bf16 hold both while
        // 8 consecutive tokens decay by less than 2^kMaxExp2 (about 87 nat).
        // Beyond that the exponents are clamped: results stay finite but are
        // no longer exact (the precondition stated with the C ABI).
        float anc[2][8];
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
            load_g8(16 * I + kAnchorRow, 2 * sh + sl, anc[sl]);
        }
        bf16x8 Rh[2], Rl[2], Qh[2], Ql[2];
        float qg[2][8];  // q e^G of this half's two slices: one record scale
        float ke[2][8];  // e^G k of the same rows and channels: one record scale
        float l1 = 0.f;  // this lane's share of the row's sum of |e^G k| over the half
#pragma unroll
        for (int sl = 0; sl < 2; ++sl) {
            const int s = 2 * sh + sl;
            float kk[8], gg[8], rv[8], qa[8];
            load_k8(ri, s, kk);
            load_g8(ri, s, gg);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float ex = ex2(fminf(gg[e] - anc[sl][e], kMaxExp2));
                const float eg = ex2(gg[e]);
                const float qn = qv[sl][e] * qscale;
                rv[e] = kk[e] * ex;
                qa[e] = qn * ex;
                qg[sl][e] = qn * eg;
                ke[sl][e] = kk[e] * eg;
                l1 += fabsf(ke[sl][e]);
            }
            split_bf16x8(rv, Rh[sl], Rl[sl]);
            split_bf16x8(qa, Qh[sl], Ql[sl]);
        }
        float *sc = reinterpret_cast<float *>(rec + kOffSc);
        store_frags_f16<2>(rec, kOffQg, I * 4 + 2 * sh, sc + kScQg + I * 4 + 2 * sh, lane, qg, 2);
        // e^G k: the A fragments of row tile I, slices 2sh and 2sh+1, for the
        // scan's (e^G k) S; and this half's max over the tile's rows of
        // sum_k |e^G k|, which the scan adds to the other half's to bound that
        // product with max |S|
        store_frags_f16<2>(rec, kOffKe, I * 4 + 2 * sh, sc + kScKe + I * 4 + 2 * sh, lane, ke, 2);
        l1 += __shfl_xor(l1, 16);
        l1 += __shfl_xor(l1, 32);
        l1 = wave_max_mag(l1);
        if (lane == 0) {
            sc[kScKel1 + 4 * sh + I] = l1;
        }
        // pairs (I, J), J <= I, over this half's channels
#pragma unroll
        for (int J = 0; J < (ii == 0 ? 4 : 2); ++J) {
            if (J > I) {
                break;  // uniform per wave
            }
            const int rj = 16 * J + r;
            f32x4 akk = {0.f, 0.f, 0.f, 0.f};
            f32x4 aqt = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sl = 0; sl < 2; ++sl) {
                const int s = 2 * sh + sl;
                float kk[8], gg[8], cv[8];
                load_k8(rj, s, kk);
                load_g8(rj, s, gg);
                // blocks 0 and 1 against the upper row block I = IA >= 2 are
                // earlier blocks: anchor - G_j <= 0 (g <= 0), no clamp needed
                const bool earlier = ii == 0 && J < 2;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float d = anc[sl][e] - gg[e];
                    cv[e] = kk[e] * ex2(earlier ? d : fminf(d, kMaxExp2));
                }
                bf16x8 Ch, Cl;
                split_bf16x8(cv, Ch, Cl);
                // Akk in three passes like Aqk: with one, its bf16 rounding
                // (2^-9 per term) reaches T, and where the decay is weak the
                // state keeps every chunk's error (8.5e-4 against 3.5e-4 of
                // the final state's max after 16384 tokens at g ~ -1e-4)
                akk = mfma(Rh[sl], Ch, akk);  // Akk[16I + 4gq + e][16J + r]
                akk = mfma(Rh[sl], Cl, akk);
                akk = mfma(Rl[sl], Ch, akk);
                aqt = mfma(Ch, Qh[sl], aqt);  // Aqk[16I + r][16J + 4gq + e]
                aqt = mfma(Ch, Ql[sl], aqt);
                aqt = mfma(Cl, Qh[sl], aqt);
            }
            // lane (r, gq) holds Akk[16I + 4gq + e][16J + r] and Aqk[16I + r][16J + 4gq + e]
            pk[ii][J] = akk;
            pq[ii][J] = aqt;
        }
    }
    // ---- S4: kd fragments (kept for S6), e^(G_last), tracking operands, e^G k
    // fragments of the record --------------------------------------------------
    // k[t][16mk + r] for the rows t = 32s + kperm(gq, e) of a kd^T fragment:
    // eight column reads (rows 4 apart land 16 banks apart, so none conflict)
    auto kd_rows = [&](int s, int mk, float (&kr)[8]) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            kr[e] = sm.u.early.K[32 * s + kperm(gq, e)][16 * mk + r];
        }
    };
    // kd[t][16mk + r] = k_t e^(G_last - G_t) for the rows t = 32s + kperm(gq, e)
    // (B fragments of T^T kd, mk = 2 wave + tt), fp16 hi + lo with one
    // power-of-two scale 2^-shift per mk; S6 uses them from registers.
    u32x4 kdh[2][2], kdl[2][2];
    int kdsh[2];
    auto to_frags = [&](const float (&x)[2][8], u32x4 (&fh)[2], u32x4 (&fl)[2], int &shift) {
        float m = 0.f;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                m = fmaxf(m, fabsf(x[s][e]));
            }
        }
        const int sh = f16_shift(wave_max_mag(m));
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            f16x8 hi, lo;
            split_f16x8(x[s], sh, hi, lo);
            fh[s] = as_u32x4(hi);
            fl[s] = as_u32x4(lo);
        }
        shift = sh;
    };
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int mk = 2 * wave + tt;
        const int k = 16 * mk + r;
        const float gl = sm.u.early.G[BT - 1][k];
        float x[2][8];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            float kr[8];
            kd_rows(s, mk, kr);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int t = 32 * s + kperm(gq, e);
                x[s][e] = kr[e] * ex2(gl - sm.u.early.G[t][k]);
            }
        }
        to_frags(x, kdh[tt], kdl[tt], kdsh[tt]);
    }
    if (tid < DK) {
        reinterpret_cast<float *>(rec + kOffGl)[tid] = ex2(sm.u.early.G[BT - 1][tid]);
    }
    // The tracked prefix inside this chunk (0 < rr < len): its state is
    // e^(G_{rr-1}) S + (e^(G_{rr-1} - G_t) k_t)_{t<rr}^T vnew, i.e.
    // e^(G_{rr-1}) S + (T^T kd_r)^T y with kd_r that prefix's kd; its kd
    // fragments wait in registers for S6, like the chunk's.
    bool tracked = false;
    char *tr = nullptr;
    u32x4 kth[2][2], ktl[2][2];
    int ktsh[2] = {0, 0};
    if (a.track_indices != nullptr) {
        const int ts = a.track_indices[n];
        const int tl = a.track_lens[n];
        const int rr = tl - BT * jc;
        if (ts > 0 && static_cast<int64_t>(ts) < a.num_slots && rr > 0 && rr < len) {
            tracked = true;
            tr = ws + LY.tracks + (static_cast<size_t>(n) * H + h) * kTrBytes;
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
                const int mk = 2 * wave + tt;
                const int k = 16 * mk + r;
                const float gr = sm.u.early.G[rr - 1][k];
                float x[2][8];
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    float kr[8];
                    kd_rows(s, mk, kr);
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int t = 32 * s + kperm(gq, e);
                        x[s][e] = t < rr ? kr[e] * ex2(gr - sm.u.early.G[t][k]) : 0.f;
                    }
                }
                to_frags(x, kth[tt], ktl[tt], ktsh[tt]);
            }
            if (tid < DK) {
                reinterpret_cast<float *>(tr + kTrOffGl)[tid] = ex2(sm.u.early.G[rr - 1][tid]);
            }
        }
    }
    // A chunk beyond the anchors' span: S3's products were formed from
    // clamped factors; the exact form replaces them here, behind S4 and
    // before G and K die (the q rows reloaded, so nothing of S3 stays live
    // for it). The flags are read only here: their wait would otherwise
    // land on the cumsum's path.
    const bool exact = __builtin_amdgcn_readfirstlane(sm.far[0] | sm.far[1] | sm.far[2] | sm.far[3]) != 0;
    if (__builtin_expect(exact, 0)) {  // laid out after the kernel's straight-line path
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int I = ii == 0 ? IA : 3 - IA;
            const int ri = 16 * I + r;
            int tc = ri < len ? ri : len - 1;
            // opaque, so this address is formed here rather than shared with
            // S1's q loads (whose registers would then stay live through S4)
            asm volatile("" : "+v"(tc));
            const uint16_t *row = qp + (static_cast<int64_t>(t0 + tc) * H + h) * DK;
            const uint32_t keep = keep_mask(ri < len);
            float qv[2][8];
#pragma unroll
            for (int q2 = 0; q2 < 2; ++q2) {
                const int s = 2 * sh + q2;
                const uint2 q0 = *reinterpret_cast<const uint2 *>(row + 32 * s + 4 * gq);
                const uint2 q1 = *reinterpret_cast<const uint2 *>(row + 32 * s + 16 + 4 * gq);
                const uint32_t w[4] = {q0.x & keep, q0.y & keep, q1.x & keep, q1.y & keep};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    qv[q2][2 * e] = __uint_as_float(w[e] << 16);
                    qv[q2][2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
                }
            }
            float qscale = a.scale;
            if (norm) {
                qscale = a.scale * __builtin_amdgcn_rsqf(sm.u.early.qss[0][ri] + sm.u.early.qss[1][ri] + 1e-6f);
            }
            const int nj = ii == 0 ? I + 1 : (I + 1 < 2 ? I + 1 : 2);
#pragma unroll 1
            for (int J = 0; J < nj; ++J) {
                f32x4 akk = {0.f, 0.f, 0.f, 0.f};
                f32x4 aqt = {0.f, 0.f, 0.f, 0.f};
                exact_pair(I, J, ri, qv, qscale, akk, aqt);
#pragma unroll
                for (int Js = 0; Js < (ii == 0 ? 4 : 2); ++Js) {
                    if (Js == J) {
                        pk[ii][Js] = akk;
                        pq[ii][Js] = aqt;
                    }
                }
            }
        }
    }

    lds_barrier();  // G and K are dead from here on
    // S3's two channel halves meet in LT, which lies over the dead G: half
    // sh = 1 stores its partial products, then half sh = 0 adds its own and
    // applies beta. Every LT element is written: block (J, I), J < I, holds
    // Akk^T; block (I, J), J < I, holds Aqk; a diagonal block holds Akk^T
    // above and Aqk on and below its diagonal.
    if (sh == 1) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int I = ii == 0 ? IA : 3 - IA;
#pragma unroll
            for (int J = 0; J < (ii == 0 ? 4 : 2); ++J) {
                if (J > I) {
                    break;
                }
                if (J < I) {
                    *reinterpret_cast<f32x4 *>(&sm.u.mid.LT[16 * J + r][16 * I + 4 * gq]) = pk[ii][J];
                    *reinterpret_cast<f32x4 *>(&sm.u.mid.LT[16 * I + r][16 * J + 4 * gq]) = pq[ii][J];
                } else {
                    f32x4 m;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        m[e] = r < 4 * gq + e ? pk[ii][J][e] : pq[ii][J][e];
                    }
                    *reinterpret_cast<f32x4 *>(&sm.u.mid.LT[16 * I + r][16 * I + 4 * gq]) = m;
                }
            }
        }
    }
    // X: the six upper 16x16 blocks (I, J > I) zero, one float4 per store
    for (int f = tid; f < 6 * 64; f += kThreads) {
        const int blk = f >> 6;                      // (0,1) (0,2) (0,3) (1,2) (1,3) (2,3)
        const int bi = blk < 3 ? 0 : (blk < 5 ? 1 : 2);
        const int bj = blk < 3 ? blk + 1 : (blk < 5 ? blk - 1 : 3);
        const int row = (f & 63) >> 2;
        *reinterpret_cast<float4 *>(&sm.u.mid.X[16 * bi + row][16 * bj + 4 * (f & 3)]) =
            make_float4(0.f, 0.f, 0.f, 0.f);
    }
    lds_barrier();
    if (sh == 0) {
#pragma unroll
        for (int ii = 0; ii < 2; ++ii) {
            const int I = ii == 0 ? IA : 3 - IA;
            const float4 b4 = *reinterpret_cast<const float4 *>(&sm.beta[16 * I + 4 * gq]);
            const f32x4 bv = {b4.x, b4.y, b4.z, b4.w};
#pragma unroll
            for (int J = 0; J < (ii == 0 ? 4 : 2); ++J) {
                if (J > I) {
                    break;
                }
                if (J < I) {
                    f32x4 *pa = reinterpret_cast<f32x4 *>(&sm.u.mid.LT[16 * J + r][16 * I + 4 * gq]);
                    f32x4 *pb = reinterpret_cast<f32x4 *>(&sm.u.mid.LT[16 * I + r][16 * J + 4 * gq]);
                    const f32x4 xa = *pa;
                    const f32x4 xb = *pb;
                    *pa = (xa + pk[ii][J]) * bv;
                    *pb = xb + pq[ii][J];
                } else {
                    f32x4 *pd = reinterpret_cast<f32x4 *>(&sm.u.mid.LT[16 * I + r][16 * I + 4 * gq]);
                    const f32x4 xd = *pd;
                    f32x4 m;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        m[e] = r < 4 * gq + e ? (xd[e] + pk[ii][J][e]) * bv[e] : xd[e] + pq[ii][J][e];
                    }
                    *pd = m;
                }
            }
        }
    }
    lds_barrier();

    // ---- S5: X = (I + L)^-1 (blocked, fp32); T = X diag(beta) is formed as S6 reads X
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
                const float4 t4 = *reinterpret_cast<const float4 *>(&sm.u.mid.LT[b0 + j][b0 + 4 * q]);
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
            sm.u.mid.X[b0 + i][b0 + col] = acc[i];
        }
    }
    lds_barrier();
    // Off-diagonal blocks by level d = I - J, one (I, J) per wave (wave J),
    // on the fp32 MFMA (v_mfma_f32_16x16x4_f32: lane (r, g) supplies A[r][g]
    // and B[g][r] of each 4-wide K step; C as for the bf16 tiles):
    //   M_IJ = sum_{K=J}^{I-1} L_IK X_KJ,   X_IJ = -X_II M_IJ.
    // M_IJ passes through the wave's still-zero upper block (J, I) of X, which
    // is cleared again before the level's barrier.
    for (int d = 1; d < 4; ++d) {
        const int J = wave;
        const int I = J + d;
        if (I < 4) {
            f32x4 m = {0.f, 0.f, 0.f, 0.f};
            for (int K = J; K < I; ++K) {
#pragma unroll
                for (int k4 = 0; k4 < 4; ++k4) {
                    const int kk = 16 * K + 4 * k4 + gq;
                    m = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.u.mid.LT[kk][16 * I + r],
                                                            sm.u.mid.X[kk][16 * J + r], m, 0, 0, 0);
                }
            }
            // lane (r, gq) holds M[4gq + i][r]; park it row-major in block (J, I)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sm.u.mid.X[16 * J + 4 * gq + i][16 * I + r] = m[i];
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            f32x4 x = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int k4 = 0; k4 < 4; ++k4) {
                x = __builtin_amdgcn_mfma_f32_16x16x4f32(sm.u.mid.X[16 * I + r][16 * I + 4 * k4 + gq],
                                                        sm.u.mid.X[16 * J + 4 * k4 + gq][16 * I + r], x,
                                                        0, 0, 0);
            }
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                sm.u.mid.X[16 * I + 4 * gq + i][16 * J + r] = -x[i];
                sm.u.mid.X[16 * J + 4 * gq + i][16 * I + r] = 0.f;
            }
        }
        lds_barrier();
    }

    // ---- S6: T^T kd and Aqk T, T = X diag(beta) --------------------------------
    // The scan never forms u = T v or w = T (e^G k): with y = v - (e^G k) S,
    // vnew = u - w S = T y, so the state update takes (T^T kd)^T y and the
    // output (Aqk T) y. Both are stored as A fragments: a pair of 16x16
    // result tiles over token rows [32s, 32s+16) and [32s+16, 32s+32) is the
    // A fragment of token slice s.
    float *sc = reinterpret_cast<float *>(rec + kOffSc);
    {
        // T^T fragments of row tile tt = wave (both token slices): lane (r, g)
        // element e holds T[32s + kperm(g, e)][16 wave + r] (zero where the
        // token is earlier than the column: X is lower triangular), fp16 hi +
        // lo with one scale per tile
        const int tcol = 16 * wave + r;
        const float bt = sm.beta[tcol];
        float tx[2][8];
        float m = 0.f;
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                tx[s][e] = sm.u.mid.X[32 * s + kperm(gq, e)][tcol] * bt;
                m = fmaxf(m, fabsf(tx[s][e]));
            }
        }
        const int sh = f16_shift(wave_max_mag(m));
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            f16x8 hi, lo;
            split_f16x8(tx[s], sh, hi, lo);
            sm.u.mid.TT[wave][s][0][lane] = as_u32x4(hi);
            sm.u.mid.TT[wave][s][1][lane] = as_u32x4(lo);
        }
        if (lane == 0) {
            sm.u.mid.ttsh[wave] = sh;
        }
    }
    lds_barrier();
    int ttsh[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt) {
        ttsh[tt] = sm.u.mid.ttsh[tt];
    }
    // T^T B (rows t, B's columns) for the B fragments bh[s] + bl[s] of a
    // 16-column block, B scaled by 2^bsh (three passes: T hi B hi, T hi B lo,
    // T lo B hi), K = token slices s >= tt / 2 (T^T is zero below); the four
    // row tiles land unscaled in x[2][8] in A-fragment order, tile tt's
    // exponent in ex[tt]
    auto ttb = [&](const u32x4 (&bh)[2], const u32x4 (&bl)[2], int bsh, float (&x)[2][8], int tmax,
                   int (&ex)[4]) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) {
            if (tt > tmax) {
                break;  // uniform per wave
            }
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int s = tt / 2; s < 2; ++s) {
                const f16x8 th = as_f16x8(sm.u.mid.TT[tt][s][0][lane]);
                acc = mfma(th, as_f16x8(bh[s]), acc);
                acc = mfma(th, as_f16x8(bl[s]), acc);
                acc = mfma(as_f16x8(sm.u.mid.TT[tt][s][1][lane]), as_f16x8(bh[s]), acc);
            }
            ex[tt] = -(ttsh[tt] + bsh);
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                x[tt >> 1][4 * (tt & 1) + i] = acc[i];
            }
        }
    };
    // (T^T kd) fragments, row tiles mk = 2 wave + tt of kd^T T
#pragma unroll
    for (int tt = 0; tt < 2; ++tt) {
        const int mk = 2 * wave + tt;
        float x[2][8];
        int ex[4];
        ttb(kdh[tt], kdl[tt], kdsh[tt], x, 3, ex);
        store_frags_f16_exp<2>(rec, kOffKd, mk * 2, sc + kScKd + mk, lane, x, ex);
    }
    if (tracked) {
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
            const int mk = 2 * wave + tt;
            float x[2][8];
            int ex[4];
            ttb(kth[tt], ktl[tt], ktsh[tt], x, 3, ex);
            store_frags_f16_exp<2>(tr, kTrOffKd, mk * 2, reinterpret_cast<float *>(tr + kTrOffSc) + mk, lane, x,
                                   ex);
        }
    }
    {
        // (Aqk T) fragments of row tile mt = wave: B = Aqk^T, lane (r, g)
        // element e = Aqk[16 wave + r][32s + kperm(g, e)] (zero above the
        // diagonal); tokens after the row's last contribute nothing, so only
        // the tiles tt <= wave are formed and slice 1 only for wave >= 2
        const int row = 16 * wave + r;
        float ax[2][8];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
            const float4 x0 = *reinterpret_cast<const float4 *>(&sm.u.mid.LT[row][32 * s + 4 * gq]);
            const float4 x1 = *reinterpret_cast<const float4 *>(&sm.u.mid.LT[row][32 * s + 16 + 4 * gq]);
            const float xv[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                ax[s][e] = 32 * s + kperm(gq, e) <= row ? xv[e] : 0.f;
            }
        }
        u32x4 aqh[2], aql[2];
        int aqsh;
        to_frags(ax, aqh, aql, aqsh);
        float x[2][8];
#pragma unroll
        for (int s = 0; s < 2; ++s) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                x[s][e] = 0.f;
            }
        }
        int ex[4] = {0, 0, 0, 0};
        ttb(aqh, aql, aqsh, x, wave, ex);
        float *asc = sc + kScAq + wave;
        if (wave < 2) {
            float x1[1][8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                x1[0][e] = x[0][e];
            }
            const int ex1[2] = {ex[0], ex[1]};
            store_frags_f16_exp<1>(rec, kOffAq, aq_frag(wave, 0), asc, lane, x1, ex1);
        } else {
            store_frags_f16_exp<2>(rec, kOffAq, aq_frag(wave, 0), asc, lane, x, ex);
        }
    }
}

// ---------------------------------------------------------------------------
// K2: the serial chunk scan per (sequence, head, CW = 16 NT value columns).
//
// Twelve waves in three roles. Every wave meets the same two workgroup
// barriers per chunk j: B1(j) after S_j is published, B2(j) after y_j is.
//   chain waves 0-3   own S rows [32c, 32c+32) x CW columns (fp32, registers)
//                     and run the recurrence: publish S_j, y_j = v - (e^G k)
//                     S_j, publish y_j, S_{j+1} = e^(G_last) S_j +
//                     (T^T kd)^T y_j;
//   output waves 4-7  own token rows [16o, 16o+16): (q e^G) S_j between B1(j)
//                     and B2(j), (Aqk T) y_j between B1(j+1) and B2(j+1)
//                     (Aqk T from the stage, y_j from its LDS hand-over),
//                     then o_j = the sum and its store after B2(j+1); they
//                     load their q e^G fragments themselves, a chunk ahead;
//   loader waves 8-11 copy the chain's operands of chunk j+1 (e^G k,
//                     (T^T kd)^T, Aqk T, e^(G_last), the scales) and this
//                     group's v (with its largest magnitude), loaded into
//                     their registers after B2(j-2), into the LDS stage of
//                     j+1's parity between B1(j) and B2(j) (every reader of
//                     that stage's previous chunk j-1 finished before B1(j)),
//                     then issue the loads of chunk j+3. The recurrence never
//                     waits to issue a global load.
// The affine form's first pass runs a lean variant: the chain waves load
// their e^G k and (T^T kd)^T fragments, and the output waves their Aqk T,
// from the record themselves a chunk ahead (every fragment has one reader
// wave), and the loaders stage only v and the misc fragment. Its chains,
// spread over the segments of one sequence, ran 6-11% faster so; the
// one-pass and segmented scans are faster staged.
// S_j, y_j and the stage are indexed by j's parity; a buffer of parity
// j&1 is rewritten only after B1(j+1) or later, when its chunk-j readers are
// done (the stage after B2(j+1): the output waves read its Aqk until then). One barrier B0 before the first chunk publishes
// the first stage; one after the last chunk covers the last hand-over.
//
// S_j is published as fp16 scaled per 32-row slice (the state itself stays
// fp32 in registers). y is exchanged as fp16 hi + lo scaled by 2^sv, where
// 2^-sv bounds |y| <= max|v| + max_t sum_k |(e^G k)[t][k]| max|S_j| (max|v|
// from the loaders, the sum from the record, max|S_j| from the publish)
// inside [2^13, 2^14): the pair holds y to ~2^-22 of that bound and cannot
// overflow.
//
// The chunk operands (~38 KiB of e^G k, (T^T kd)^T and Aqk T plus 16 KiB of
// q e^G) are the same for every column group of a (sequence, head), so a
// wider group (NT = 2) reads fewer operand bytes per unit of work; a
// narrower one (NT = 1) has the shorter serial step. The host picks NT from
// the number of chains.
// ---------------------------------------------------------------------------

constexpr int kScanThreads = 768;
// s_waitcnt vmcnt(0) (expcnt and lgkmcnt at their maxima: not waited for)
constexpr int kWaitVm0 = 0x0F70;
constexpr int kStKd = 16;  // stage fragment indices: e^G k at 0, (T^T kd)^T, Aqk T, then v
constexpr int kStAq = 32;
constexpr int kStV = 38;
static_assert(kOffKd == kStKd * kFrag && kOffAq == kStAq * kFrag && kOffQg == kStV * kFrag &&
                  kOffSc == kOffGl + DK * 4,
              "the stage copies the record's first 38 fragments in order, then gl and the scale block");

// Stage of one chunk for NT column tiles. Staged form: 38 shared fragments
// from the record, this group's v as a row-major bf16 tile [64][16 NT] at
// fragment kStV (loaded from the input; its region holds 4 NT fragments),
// then e^(G_last) [128] and the scale block [128]. Lean form (LEAN): the
// record's matrix operands are loaded by the waves that use them (each
// fragment has one reader), and the stage holds the v tile and the misc
// fragment (e^(G_last) and the scale block) only.
template <int NT, bool LEAN>
struct Stage {
    static constexpr int kV = LEAN ? 0 : kStV * kFrag;  // byte offset of the v tile
    static constexpr int kMisc = LEAN ? BT * 16 * NT * 2 : (kStV + 4 * NT) * kFrag;
    static constexpr int kBytes = kMisc + kFrag;
    static constexpr int kRecFrags = LEAN ? 1 : kStV + 1;  // copied from the record: shared fragments, misc
    static constexpr int kLoadPer = (kRecFrags + 3) / 4;   // record fragments per loader wave
    // stage and record offsets of record fragment f (the last one is misc)
    __device__ static int dst(int f) { return f < kRecFrags - 1 ? f * kFrag : kMisc; }
    __device__ static int src(int f) { return f < kRecFrags - 1 ? f * kFrag : kOffGl; }
};

template <int NT, bool LEAN>
struct ScanShared {
    char stg[2][Stage<NT, LEAN>::kBytes];  // chain operands by parity, fragments in lane order
    u32x4 sbuf[2][4][NT][64];                // S_j as fp16 B fragments: [parity][slice][tile][lane]
    u32x4 vbuf[2][2][2][NT][64];             // y_j as fp16 B fragments: [parity][slice][hi, lo][tile][lane]
    float sscale[2][4];                      // 2^-shift of each S_j slice in sbuf
    float smax[2][4];                        // max |S_j| of each slice
    float vmax[2][4];                        // max |v| of each row tile of the staged v
    uint32_t otile[4][16][8 * NT];           // per output wave: 16 rows x CW bf16 columns
};
static_assert(sizeof(ScanShared<2, false>) <= 160 * 1024, "the scan's LDS budget");

__device__ __forceinline__ f16x8 stage_frag(const char *st, int f, int lane) {
    return as_f16x8(reinterpret_cast<const u32x4 *>(st + f * kFrag)[lane]);
}

// SEG: one segment [s_lo, s_hi) of a single sequence's chunks (the state
// comes from the pool in the first segment and from the carry area after,
// goes to the carry area until the segment that holds the last chunk);
// without it every launch scans whole sequences and the segment logic
// compiles away. Chunk c's record is in ring slot c % ring.
//
// AFF: the first pass of the affine form of one sequence, s_lo = P
// segments of s_hi = W chunks. The scan is linear in (initial state, v), so
// a later segment s (chunks [sW, sW + W)) runs as two independent scans
// from its start: from zero with the real v (outputs o', final state Z_s)
// and from the identity with v = 0 (outputs O, final state Phi_s, the
// segment's transition), while segment 0 runs as usual from the pool.
// Every (role, head) is a chain of its own: role 0 is segment 0, roles
// 2s - 1 and 2s the zero-start and identity-start scans of segment s. The
// later roles write fp32 outputs and their final and tracked states to the
// affine areas; chunk_affine_combine_kernel and chunk_affine_correct_kernel
// finish the sequence.
//
// PERS: one pass over several sequences with one workgroup per CU. The
// workgroups form teams of NV (one per column group, on one XCD); team t of
// TM takes the (sequence, head) items of ranks k TM + t (k even) and k TM +
// TM - 1 - t (k odd) in the order chunk_index_kernel sorted them (longest
// first, so the teams' loads balance), and runs their chunks as one stream:
// virtual chunk J is local chunk j of item k. The loaders' look-ahead, the
// output waves' lag and the stage parity (J & 1) run across items, so an
// item's first chunks are staged while the previous one finishes, and the
// chain loads the next item's initial state a whole item ahead; what a
// workgroup per item paid at its start (about 3.9 us: dispatch, the first
// loads, the pipeline's fill and drain) is paid once per workgroup.
template <int NT, bool SEG, bool AFF = false, bool PERS = false>
__global__ __launch_bounds__(kScanThreads) void chunk_scan_kernel(const KdaChunkArgs a, const char *ws,
                                                                  int ring, int s_lo, int s_hi) {
    // the affine first pass runs the lean form (its chains, spread over the
    // segments of a long sequence, were measured faster loading their own
    // operands; the one-sequence-per-chain scan is faster staged)
    constexpr bool LEAN = AFF;
    using St = Stage<NT, LEAN>;
    constexpr int NV = 8 / NT;  // column groups per (sequence, head)
    constexpr int CW = 16 * NT;
    static_assert(!AFF || (NT == 1 && !SEG), "the affine pass scans 16-column groups of one sequence");
    static_assert(!PERS || (!SEG && !AFF), "the persistent scan is one pass over several sequences");
    __shared__ ScanShared<NT, LEAN> sm;
    // PERS: the team's items ((n << 16 | h, first record chunk, bos, eos),
    // (pool slot, tracked slot, tracked length, 0)), the nonempty ones first;
    // the chunk total of those; the items of sequences
    // 0 and N - 1 (a bit per item), which also write the rows outside every
    // sequence
    __shared__ int4 items[PERS ? kPersMaxItems : 1][2];
    __shared__ int item_chunks[1];
    __shared__ uint32_t edge_items[PERS ? kPersMaxItems / 32 : 1];

    const int H = a.num_heads;
    const int N = a.num_seqs;
    const int pairs = AFF ? H * (2 * s_lo - 1) : N * H;
    // XCD-aware order: the NV column groups of one (sequence, head) share an
    // XCD (and its L2), since they read the same chunk records.
    const int b = blockIdx.x;
    const int xcd = b & 7;
    const int rest = b >> 3;
    const int vt = rest % NV;
    const int pair = (rest / NV) * 8 + xcd;  // PERS: the team
    if (!PERS && pair >= pairs) {
        return;
    }
    // AFF: the chain's role (0: segment 0; 2s - 1: zero start, 2s: identity
    // start of segment s) in place of the sequence index (a single sequence)
    const int role = AFF ? pair / H : 0;
    const bool aff_zero = AFF && (role & 1) != 0;
    const bool aff_phi = AFF && role > 0 && (role & 1) == 0;
    // PERS: set per item by each role
    int n = AFF || PERS ? 0 : pair / H;
    int h = AFF ? pair - role * H : PERS ? 0 : pair - n * H;
    const Layout LY = layout(a.num_tokens, N, H, ring);
    const int *cs = reinterpret_cast<const int *>(ws + LY.chunk_start);
    int bos, eos;
    seq_bounds(a, n, bos, eos);
    // one sequence: its records start at 0 (no chunk-index pass ran)
    const int c0 = N == 1 ? 0 : cs[n];
    const int nch = N == 1 ? (eos - bos + BT - 1) / BT : cs[n + 1] - c0;
    // chunks [j0, j1) of this launch; `first` takes the state from the pool
    // (and writes the rows before the sequence), `last` stores it (and the
    // rows after); a segment past the sequence's end does nothing
    int j0 = 0;
    int j1 = nch;
    bool first = true;
    bool last = true;
    if constexpr (SEG) {
        if (s_lo >= nch && !(s_lo == 0 && nch == 0)) {
            return;
        }
        j0 = s_lo;
        j1 = s_hi < nch ? s_hi : nch;
        first = s_lo == 0;
        last = s_hi >= nch;
    }
    // AFF: the later roles start from zero or the identity and end in the
    // affine areas (fin_state), tracking into them too (trk_state); their
    // outputs are fp32 (out32); only role 0 writes the rows outside the
    // sequence
    float *fin_state = nullptr;
    float *trk_state = nullptr;
    float *out32 = nullptr;
    bool zero_outside = false;
    if constexpr (AFF) {
        const int seg = (role + 1) >> 1;
        j0 = seg * s_hi;
        j1 = j0 + s_hi < nch ? j0 + s_hi : nch;
        if (j0 >= nch && !(role == 0 && nch == 0)) {
            return;
        }
        first = role == 0;
        last = role == 0 && j1 >= nch;
        zero_outside = role == 0;
        if (role > 0) {
            const AffLayout AL = aff_layout(a.num_tokens, H, s_lo);
            char *wsm = const_cast<char *>(ws);
            const size_t st = static_cast<size_t>(H) * DK * DK * 4;
            const size_t hoff = static_cast<size_t>(h) * DK * DK;
            fin_state = reinterpret_cast<float *>(wsm + (aff_zero ? AL.fin_zero : AL.fin_phi) + st * (seg - 1)) + hoff;
            trk_state = reinterpret_cast<float *>(wsm + (aff_zero ? AL.trk_zero : AL.trk_phi)) + hoff;
            out32 = reinterpret_cast<float *>(wsm + (aff_zero ? AL.out_zero : AL.out_phi));
        }
    }
    float *carry = reinterpret_cast<float *>(const_cast<char *>(ws) + LY.carry) +
                   static_cast<size_t>(h) * DK * DK;

    // PERS: the team's item table (KA items, the first KT nonempty) and the
    // stream's length; every role derives its loop and barrier count from it
    int KT = 0;
    int KA = 0;
    if constexpr (PERS) {
        const int TM = static_cast<int>(gridDim.x) / NV;
        const int t = pair;
        const int4 *sched = reinterpret_cast<const int4 *>(ws + LY.sched);
        // items of ranks below X: all k < X / TM, and k = X / TM if its rank is
        auto count = [&](int X) {
            const int q = X / TM;
            const int off = (q & 1) ? TM - 1 - t : t;
            return q + (off < X - q * TM ? 1 : 0);
        };
        KA = count(N * H);
        KT = count(sched[2 * N].x * H);
        const int tk = static_cast<int>(threadIdx.x);
        if (tk == 0) {
            item_chunks[0] = 0;
        }
        if (tk < kPersMaxItems / 32) {
            edge_items[tk] = 0u;
        }
        __syncthreads();
        if (tk < KA) {
            const int rk = tk * TM + ((tk & 1) ? TM - 1 - t : t);
            const int4 e = sched[2 * (rk / H)];
            items[tk][0] = make_int4((e.x << 16) | (rk % H), e.y, e.z, e.w);
            items[tk][1] = sched[2 * (rk / H) + 1];
            if (tk < KT) {
                atomicAdd(&item_chunks[0], (e.w - e.z + BT - 1) / BT);
            }
            if (e.x == 0 || e.x == N - 1) {
                atomicOr(&edge_items[tk >> 5], 1u << (tk & 31));
            }
        }
        __syncthreads();
        j0 = 0;
        j1 = item_chunks[0];
    }
    // PERS: a role's position in the stream: item k (virtual chunks [base,
    // base + nch)) of sequence n and head h, its first record chunk c0 and
    // tokens [bos, eos)
    // The next item's table entries are read from LDS when an item is
    // entered (nx, and for the chain nx1) and used at the next item
    // boundary, so crossing one waits on no LDS read.
    struct Cur {
        int base, k, nch, n, h, c0, bos, eos;
        int4 nx, nx1;  // items[k + 1][0] and [1] (nx1: the chain's cursors only)
    };
    auto cur_set = [&](Cur &c, int k, const int4 e, bool with1) {
        c.k = k;
        c.n = __builtin_amdgcn_readfirstlane(e.x >> 16);
        c.h = __builtin_amdgcn_readfirstlane(e.x & 0xffff);
        c.c0 = __builtin_amdgcn_readfirstlane(e.y);
        c.bos = __builtin_amdgcn_readfirstlane(e.z);
        c.eos = __builtin_amdgcn_readfirstlane(e.w);
        c.nch = (c.eos - c.bos + BT - 1) / BT;
        const int kn = k + 1 < KA ? k + 1 : k;
        c.nx = items[kn][0];
        if (with1) {
            c.nx1 = items[kn][1];
        }
    };
    auto cur_load = [&](Cur &c, int k, bool with1 = false) { cur_set(c, k, items[k][0], with1); };
    auto cur_init = [&](Cur &c, bool with1 = false) {
        c.base = 0;
        cur_load(c, 0, with1);
    };
    // local chunk of virtual chunk J (clamped to the stream's last), moving c
    // forward (the calls at one site never go back)
    auto cur_seek = [&](Cur &c, int J) {
        J = J < j1 ? J : j1 - 1;
        while (J >= c.base + c.nch && c.k + 1 < KT) {
            c.base += c.nch;
            cur_set(c, c.k + 1, c.nx, false);
        }
        return J - c.base;
    };
    // record of virtual chunk J (chunk c's record is in slot c: one pass)
    auto cur_rec = [&](Cur &c, int J) {
        const int j = cur_seek(c, J);
        return ws + LY.recs + (static_cast<size_t>(c.c0 + j) * H + c.h) * kRecBytes;
    };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    // wave index as a scalar: the role branches below must be wave-uniform,
    // since every role meets the same workgroup barriers
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wr = w & 3;
    const int r = lane & 15;
    const int gq = lane >> 4;
    const int col0 = CW * vt;  // first value column of this group
    const f32x4 z4 = {0.f, 0.f, 0.f, 0.f};
    uint16_t *out = static_cast<uint16_t *>(a.out);
    // ring slot of chunk j: the launch's chunks are consecutive and at most a
    // ring apart from its first, so one wrap suffices past (c0 + j0) % ring
    const int slot0 = (c0 + j0) % ring;
    auto rec_of = [&](int j) {
        int sl = slot0 + (j - j0);
        sl = sl >= ring ? sl - ring : sl;
        return ws + LY.recs + (static_cast<size_t>(sl) * H + h) * kRecBytes;
    };

    if (w < 4) {
        // ------------------------------- chain waves -------------------------------
        // pool slot, tracked slot and length of sequence n, head h (PERS: of
        // the item being scanned)
        int slot = 0;
        int track_slot = 0;
        int track_len = -1;
        int64_t head_off = 0;
        auto item_ctx = [&]() {
            slot = a.state_indices[n];
            if (slot < 0 || static_cast<int64_t>(slot) >= a.num_slots) {
                slot = 0;
            }
            track_slot = 0;
            track_len = -1;
            if (a.track_indices != nullptr) {
                track_slot = a.track_indices[n];
                if (track_slot <= 0 || static_cast<int64_t>(track_slot) >= a.num_slots) {
                    track_slot = 0;
                } else {
                    track_len = a.track_lens[n];
                }
            }
            head_off = static_cast<int64_t>(h) * a.state_stride_head;
        };
        if constexpr (!PERS) {
            item_ctx();
        }
        // S rows [32wr, 32wr+32): tiles (kt = 2wr + tt, ct), lane holds
        // S[16kt + 4gq + i][col0 + 16ct + r]; the same element of slot s, and
        // of the carry buffer between segments
        auto state_ptr = [&](int s, int tt, int ct) {
            return a.state + s * a.state_stride_slot + head_off +
                   static_cast<int64_t>(col0 + 16 * ct + r) * DK + 16 * (2 * wr + tt) + 4 * gq;
        };
        auto carry_ptr = [&](int tt, int ct) {
            return carry + static_cast<int64_t>(col0 + 16 * ct + r) * DK + 16 * (2 * wr + tt) + 4 * gq;
        };
        f32x4 S[2][NT];
#pragma unroll
        for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                if (PERS) {
                    S[tt][ct] = z4;  // set per item below
                } else if (AFF && role > 0) {
                    // zero, or the identity's columns col0 + 16ct + r
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        S[tt][ct][i] = aff_phi && 16 * (2 * wr + tt) + 4 * gq + i == col0 + 16 * ct + r ? 1.f : 0.f;
                    }
                } else if (!first) {
                    const float4 s4 = load4(carry_ptr(tt, ct));
                    S[tt][ct] = f32x4{s4.x, s4.y, s4.z, s4.w};
                } else if (slot > 0) {
                    const float4 s4 = load4(state_ptr(slot, tt, ct));
                    S[tt][ct] = f32x4{s4.x, s4.y, s4.z, s4.w};
                } else {
                    S[tt][ct] = z4;
                }
            }
        }
        // Tile (tt, ct) of a later role's state into an affine area: [V][K]
        // like the pool, except the identity-start role's, whose transitions
        // go [K][V] (row k holds Phi[k][v'] for all v'), the layout the
        // combine reads them in.
        auto put_aff = [&](float *base, int tt, int ct, const f32x4 &val) {
            const int k = 16 * (2 * wr + tt) + 4 * gq;
            const int c = col0 + 16 * ct + r;
            if (aff_phi) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    base[static_cast<int64_t>(k + i) * DK + c] = val[i];
                }
            } else {
                *reinterpret_cast<float4 *>(base + static_cast<int64_t>(c) * DK + k) =
                    make_float4(val[0], val[1], val[2], val[3]);
            }
        };
        // the tracked state's tile: into the pool's track slot, or the
        // affine area of a later role
        auto put_track = [&](int tt, int ct, const f32x4 &val) {
            if (AFF && trk_state != nullptr) {
                put_aff(trk_state, tt, ct, val);
            } else {
                *reinterpret_cast<float4 *>(state_ptr(track_slot, tt, ct)) =
                    make_float4(val[0], val[1], val[2], val[3]);
            }
        };
        auto store_track = [&](const f32x4 (&val)[2][NT]) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                for (int ct = 0; ct < NT; ++ct) {
                    put_track(tt, ct, val[tt][ct]);
                }
            }
        };
        auto store_S = [&](int dst_slot, const f32x4 (&val)[2][NT]) {
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                for (int ct = 0; ct < NT; ++ct) {
                    *reinterpret_cast<float4 *>(state_ptr(dst_slot, tt, ct)) =
                        make_float4(val[tt][ct][0], val[tt][ct][1], val[tt][ct][2], val[tt][ct][3]);
                }
            }
        };
        if (!PERS && track_slot > 0 && track_len == 0 && first) {
            store_S(track_slot, S);
        }
        const char *tr = ws + LY.tracks + (static_cast<size_t>(n) * H + h) * kTrBytes;

        // Chunk j's operands are read from the stage after B1(j) (the loaders
        // write it between B2(j-1) and B1(j)): those of phase B first, then
        // those of phase C behind the first tile's S fragments. In the lean
        // form the matrix operands, e^G k (row tile wr) and (T^T kd)^T (row
        // tiles 2wr, 2wr+1), are this wave's own loads from the record, a
        // chunk ahead, into the register set chunk j-1 left.
        struct OpsG {
            f16x8 Kef[4];
            f16x8 Kd[2][2];
        };
        auto load_g = [&](OpsG &op, int j) {
            const u32x4 *rec = reinterpret_cast<const u32x4 *>(rec_of(j < j1 ? j : j1 - 1));
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                op.Kef[s] = as_f16x8(rec[(kOffKe / kFrag + wr * 4 + s) * 64 + lane]);
            }
#pragma unroll
            for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    op.Kd[tt][s] = as_f16x8(rec[(kOffKd / kFrag + (2 * wr + tt) * 2 + s) * 64 + lane]);
                }
            }
        };
        struct OpsB {
            f16x8 Kef[4];
            f32x4 vv[NT];
            float4 kesc;
            float vmax, kel1;
        };
        auto read_b = [&](OpsB &op, int p) {
            const char *st = sm.stg[p];
            const float *sc = reinterpret_cast<const float *>(st + St::kMisc) + DK;
            if constexpr (!LEAN) {
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    op.Kef[s] = stage_frag(st, wr * 4 + s, lane);
                }
            }
            // v C tiles (rows 16 wr + 4gq + i, column 16 ct + r) from the
            // row-major bf16 tile: transposing reads, then widened
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                const int g = lane >> 4;
                const int m = (lane >> 2) & 3;
                const int c4 = lane & 3;
                const uint16_t *vt_tile = reinterpret_cast<const uint16_t *>(st + St::kV);
                const s16x4 x = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                    (lds_s16x4 *)(vt_tile + (16 * wr + 4 * g + m) * CW + 16 * ct + 4 * c4));
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    op.vv[ct][i] = __uint_as_float(static_cast<uint32_t>(static_cast<uint16_t>(x[i])) << 16);
                }
            }
            const float4 um = *reinterpret_cast<const float4 *>(&sm.vmax[p][0]);
            op.vmax = max4_mag(um);
            op.kesc = *reinterpret_cast<const float4 *>(sc + kScKe + 4 * wr);
            op.kel1 = kel1_bound(sc);
        };
        // chunk j (of the item, PERS) in the stage of parity p
        auto step = [&](int j, int p, const OpsG &og, OpsG &next) {
            const int len = eos - (bos + BT * j) < BT ? eos - (bos + BT * j) : BT;
            const char *st = sm.stg[p];
            const float *sc = reinterpret_cast<const float *>(st + St::kMisc) + DK;
            if constexpr (LEAN) {
                load_g(next, j + 1);
            }

            // A. publish S_j (slice wr) as fp16 B fragments, scaled by a power
            // of two from the slice's largest magnitude (the state itself stays
            // fp32 in registers; only its products with w and q e^G use the
            // rounded copy)
            {
                float m = 0.f;
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                    for (int ct = 0; ct < NT; ++ct) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            m = fmaxf(m, fabsf(S[tt][ct][i]));
                        }
                    }
                }
                m = wave_max_mag(m);
                const int ssh = f16_shift(m);
#pragma unroll
                for (int ct = 0; ct < NT; ++ct) {
                    float x[8];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        x[i] = S[0][ct][i];
                        x[4 + i] = S[1][ct][i];
                    }
                    sm.sbuf[p][wr][ct][lane] = as_u32x4(to_f16x8(x, ssh));
                }
                if (lane == 0) {
                    sm.sscale[p][wr] = ldexpf(1.f, -ssh);
                    sm.smax[p][wr] = m;
                }
            }
            lds_barrier();  // B1(j)
            OpsB ob;
            read_b(ob, p);
            // B. y rows [16wr, 16wr+16) = v - (e^G k) S_j (one product per
            // slice, then scaled), published as fp16 hi/lo scaled by 2^sv;
            // tile wr is half wr%2 of slice wr/2. Phase C's operands of chunk
            // j are read behind the first tile's S fragments.
            const float4 sx = *reinterpret_cast<const float4 *>(&sm.smax[p][0]);
            const float4 ss = *reinterpret_cast<const float4 *>(&sm.sscale[p][0]);
            const int sv = f16_shift(ob.vmax + ob.kel1 * max4_mag(sx));
            const float inv_v = ldexpf(1.f, -sv);
            const float fw[4] = {ob.kesc.x * ss.x, ob.kesc.y * ss.y, ob.kesc.z * ss.z, ob.kesc.w * ss.w};
            f16x8 Kd[2][2];
            f32x4 gl[2];
            float2 kdsc;
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                f32x4 acc[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    acc[s] = mfma(LEAN ? og.Kef[s] : ob.Kef[s], as_f16x8(sm.sbuf[p][s][ct][lane]), z4);
                }
                if (ct == 0) {
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                        for (int s = 0; s < 2; ++s) {
                            Kd[tt][s] = LEAN ? og.Kd[tt][s] : stage_frag(st, kStKd + (2 * wr + tt) * 2 + s, lane);
                        }
                    }
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        gl[tt] = reinterpret_cast<const f32x4 *>(st + St::kMisc)[4 * (2 * wr + tt) + gq];
                    }
                    kdsc = *reinterpret_cast<const float2 *>(sc + kScKd + 2 * wr);
                }
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float x = 0.f;
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        x += fw[s] * acc[s][i];
                    }
                    v[i] = ob.vv[ct][i] - x;
                }
                uint32_t hp[2], lp[2];
                split_f16x2(v[0], v[1], sv, hp[0], lp[0]);
                split_f16x2(v[2], v[3], sv, hp[1], lp[1]);
                const int sl = wr >> 1;
                const int hf = (wr & 1) * 2;
                uint32_t *vh = reinterpret_cast<uint32_t *>(&sm.vbuf[p][sl][0][ct][lane]);
                uint32_t *vl = reinterpret_cast<uint32_t *>(&sm.vbuf[p][sl][1][ct][lane]);
                vh[hf] = hp[0];
                vh[hf + 1] = hp[1];
                vl[hf] = lp[0];
                vl[hf + 1] = lp[1];
            }
            lds_barrier();  // B2(j)
            // C. S_{j+1} = e^(G_last) S_j + (T^T kd)^T y_j (fp16 (T^T kd)^T
            // against y hi + lo, then both scales), one column tile at a time;
            // the tracked prefix strictly inside this chunk is taken from S_j
            // first.
            const int rr = track_len - BT * j;
            const bool track_in = track_slot > 0 && rr > 0 && rr < len;
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                f16x8 vh[2], vl[2];
#pragma unroll
                for (int s = 0; s < 2; ++s) {
                    vh[s] = as_f16x8(sm.vbuf[p][s][0][ct][lane]);
                    vl[s] = as_f16x8(sm.vbuf[p][s][1][ct][lane]);
                }
                if (track_in) {
                    const float *tsc = reinterpret_cast<const float *>(tr + kTrOffSc);
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
                        const f32x4 g2 = *reinterpret_cast<const f32x4 *>(
                            tr + kTrOffGl + 4 * (16 * (2 * wr + tt) + 4 * gq));
                        f32x4 tu = z4;
#pragma unroll
                        for (int s = 0; s < 2; ++s) {
                            const f16x8 th = as_f16x8(reinterpret_cast<const u32x4 *>(
                                tr + kTrOffKd)[((2 * wr + tt) * 2 + s) * 64 + lane]);
                            tu = mfma(th, vh[s], tu);
                            tu = mfma(th, vl[s], tu);
                        }
                        const float f = tsc[2 * wr + tt] * inv_v;
                        const f32x4 tv = {S[tt][ct][0] * g2[0] + tu[0] * f, S[tt][ct][1] * g2[1] + tu[1] * f,
                                          S[tt][ct][2] * g2[2] + tu[2] * f, S[tt][ct][3] * g2[3] + tu[3] * f};
                        put_track(tt, ct, tv);
                    }
                }
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    f32x4 su = z4;
#pragma unroll
                    for (int s = 0; s < 2; ++s) {
                        su = mfma(Kd[tt][s], vh[s], su);
                        su = mfma(Kd[tt][s], vl[s], su);
                    }
                    const float f = (tt == 0 ? kdsc.x : kdsc.y) * inv_v;
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        S[tt][ct][i] = S[tt][ct][i] * gl[tt][i] + su[i] * f;
                    }
                }
            }
            if (track_slot > 0 && rr == len) {
                store_track(S);
            }
        };

        OpsG gA, gB;
        if constexpr (LEAN) {
            // the initial state's loads are waited for here, not at the loop's
            // first use of S, where the wait would cover the prefetch too
            __builtin_amdgcn_s_waitcnt(kWaitVm0);
            if (j1 > j0) {
                load_g(gA, j0);
            }
        }
        if constexpr (PERS) {
            Cur cc;  // the item being scanned
            Cur cn;  // the next one, whose initial state is in Sn
            f32x4 Sn[2][NT];
            bool sn_zero = false;  // the next item has no state: Sn is a dummy load
            // the chain's context of item c: sequence, head, tokens, and the
            // slots from the table (no global loads at an item change)
            int4 cn1;  // items[cn.k][1]
            auto enter = [&](const Cur &c, const int4 e) {
                n = c.n;
                h = c.h;
                bos = c.bos;
                eos = c.eos;
                slot = __builtin_amdgcn_readfirstlane(e.x);
                track_slot = __builtin_amdgcn_readfirstlane(e.y);
                track_len = __builtin_amdgcn_readfirstlane(e.z);
                head_off = static_cast<int64_t>(h) * a.state_stride_head;
                tr = ws + LY.tracks + (static_cast<size_t>(n) * H + h) * kTrBytes;
            };
            // the next item's initial state, loaded a whole item ahead. The
            // loads are unconditional (an item without state reads the record
            // area instead and is zeroed where Sn is used), so they go straight
            // into Sn and are waited for only at the item change.
            auto prefetch = [&]() {
                if (cc.k + 1 < KT) {
                    cn.base = cc.base + cc.nch;
                    cur_set(cn, cc.k + 1, cc.nx, true);
                    cn1 = cc.nx1;
                    const int ns = __builtin_amdgcn_readfirstlane(cn1.x);
                    sn_zero = ns == 0;
                    const float *src = sn_zero ? reinterpret_cast<const float *>(ws + LY.recs)
                                               : a.state + ns * a.state_stride_slot +
                                                     static_cast<int64_t>(cn.h) * a.state_stride_head;
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                        for (int ct = 0; ct < NT; ++ct) {
                            const float4 s4 = load4(src + static_cast<int64_t>(col0 + 16 * ct + r) * DK +
                                                    16 * (2 * wr + tt) + 4 * gq);
                            Sn[tt][ct] = f32x4{s4.x, s4.y, s4.z, s4.w};
                        }
                    }
                }
            };
            if (j1 > 0) {
                cur_init(cc, true);
                enter(cc, items[0][1]);
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                    for (int ct = 0; ct < NT; ++ct) {
                        if (slot > 0) {
                            const float4 s4 = load4(state_ptr(slot, tt, ct));
                            S[tt][ct] = f32x4{s4.x, s4.y, s4.z, s4.w};
                        } else {
                            S[tt][ct] = z4;
                        }
                    }
                }
                if (track_slot > 0 && track_len == 0) {
                    store_S(track_slot, S);
                }
                // the first item's state is waited for here, so the loop's
                // steps do not wait for the prefetch behind it (that wait is
                // at the item change, where Sn is used)
                __builtin_amdgcn_s_waitcnt(kWaitVm0);
                prefetch();
            }
            lds_barrier();  // B0: the first chunk's stage is written
            // the stream: item after item, J the virtual chunk (every item has
            // at least one chunk; the loop ends after KT items)
            for (int J = 0; J < j1;) {
                for (int j = 0; j < cc.nch; ++j, ++J) {
                    step(j, J & 1, gA, gA);
                }
                // The next item's state is taken before this item's is
                // stored: a wait for the prefetch issued behind those stores
                // would wait for the stores too (the wave's memory counter is
                // in order, and the stores' branch makes it count them all).
                const bool more = cc.k + 1 < KT;
                f32x4 Sx[2][NT];
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                    for (int ct = 0; ct < NT; ++ct) {
                        Sx[tt][ct] = sn_zero || !more ? z4 : Sn[tt][ct];
                        // complete here, and the stores below stay behind
                        asm volatile("" : "+v"(Sx[tt][ct]));
                    }
                }
                if (slot > 0) {
                    store_S(slot, S);
                }
                if (!more) {
                    break;
                }
                cc = cn;
                enter(cc, cn1);
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                    for (int ct = 0; ct < NT; ++ct) {
                        S[tt][ct] = Sx[tt][ct];
                    }
                }
                if (track_slot > 0 && track_len == 0) {
                    store_S(track_slot, S);
                }
                prefetch();
            }
            if (j1 > 0) {
                lds_barrier();  // B1(j1)
            }
            // empty items keep their state; a tracked length of 0 copies it
            for (int k = KT; k < KA; ++k) {
                Cur ce;
                cur_load(ce, k);
                enter(ce, items[k][1]);
                if (track_slot > 0 && track_len == 0) {
#pragma unroll
                    for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                        for (int ct = 0; ct < NT; ++ct) {
                            if (slot > 0) {
                                const float4 s4 = load4(state_ptr(slot, tt, ct));
                                S[tt][ct] = f32x4{s4.x, s4.y, s4.z, s4.w};
                            } else {
                                S[tt][ct] = z4;
                            }
                        }
                    }
                    store_S(track_slot, S);
                }
            }
        } else {
            lds_barrier();  // B0: the first chunk's stage is written
            if constexpr (LEAN) {
                // chunk c's matrix operands are in gA when c - j0 is even, else gB
                for (int j = j0; j < j1; j += 2) {
                    step(j, j & 1, gA, gB);
                    if (j + 1 >= j1) {
                        break;
                    }
                    step(j + 1, (j + 1) & 1, gB, gA);
                }
            } else {
                for (int j = j0; j < j1; ++j) {
                    step(j, j & 1, gA, gA);
                }
            }
            if (j1 > j0) {
                lds_barrier();  // B1(j1)
            }
            if (AFF && fin_state != nullptr) {
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                    for (int ct = 0; ct < NT; ++ct) {
                        put_aff(fin_state, tt, ct, S[tt][ct]);
                    }
                }
            } else if (!last) {
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
#pragma unroll
                    for (int ct = 0; ct < NT; ++ct) {
                        *reinterpret_cast<float4 *>(carry_ptr(tt, ct)) =
                            make_float4(S[tt][ct][0], S[tt][ct][1], S[tt][ct][2], S[tt][ct][3]);
                    }
                }
            } else if (slot > 0) {
                store_S(slot, S);
            }
        }
    } else if (w < 8) {
        // ------------------------------- output waves ------------------------------
        f32x4 P[NT];  // (q e^G) S of the chunk whose output is pending
        f32x4 A[NT];  // (Aqk T) y of that chunk
#pragma unroll
        for (int ct = 0; ct < NT; ++ct) {
            P[ct] = z4;
            A[ct] = z4;
        }
        // A = (Aqk T) y_j for rows [16wr, 16wr+16): Aqk T from chunk j's
        // stage (rewritten only after B2(j+1)), y_j hi + lo from vbuf
        // (published before B2(j), rewritten after B1(j+2)), scaled as the
        // chain scaled it.
        // q e^G rows [16wr, 16wr+16) and their scales (and in the lean form
        // Aqk T rows [16wr, 16wr+16), which meet tokens >= 32 only for wr >=
        // 2), loaded by this wave one chunk ahead (two sets; indices past the
        // end clamped)
        struct OpsO {
            f16x8 Qg[4];
            f16x8 Aq[2];
            float4 qsc;
        };
        Cur cl;  // PERS: load_out's position (one chunk ahead)
        Cur co;  // PERS: finish's position (one chunk behind)
        if (PERS && j1 > 0) {
            cur_init(cl);
            cur_init(co);
        }
        auto load_out = [&](OpsO &op, int j) {
            const char *rec = PERS ? cur_rec(cl, j) : rec_of(j < j1 ? j : j1 - 1);
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                op.Qg[s] = as_f16x8(reinterpret_cast<const u32x4 *>(rec + kOffQg)[(wr * 4 + s) * 64 + lane]);
            }
            if constexpr (LEAN) {
                const u32x4 *aq = reinterpret_cast<const u32x4 *>(rec + kOffAq);
                op.Aq[0] = as_f16x8(aq[aq_frag(wr, 0) * 64 + lane]);
                op.Aq[1] = as_f16x8(aq[aq_frag(wr, wr >= 2 ? 1 : 0) * 64 + lane]);
            }
            op.qsc = *reinterpret_cast<const float4 *>(rec + kOffSc + 4 * (kScQg + 4 * wr));
        };
        auto aqk_y = [&](const OpsO &op, int j) {
            const int p = j & 1;
            const char *st = sm.stg[p];
            const float *sc = reinterpret_cast<const float *>(st + St::kMisc) + DK;
            const float4 um = *reinterpret_cast<const float4 *>(&sm.vmax[p][0]);
            const float4 sx = *reinterpret_cast<const float4 *>(&sm.smax[p][0]);
            const int sv = f16_shift(max4_mag(um) + kel1_bound(sc) * max4_mag(sx));
            const float f = sc[kScAq + wr] * ldexpf(1.f, -sv);
            // rows [16wr, 16wr+16) meet tokens >= 32 only for wr >= 2
            const f16x8 aq0 = LEAN ? op.Aq[0] : stage_frag(st, kStAq + aq_frag(wr, 0), lane);
            const f16x8 aq1 = LEAN ? op.Aq[1] : stage_frag(st, kStAq + aq_frag(wr, wr >= 2 ? 1 : 0), lane);
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                f32x4 acc = mfma(aq0, as_f16x8(sm.vbuf[p][0][0][ct][lane]), z4);
                acc = mfma(aq0, as_f16x8(sm.vbuf[p][0][1][ct][lane]), acc);
                if (wr >= 2) {
                    acc = mfma(aq1, as_f16x8(sm.vbuf[p][1][0][ct][lane]), acc);
                    acc = mfma(aq1, as_f16x8(sm.vbuf[p][1][1][ct][lane]), acc);
                }
                A[ct] = acc * f;
            }
        };
        // o_j = P + A; rows t < len of chunk j are stored, transposed through
        // this wave's LDS tile so each lane writes CW/4 consecutive columns of
        // one row (nontemporal stores).
        auto finish = [&](int j) {
            if (AFF && out32 != nullptr) {
                // a later affine role: fp32 rows, straight from the C tiles
                // (16 lanes write 64 consecutive bytes of one row)
                const int t0 = bos + BT * j;
                const int len = eos - t0 < BT ? eos - t0 : BT;
#pragma unroll
                for (int ct = 0; ct < NT; ++ct) {
                    const f32x4 acc = P[ct] + A[ct];
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int t = 16 * wr + 4 * gq + i;
                        if (t < len) {
                            out32[(static_cast<int64_t>(t0 + t) * H + h) * DK + col0 + 16 * ct + r] = acc[i];
                        }
                    }
                }
                return;
            }
            uint16_t *ot = reinterpret_cast<uint16_t *>(&sm.otile[wr][0][0]);
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                const f32x4 acc = P[ct] + A[ct];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    ot[(4 * gq + i) * CW + 16 * ct + r] = f32_to_bf16(acc[i]);
                }
            }
            int jo = j;
            int ob = bos;
            int oe = eos;
            int oh = h;
            if constexpr (PERS) {
                jo = cur_seek(co, j);
                ob = co.bos;
                oe = co.eos;
                oh = co.h;
            }
            const int t0 = ob + BT * jo;
            const int len = oe - t0 < BT ? oe - t0 : BT;
            asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
            const int row = lane >> 2;
            const int cq = lane & 3;
            const int t = 16 * wr + row;
            uint16_t *dst = out + (static_cast<int64_t>(t0 + t) * H + oh) * DK + col0 + cq * (CW / 4);
            if constexpr (NT == 1) {
                typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));
                const u32x2 val = *reinterpret_cast<const u32x2 *>(&sm.otile[wr][row][2 * cq]);
                if (t < len) {
                    __builtin_nontemporal_store(val, reinterpret_cast<u32x2 *>(dst));
                }
            } else {
                u32x4 val[NT / 2];
#pragma unroll
                for (int k = 0; k < NT / 2; ++k) {
                    val[k] = *reinterpret_cast<const u32x4 *>(&sm.otile[wr][row][(CW / 8) * cq + 4 * k]);
                }
                if (t < len) {
#pragma unroll
                    for (int k = 0; k < NT / 2; ++k) {
                        __builtin_nontemporal_store(val[k], reinterpret_cast<u32x4 *>(dst) + k);
                    }
                }
            }
        };
        // Iteration j: [B1(j)] load chunk j+1 into `other` and form A of chunk
        // j-1 (in the lean form A first: `other` holds chunk j-1's Aqk T),
        // then P = (q e^G) S_j from `cur` (fp16 q e^G against fp16 S_j,
        // one product per slice, then scaled; S_j's buffer is rewritten only
        // after B1(j+1)), [B2(j)] finish chunk j-1 (its P and A), keep P_j.
        auto iter = [&](const OpsO &cur, OpsO &other, int j) {
            const int p = j & 1;
            lds_barrier();  // B1(j)
            if constexpr (LEAN) {
                if (j > j0) {
                    aqk_y(other, j - 1);  // `other` still holds chunk j-1's Aqk T
                }
                load_out(other, j + 1);
            } else {
                load_out(other, j + 1);
                if (j > j0) {
                    aqk_y(other, j - 1);  // Aqk T from the stage
                }
            }
            f32x4 Pn[NT];
            const float4 ss = *reinterpret_cast<const float4 *>(&sm.sscale[p][0]);
            const float fq[4] = {cur.qsc.x * ss.x, cur.qsc.y * ss.y, cur.qsc.z * ss.z, cur.qsc.w * ss.w};
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                f32x4 acc[4];
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    acc[s] = mfma(cur.Qg[s], as_f16x8(sm.sbuf[p][s][ct][lane]), z4);
                }
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    float x = 0.f;
#pragma unroll
                    for (int s = 0; s < 4; ++s) {
                        x += fq[s] * acc[s][i];
                    }
                    Pn[ct][i] = x;
                }
            }
            lds_barrier();  // B2(j)
            if (j > j0) {
                finish(j - 1);
            }
#pragma unroll
            for (int ct = 0; ct < NT; ++ct) {
                P[ct] = Pn[ct];
            }
        };
        OpsO opA, opB;
        if (j1 > j0) {
            load_out(opA, j0);
        }
        lds_barrier();  // B0
        for (int j = j0; j < j1; j += 2) {
            iter(opA, opB, j);
            if (j + 1 >= j1) {
                break;
            }
            iter(opB, opA, j + 1);
        }
        if (j1 > j0) {
            lds_barrier();  // B1(j1)
            aqk_y(((j1 - 1 - j0) & 1) == 0 ? opA : opB, j1 - 1);
            finish(j1 - 1);
        }
    } else {
        // ------------------------------- loader waves ------------------------------
        // Loader wave wl carries record fragments wl, wl + 4, ... of a chunk and
        // this group's v of row tile wl in registers from their load to their
        // LDS write. Two register sets (chunks at even / odd distance from j0)
        // keep each chunk's loads in flight for a chunk and a half: chunk c is
        // loaded after B1(c-2) and written to the stage of its parity after
        // B2(c-1) (every reader of that stage's previous chunk c-2 finished
        // before B2(c-1): the chain reads a stage between B1 and B2 of its
        // chunk, the output waves its Aqk T before B2 of the next).
        constexpr int kPer = St::kLoadPer;
        const int wl = w - 8;
        u32x4 RA[kPer], RB[kPer];
        uint2 V0[NT], V1[NT], V2[NT], V3[NT];
        // Every loader wave issues the same number of loads (a surplus one
        // repeats the last fragment, which another wave also writes with the
        // same bytes), so the compiler's load counters stay exact and a write
        // waits only for its own set's loads.
        auto frag_of = [&](int k) {
            const int f = wl + 4 * k;
            return f < St::kRecFrags ? f : St::kRecFrags - 1;
        };
        const uint16_t *vp = static_cast<const uint16_t *>(a.v);
        // this group's v rows [16 wl, 16 wl + 16) of a chunk, 8 bytes (four
        // columns) per lane: load k covers rows 16 wl + k (16 / NT) + lane /
        // (4 NT), columns 4 (lane % (4 NT)); rows past the chunk's end load its
        // last row and are zeroed
        auto vrow = [&](int k) { return 16 * wl + k * (16 / NT) + lane / (4 * NT); };
        auto vcol = [&]() { return 4 * (lane % (4 * NT)); };
        Cur cf;  // PERS: fetch's position (two chunks ahead)
        Cur cv;  // PERS: fetch_v's (three ahead)
        Cur cw;  // PERS: touch's (kWarmAhead ahead)
        if (PERS && j1 > 0) {
            cur_init(cf);
            cur_init(cv);
            cur_init(cw);
        }
        auto fetch = [&](u32x4 (&R)[kPer], int j) {
            const char *rec = PERS ? cur_rec(cf, j) : rec_of(j < j1 ? j : j1 - 1);
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                R[k] = reinterpret_cast<const u32x4 *>(rec + St::src(frag_of(k)))[lane];
            }
        };
        auto fetch_v = [&](uint2 (&V)[NT], int j) {
            if (aff_phi) {  // the identity-start scan runs on v = 0
#pragma unroll
                for (int k = 0; k < NT; ++k) {
                    V[k] = make_uint2(0u, 0u);
                }
                return;
            }
            int jc = j < j1 ? j : j1 - 1;
            int vb = bos;
            int ve = eos;
            int vh = h;
            if constexpr (PERS) {
                jc = cur_seek(cv, j);
                vb = cv.bos;
                ve = cv.eos;
                vh = cv.h;
            }
            const int t0 = vb + BT * jc;
            const int len = ve - t0 < BT ? ve - t0 : BT;
#pragma unroll
            for (int k = 0; k < NT; ++k) {
                const int row = vrow(k);
                const int tc = row < len ? row : len - 1;
                V[k] = *reinterpret_cast<const uint2 *>(vp + (static_cast<int64_t>(t0 + tc) * H + vh) * DK + col0 +
                                                        vcol());
                const uint32_t keep = keep_mask(row < len);
                V[k].x &= keep;
                V[k].y &= keep;
            }
        };
        auto put = [&](const u32x4 (&R)[kPer], const uint2 (&V)[NT], int par) {
#pragma unroll
            for (int k = 0; k < kPer; ++k) {
                reinterpret_cast<u32x4 *>(sm.stg[par] + St::dst(frag_of(k)))[lane] = R[k];
            }
            uint16_t *vt_tile = reinterpret_cast<uint16_t *>(sm.stg[par] + St::kV);
            uint32_t m = 0;  // largest |v| as bf16 bits (order-preserving for magnitudes)
#pragma unroll
            for (int k = 0; k < NT; ++k) {
                *reinterpret_cast<uint2 *>(vt_tile + vrow(k) * CW + vcol()) = V[k];
                m = max(m, max(max(V[k].x & 0x7fffu, (V[k].x >> 16) & 0x7fffu),
                               max(V[k].y & 0x7fffu, (V[k].y >> 16) & 0x7fffu)));
            }
            const float mf = wave_max_mag(__uint_as_float(m << 16));
            if (lane == 0) {
                sm.vmax[par][wl] = mf;
            }
        };
        // L2 warm-up: at chunk j each workgroup reads one dword of each line of
        // its 1/NV share of chunk j + kWarmAhead's record, so the record is in
        // L2 before the column groups load it. Each value is folded in two
        // chunks later, when the loads issued after it have been waited for.
        constexpr int kWarmAhead = 4;
        constexpr int kLines = kRecBytes / 128;
        constexpr int kShare = (kLines + NV - 1) / NV;
        constexpr int kTouch = (kShare + 255) / 256;  // lines per loader lane
        uint32_t warm = 0, wa[kTouch], wb[kTouch];
#pragma unroll
        for (int k = 0; k < kTouch; ++k) {
            wa[k] = 0;
            wb[k] = 0;
        }
        auto touch = [&](uint32_t (&dst)[kTouch], int jj) {
            const char *rec = PERS ? cur_rec(cw, jj) : rec_of(jj < j1 ? jj : j1 - 1);
#pragma unroll
            for (int k = 0; k < kTouch; ++k) {
                warm ^= dst[k];
                int i = k * 256 + wl * 64 + lane;
                i = i < kShare ? i : kShare - 1;
                int l = vt * kShare + i;
                l = l < kLines - 1 ? l : kLines - 1;
                dst[k] = *reinterpret_cast<const uint32_t *>(rec + l * 128);
            }
        };
        // Chunk j+2's record fragments are loaded after B1(j) into the set
        // chunk j left (written after B2(j-1)), and chunk j+3's v into the
        // one of four v sets chunk j-1 left (v, read straight from the input,
        // gets the longer head start); chunk j+1 goes into the stage of its
        // parity after B2(j). Indices past the end are clamped to the last
        // chunk: the extra copies land in a stage no one reads again, and
        // every wait count on the loop's path stays exact.
        auto iter = [&](u32x4 (&Rload)[kPer], const u32x4 (&Rput)[kPer], uint2 (&Vload)[NT],
                        const uint2 (&Vput)[NT], uint32_t (&dst)[kTouch], int j) {
            lds_barrier();  // B1(j)
            fetch(Rload, j + 2);
            fetch_v(Vload, j + 3);
            touch(dst, j + kWarmAhead);
            lds_barrier();  // B2(j)
            put(Rput, Vput, (j + 1) & 1);
        };
        if (j1 > j0) {
            fetch(RA, j0);
            fetch_v(V0, j0);
            fetch_v(V1, j0 + 1);
            fetch_v(V2, j0 + 2);
            put(RA, V0, j0 & 1);
            fetch(RB, j0 + 1);
        }
        lds_barrier();  // B0
        // chunk c's record fragments are in RA when c - j0 is even, else RB;
        // its v in V0..V3 by (c - j0) % 4
        for (int j = j0; j < j1; j += 4) {
            iter(RA, RB, V3, V1, wa, j);
            if (j + 1 >= j1) {
                break;
            }
            iter(RB, RA, V0, V2, wb, j + 1);
            if (j + 2 >= j1) {
                break;
            }
            iter(RA, RB, V1, V3, wa, j + 2);
            if (j + 3 >= j1) {
                break;
            }
            iter(RB, RA, V2, V0, wb, j + 3);
        }
        if (j1 > j0) {
            lds_barrier();  // B1(j1)
        }
#pragma unroll
        for (int k = 0; k < kTouch; ++k) {
            warm ^= wa[k] ^ wb[k];
        }
        // keeps the warm-up loads (never true: num_tokens >= 0)
        if (warm == 0x9e3779b9u && a.num_tokens < 0) {
            out[0] = 0;
        }
    }

    // Tokens outside every sequence are written as zero.
    auto zero_rows = [&](int ta, int tb, int hh) {
        for (int t = ta + tid / 16; t < tb; t += kScanThreads / 16) {
            if ((tid & 15) == 0) {
                // one thread per token row writes this group's CW columns
                for (int cidx = 0; cidx < CW; ++cidx) {
                    out[(static_cast<int64_t>(t) * H + hh) * DK + col0 + cidx] = 0;
                }
            }
        }
    };
    if constexpr (PERS) {
        // the team's items of sequences 0 and N - 1 (bits set with the table)
        for (int word = 0; word < (KA + 31) / 32; ++word) {
            uint32_t bits = edge_items[word];
            while (bits != 0u) {
                const int k = 32 * word + __builtin_ctz(bits);
                bits &= bits - 1u;
                Cur ce;
                cur_load(ce, k);
                if (ce.n == 0) {
                    zero_rows(0, ce.bos, ce.h);
                }
                if (ce.n == N - 1) {
                    zero_rows(ce.eos, a.num_tokens, ce.h);
                }
            }
        }
    } else {
        if (n == 0 && first) {
            zero_rows(0, bos, h);
        }
        if (n == N - 1 && (last || zero_outside)) {
            zero_rows(eos, a.num_tokens, h);
        }
    }
}

// ---------------------------------------------------------------------------
// The affine form of one long sequence on few heads: chunk_scan_kernel<1,
// false, true> scans segment 0 from the pool and every later segment s
// twice from its start (from zero with the real v: outputs o', final state
// Z_s; from the identity with v = 0: outputs O, final state Phi_s). With
// S_s the true state at segment s's start,
//     S_{s+1} = Phi_s S_s + Z_s,     o_t = o'_t + O_t S_s   (t in segment s),
// since the recurrence and the readout are linear in (state, v). The first
// is a short serial pass over the segments (this kernel); the second a
// parallel product over the later segments' chunks (the next one). The
// chains of the first pass fill the CUs a few-head sequence leaves idle.
// ---------------------------------------------------------------------------

constexpr int kAffThreads = 256;

// One workgroup per (head, 16 value columns), four waves: S_{s+1} = Phi_s
// S_s + Z_s for s = 1 .. P-1 (S_1 is segment 0's final state, the carry
// area), each S_s kept for the correction of segment s's outputs, the
// tracked state when the tracked length ends inside a later segment (its two
// tracked scan states combined the same way), and the final state into the
// pool. The products run on the fp32 MFMA (v_mfma_f32_16x16x4f32, lane (r, g)
// supplying A[r][g] and B[g][r] of each 4-wide K step, C as for the bf16
// tiles) with the K index v' permuted: at step kk lane (r, g) supplies v' =
// 32 g + kk, so its A values are 32 consecutive entries of a row of Phi
// (stored [k][v'] by the identity-start scan) and its B values 32
// consecutive entries of a column of S_s ([v'][k], the pool's layout). Every
// wave holds all of S_s as B operands; wave w forms rows [32w, 32w + 32) of
// S_{s+1}, and the new columns pass to the next step through LDS.
__global__ __launch_bounds__(kAffThreads) void chunk_affine_combine_kernel(const KdaChunkArgs a, char *ws,
                                                                         int P, int W) {
    __shared__ float sb[2][16][DK + 4];  // S_{s+1} by step parity: [column][k], rows padded
    const int H = a.num_heads;
    const int h = blockIdx.x >> 3;
    const int g = blockIdx.x & 7;
    if (h >= H) {
        return;
    }
    int bos, eos;
    seq_bounds(a, 0, bos, eos);
    const int nch = (eos - bos + BT - 1) / BT;
    if (nch <= W) {
        return;  // segment 0 held the whole sequence and finished it
    }
    int slot = a.state_indices[0];
    if (slot < 0 || static_cast<int64_t>(slot) >= a.num_slots) {
        slot = 0;
    }
    int track_slot = 0;
    int track_len = -1;
    if (a.track_indices != nullptr) {
        track_slot = a.track_indices[0];
        if (track_slot <= 0 || static_cast<int64_t>(track_slot) >= a.num_slots) {
            track_slot = 0;
        } else {
            track_len = a.track_lens[0];
        }
    }
    const Layout LY = layout(a.num_tokens, 1, H);
    const AffLayout AL = aff_layout(a.num_tokens, H, P);
    const size_t st = static_cast<size_t>(H) * DK * DK * 4;
    const size_t hoff = static_cast<size_t>(h) * DK * DK;
    auto area = [&](size_t off, int s) { return reinterpret_cast<float *>(ws + off + st * s) + hoff; };
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int r = lane & 15;
    const int gq = lane >> 4;
    const int col = 16 * g + r;  // this lane's column of S (B and C operands)
    // S_s as B operands: bv[i][e] = S_s[32 gq + 4 i + e][col]; S_1 from the
    // carry area ([V][K])
    float4 bv[8];
    const float *carry = reinterpret_cast<const float *>(ws + LY.carry) + hoff;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        bv[i] = load4(carry + static_cast<int64_t>(col) * DK + 32 * gq + 4 * i);
    }
    // A operands of this wave's two row tiles t: Phi[16 (2w + t) + r][32 gq + 4 i + e];
    // C initial values: Z[16 (2w + t) + 4 gq + e][col]
    struct Ops {
        float4 A[2][8];
        f32x4 Z[2];
    };
    auto fetch = [&](Ops &op, const float *M, const float *Z) {
#pragma unroll
        for (int t = 0; t < 2; ++t) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                op.A[t][i] = load4(M + static_cast<int64_t>(16 * (2 * w + t) + r) * DK + 32 * gq + 4 * i);
            }
        }
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            const float4 z = load4(Z + static_cast<int64_t>(col) * DK + 16 * (2 * w + t) + 4 * gq);
            op.Z[t] = f32x4{z.x, z.y, z.z, z.w};
        }
    };
    // out[t] = Z tile t + (Phi S_s) tile t: 32 K steps per tile, the two
    // tiles' chains interleaved
    auto product = [&](const Ops &op, f32x4 (&out)[2]) {
        out[0] = op.Z[0];
        out[1] = op.Z[1];
#pragma unroll
        for (int i = 0; i < 8; ++i) {
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                out[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(op.A[t][i].x, bv[i].x, out[t], 0, 0, 0);
                out[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(op.A[t][i].y, bv[i].y, out[t], 0, 0, 0);
                out[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(op.A[t][i].z, bv[i].z, out[t], 0, 0, 0);
                out[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(op.A[t][i].w, bv[i].w, out[t], 0, 0, 0);
            }
        }
    };
    const int64_t head_off = static_cast<int64_t>(h) * a.state_stride_head;
    // this wave's quarter of a state held as B operands (rows 32 gq + 4 i,
    // i = 2 (w & 3) .. +1), into [V][K] at `dst`
    auto store_b = [&](float *dst) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            if ((i >> 1) == w) {
                *reinterpret_cast<float4 *>(dst + static_cast<int64_t>(col) * DK + 32 * gq + 4 * i) = bv[i];
            }
        }
    };
    // one step: S_s kept, the tracked state if it ends in segment s, the
    // next transition's loads issued into `nxt`, then S_{s+1} into bv
    auto step = [&](int s, const Ops &cur, Ops &nxt) {
        store_b(area(AL.start, s - 1));
        const int seg_end = (s + 1) * W < nch ? BT * (s + 1) * W : eos - bos;
        if (track_slot > 0 && track_len > BT * s * W && track_len <= seg_end) {
            Ops tr;
            fetch(tr, reinterpret_cast<const float *>(ws + AL.trk_phi) + hoff,
                  reinterpret_cast<const float *>(ws + AL.trk_zero) + hoff);
            f32x4 tv[2];
            product(tr, tv);
            float *pool = a.state + track_slot * a.state_stride_slot + head_off;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                *reinterpret_cast<float4 *>(pool + static_cast<int64_t>(col) * DK + 16 * (2 * w + t) + 4 * gq) =
                    make_float4(tv[t][0], tv[t][1], tv[t][2], tv[t][3]);
            }
        }
        if (s + 1 < P && (s + 1) * W < nch) {
            fetch(nxt, area(AL.fin_phi, s), area(AL.fin_zero, s));
        }
        f32x4 out[2];
        product(cur, out);
        float(*buf)[DK + 4] = sb[s & 1];
#pragma unroll
        for (int t = 0; t < 2; ++t) {
            *reinterpret_cast<float4 *>(&buf[r][16 * (2 * w + t) + 4 * gq]) =
                make_float4(out[t][0], out[t][1], out[t][2], out[t][3]);
        }
        // one barrier per step: the buffer this step wrote is rewritten two
        // steps later, after every wave has passed the next step's barrier
        __syncthreads();
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            bv[i] = *reinterpret_cast<const float4 *>(&buf[r][32 * gq + 4 * i]);
        }
    };
    Ops oa, ob;
    fetch(oa, area(AL.fin_phi, 0), area(AL.fin_zero, 0));
    for (int s = 1; s < P && s * W < nch; s += 2) {
        step(s, oa, ob);
        if (s + 1 >= P || (s + 1) * W >= nch) {
            break;
        }
        step(s + 1, ob, oa);
    }
    if (slot > 0) {
        store_b(a.state + slot * a.state_stride_slot + head_off);
    }
}

// Chunks per correction workgroup (they share the staged S_s).
constexpr int kAffCorrectChunks = 4;

// One workgroup per (later segment s, head, kAffCorrectChunks of the
// segment's chunks): o_t = bf16(o'_t + O_t S_s). S_s is staged once as bf16
// hi + lo B fragments (64 KiB), each 16-row tile of O is split likewise, and
// the product takes three passes (hi hi, hi lo, lo hi: about 2^-16 relative
// per term). Wave w takes token rows [16w, 16w + 16) of each chunk.
__global__ __launch_bounds__(kAffThreads) void chunk_affine_correct_kernel(const KdaChunkArgs a, char *ws, int P,
                                                                         int W) {
    __shared__ u32x4 sb[4][8][2][64];  // S_s B fragments: [K slice][column tile][hi, lo][lane]
    const int H = a.num_heads;
    const int groups = (W + kAffCorrectChunks - 1) / kAffCorrectChunks;
    const int s = 1 + static_cast<int>(blockIdx.x) / (groups * H);
    const int rest = static_cast<int>(blockIdx.x) % (groups * H);
    const int h = rest % H;
    const int c_lo = s * W + (rest / H) * kAffCorrectChunks;
    int bos, eos;
    seq_bounds(a, 0, bos, eos);
    const int nch = (eos - bos + BT - 1) / BT;
    const int seg_hi = (s + 1) * W < nch ? (s + 1) * W : nch;
    if (s >= P || c_lo >= seg_hi) {
        return;
    }
    const int c_hi = c_lo + kAffCorrectChunks < seg_hi ? c_lo + kAffCorrectChunks : seg_hi;
    const AffLayout AL = aff_layout(a.num_tokens, H, P);
    const float *S = reinterpret_cast<const float *>(ws + AL.start + static_cast<size_t>(H) * DK * DK * 4 * (s - 1)) +
                     static_cast<size_t>(h) * DK * DK;
    const float *O = reinterpret_cast<const float *>(ws + AL.out_phi);
    const float *Oz = reinterpret_cast<const float *>(ws + AL.out_zero);
    uint16_t *out = static_cast<uint16_t *>(a.out);
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int w = tid >> 6;
    const int r = lane & 15;
    const int gq = lane >> 4;
    // S_s as B fragments: lane (r, gq) of fragment (slice sl, tile nt) holds
    // S[k = 32 sl + kperm(gq, e)][v = 16 nt + r]; S is [V][K], so each half
    // of the eight is one float4 run of K
    for (int f = w; f < 32; f += 4) {
        const int sl = f & 3;
        const int nt = f >> 2;
        const float *col = S + static_cast<int64_t>(16 * nt + r) * DK + 32 * sl + 4 * gq;
        const float4 x0 = *reinterpret_cast<const float4 *>(col);
        const float4 x1 = *reinterpret_cast<const float4 *>(col + 16);
        const float x[8] = {x0.x, x0.y, x0.z, x0.w, x1.x, x1.y, x1.z, x1.w};
        bf16x8 hi, lo;
        split_bf16x8(x, hi, lo);
        sb[sl][nt][0][lane] = as_u32x4(hi);
        sb[sl][nt][1][lane] = as_u32x4(lo);
    }
    __syncthreads();
    for (int c = c_lo; c < c_hi; ++c) {
        const int t0 = bos + BT * c;
        const int len = eos - t0 < BT ? eos - t0 : BT;
        // A: row 16 w + r of O (rows past the chunk's end read its last row;
        // their results are not stored)
        const int ta = 16 * w + r < len ? 16 * w + r : len - 1;
        const float *orow = O + (static_cast<int64_t>(t0 + ta) * H + h) * DK;
        float4 ox[4][2];
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
            ox[sl][0] = *reinterpret_cast<const float4 *>(orow + 32 * sl + 4 * gq);
            ox[sl][1] = *reinterpret_cast<const float4 *>(orow + 32 * sl + 16 + 4 * gq);
        }
        // o' of this lane's outputs, loaded before the products need them
        // (rows past the chunk's end read its last row)
        float oz[8][4];
#pragma unroll
        for (int nt = 0; nt < 8; ++nt) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * w + 4 * gq + i < len ? 16 * w + 4 * gq + i : len - 1;
                oz[nt][i] = Oz[(static_cast<int64_t>(t0 + t) * H + h) * DK + 16 * nt + r];
            }
        }
        bf16x8 ah[4], al[4];
#pragma unroll
        for (int sl = 0; sl < 4; ++sl) {
            const float x[8] = {ox[sl][0].x, ox[sl][0].y, ox[sl][0].z, ox[sl][0].w,
                                ox[sl][1].x, ox[sl][1].y, ox[sl][1].z, ox[sl][1].w};
            split_bf16x8(x, ah[sl], al[sl]);
        }
#pragma unroll 2
        for (int nt = 0; nt < 8; ++nt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int sl = 0; sl < 4; ++sl) {
                const bf16x8 bh = as_bf16x8(sb[sl][nt][0][lane]);
                const bf16x8 bl = as_bf16x8(sb[sl][nt][1][lane]);
                acc = mfma(ah[sl], bh, acc);
                acc = mfma(ah[sl], bl, acc);
                acc = mfma(al[sl], bh, acc);
            }
            // lane (r, gq) holds C[4 gq + i][r]: token 16 w + 4 gq + i, column 16 nt + r
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int t = 16 * w + 4 * gq + i;
                if (t < len) {
                    out[(static_cast<int64_t>(t0 + t) * H + h) * DK + 16 * nt + r] = f32_to_bf16(oz[nt][i] + acc[i]);
                }
            }
        }
    }
}

bool aligned(const void *p, uintptr_t m) { return (reinterpret_cast<uintptr_t>(p) & (m - 1)) == 0; }

// Compute units of the device `stream` runs on, queried once per device.
int device_cus(hipStream_t stream) {
    static std::atomic<int> cache[64];
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) {
        (void)hipGetLastError();  // leave no error behind for the caller's own checks
        if (hipGetDevice(&dev) != hipSuccess) {
            return 256;
        }
    }
    if (dev < 0 || dev >= 64) {
        return 256;
    }
    int n = cache[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
            n = 256;
        }
        cache[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Value tiles per scan workgroup for `pairs` (sequence, head) chains: the
// narrow groups have the shorter chunk step, the wide ones read half the
// operand bytes per column, so the narrow ones win while all of them run at
// once (pairs x 8 <= CUs), the wide ones as soon as the narrow ones would need
// a second round.
int scan_tiles(int64_t pairs, hipStream_t stream) { return pairs * 8 <= device_cus(stream) ? 1 : 2; }

const void *scan_kernel_affine() { return reinterpret_cast<const void *>(chunk_scan_kernel<1, false, true>); }

const void *scan_kernel(int nt, bool seg) {
    if (nt == 2) {
        return seg ? reinterpret_cast<const void *>(chunk_scan_kernel<2, true>)
                   : reinterpret_cast<const void *>(chunk_scan_kernel<2, false>);
    }
    return seg ? reinterpret_cast<const void *>(chunk_scan_kernel<1, true>)
               : reinterpret_cast<const void *>(chunk_scan_kernel<1, false>);
}

// 8 / nt workgroups per (sequence, head), pairs padded to a multiple of eight
// for the XCD-aware numbering.
int64_t scan_blocks(int64_t pairs, int nt) { return (pairs + 7) / 8 * 8 * (8 / nt); }

// A second stream (default priority) and four events per device, created on
// first use and kept for the process: the segmented prefill runs K1 of
// segment s+1 on the stream while the scan of segment s runs on the caller's
// (`done1[s&1]` after each K1, waited for by the scan; `done2[s&1]` recorded
// on the caller's stream just before each scan, waited for by the next K1).
// `order` is held across one call's sequence, so calls from several host
// threads cannot interleave their records and waits.
struct SideStream {
    hipStream_t stream = nullptr;
    hipEvent_t done1[2] = {nullptr, nullptr};
    hipEvent_t done2[2] = {nullptr, nullptr};
    std::mutex *order = nullptr;
};

// Returns false (the caller then runs the single-pass form) when the stream
// of `main`'s device does not exist yet and `main` is being captured into a
// graph: streams and events are never created during a capture.
bool side_stream(hipStream_t main, SideStream &out) {
    static std::mutex mu;
    static std::mutex orders[64];
    static SideStream streams[64];
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(main, &dev) != hipSuccess) {
        (void)hipGetLastError();
        if (hipGetDevice(&dev) != hipSuccess) {
            return false;
        }
    }
    if (dev < 0 || dev >= 64) {
        return false;
    }
    std::lock_guard<std::mutex> lock(mu);
    SideStream &ss = streams[dev];
    if (ss.stream == nullptr) {
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(main, &cap) != hipSuccess || cap != hipStreamCaptureStatusNone) {
            (void)hipGetLastError();
            return false;
        }
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess) {
            return false;
        }
        SideStream fresh;
        bool ok = hipSetDevice(dev) == hipSuccess &&
                  hipStreamCreateWithFlags(&fresh.stream, hipStreamNonBlocking) == hipSuccess;
        for (int i = 0; i < 2 && ok; ++i) {
            ok = hipEventCreateWithFlags(&fresh.done1[i], hipEventDisableTiming) == hipSuccess &&
                 hipEventCreateWithFlags(&fresh.done2[i], hipEventDisableTiming) == hipSuccess;
        }
        (void)hipSetDevice(cur);
        if (!ok) {
            (void)hipGetLastError();
            return false;
        }
        fresh.order = &orders[dev];
        ss = fresh;
    }
    out = ss;
    return true;
}

// Single sequences at least this long on at most this many heads (their
// 16-column scan fills at most half of a 256-CU device) run in segments of W
// chunks: K1 of segment s+1 overlaps the scan of segment s on the CUs the
// scan leaves idle, and the records live in a ring of 2W slots per head
// instead of one slot per chunk. Each segment boundary costs the two streams'
// event hand-offs (measured 10-20 µs), so segments hold about kSegmentChunks
// chunks, at least two segments (65536 tokens on 16 heads, 1024 chunks: 8
// segments 1473 µs, 6 1471, 4 1444, two of 47% / 53% 1516; 16384 tokens on 8
// heads: 2 segments 314 µs, 4 324, 8 385).
constexpr int kSplitMinTokens = 16384;
constexpr int kSplitMaxHeads = 16;
constexpr int kSegmentChunks = 256;

bool windowed_shape(int T, int N, int H) { return N == 1 && T >= kSplitMinTokens && H <= kSplitMaxHeads; }

int chunk_bound(int T) { return (T + BT - 1) / BT; }  // chunks of one sequence of T tokens

int segment_count(int T) {
    const int segs = (chunk_bound(T) + kSegmentChunks - 1) / kSegmentChunks;
    return segs < 2 ? 2 : segs;
}
// The first segment runs its K1 alone on the device; with two segments it
// holds 47% of the chunks (the best of 35-62% measured), otherwise its share.
int first_segment(int T) {
    const int nch = chunk_bound(T);
    const int segs = segment_count(T);
    return segs == 2 ? (nch * 47 + 50) / 100 : (nch + segs - 1) / segs;
}
// The longest segment: the ring holds two of them per head.
int window_chunks(int T) {
    const int nch = chunk_bound(T);
    const int first = first_segment(T);
    const int segs = segment_count(T);
    return segs == 2 ? nch - first : first;
}

// The affine form of a single sequence (see chunk_affine_combine_kernel):
// its first pass runs 8 (2P - 1) H scan workgroups, each on a CU of its own,
// so it applies while at least two segments fit the device, with segments of
// at least kAffMinChunks chunks (the combine's serial steps and the extra
// launches cost a few microseconds each). Returns P (0: not applicable) and
// the segment length W in chunks.
// Its workspace keeps every record and two fp32 outputs per token, so it is
// taken only while that stays within kAffMaxBytes (at 4 heads about 130,000
// tokens); longer sequences keep the pipelined segments.
// Two segments pay only when they are long (measured: 8 heads x 16384
// tokens 287 against 314 us for the pipelined scan, x 8192 141 against 161;
// 4 x 4096, two segments of 32 chunks, 86 against 79 us one-pass), so P = 2
// needs kAffMinChunksTwo chunks per segment.
constexpr int kAffMinChunks = 32;
constexpr int kAffMinChunksTwo = 64;
constexpr size_t kAffMaxBytes = size_t{1} << 30;

int affine_segments(int T, int H, int cus, int &W) {
    const int nch = chunk_bound(T);
    int P = 0;
    for (int p = 2; 8 * H * (2 * p - 1) <= cus; ++p) {
        if ((nch + p - 1) / p < kAffMinChunks) {
            break;
        }
        P = p;
    }
    if (P < 2 || (P == 2 && (nch + 1) / 2 < kAffMinChunksTwo) || aff_layout(T, H, P).total > kAffMaxBytes) {
        P = 0;
    }
    W = P > 0 ? (nch + P - 1) / P : 0;
    return P;
}

// The workspace a call needs: the affine form's areas for a single sequence
// that takes it, the ring of 2W slots for the segmented shape, one slot per
// chunk otherwise.
size_t classic_bytes(int T, int N, int H) {
    return windowed_shape(T, N, H) ? layout(T, 1, H, 2 * window_chunks(T)).total : layout(T, N, H).total;
}
size_t required_bytes(int T, int N, int H, int cus) {
    int W = 0;
    const int P = N == 1 ? affine_segments(T, H, cus, W) : 0;
    return P > 0 ? aff_layout(T, H, P).total : classic_bytes(T, N, H);
}

// The largest window (segments run one after another, so a ring of W slots)
// whose layout fits `bytes` for one sequence, or 0.
int fit_window(int T, int H, size_t bytes) {
    const Layout base = layout(T, 1, H, 0);
    if (base.total > bytes) {
        return 0;
    }
    const size_t per = static_cast<size_t>(kRecBytes) * H;
    const size_t w = (bytes - base.total) / per;
    const int cap = chunk_bound(T) > 0 ? chunk_bound(T) : 1;
    return w > static_cast<size_t>(cap) ? cap : static_cast<int>(w);
}

}  // namespace chunk
}  // namespace kda

extern "C" size_t kda_chunk_workspace_bytes(int32_t num_tokens, int32_t num_seqs,
                                            int32_t num_heads, int32_t head_dim) {
    if (num_tokens < 0 || num_seqs < 0 || num_heads <= 0 || head_dim != kda::chunk::DK) {
        return 0;
    }
    return kda::chunk::required_bytes(num_tokens, num_seqs, num_heads, kda::chunk::device_cus(nullptr));
}

namespace kda {
namespace chunk {

// Argument checks shared by both chunk entry points (no device access).
int check_args(const KdaChunkArgs *args) {
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
    if (a.qk_dtype != KDA_BF16 || a.v_dtype != KDA_BF16 ||
        (a.gate_mode != KDA_GATE_RAW && a.gate_mode != KDA_GATE_LOG)) {
        return KDA_ERR_UNSUPPORTED;
    }
    if (!aligned(a.state, 16) || (a.state_stride_slot & 3) || (a.state_stride_head & 3) ||
        !aligned(a.q, 8) || !aligned(a.k, 8) || !aligned(a.v, 8) || !aligned(a.out, 8) ||
        !aligned(a.gate, a.gate_mode == KDA_GATE_RAW ? 8 : 16)) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    return KDA_OK;
}

// Enqueues the chunk kernels on `st` with `ws` (checked by the caller) as the
// workspace. `win` = 0: one pass, a record slot per chunk. `win` > 0 (one
// sequence only): segments of `win` chunks (the first of `first_seg`, when
// given, at most `win`) with records in a ring of `ring` slots per head; with
// `pipeline` (ring = 2 win) K1 of segment s+1 runs on the library's side
// stream while segment s is scanned, otherwise (ring >= win) the segments run
// one after another on `st`.
int launch(const KdaChunkArgs &a, char *ws, hipStream_t st, int ring, int win, bool pipeline, int first_seg = 0) {
    KdaChunkArgs kargs = a;
    const int nrec = max_chunks(a.num_tokens, a.num_seqs);
    const int64_t pairs = static_cast<int64_t>(a.num_seqs) * a.num_heads;
    const int nt = scan_tiles(pairs, st);
    const int64_t blocks = scan_blocks(pairs, nt);
    if (static_cast<int64_t>(nrec) * a.num_heads > 0x7fffffff || blocks > 0x7fffffff) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    // The persistent scan (see chunk_scan_kernel): one pass over several
    // sequences with 32-column groups and more (sequence, head) items than
    // teams of workgroups, one workgroup per CU, at most kPersMaxItems items
    // per team.
    const int group = 8 * (8 / nt);
    const int64_t teams = device_cus(st) / group * 8;
    const bool pers = win <= 0 && nt == 2 && a.num_seqs > 1 && a.num_seqs <= kPersMaxSeqs && teams > 0 &&
                      pairs > teams && pairs <= kPersMaxItems * teams;
    if (a.num_seqs > 1) {  // one sequence needs no chunk index (K1 and K2 derive it)
        const Layout LY = layout(a.num_tokens, a.num_seqs, a.num_heads, ring);
        int *cs = reinterpret_cast<int *>(ws + LY.chunk_start);
        int4 *sched = reinterpret_cast<int4 *>(ws + LY.sched);
        int sort = pers ? 1 : 0;
        void *params[] = {&kargs, &cs, &sched, &sort};
        if (hipLaunchKernel(reinterpret_cast<const void *>(chunk_index_kernel), dim3(1), dim3(1024),
                            params, 0, st) != hipSuccess) {
            return KDA_ERR_LAUNCH;
        }
    }
    const void *prep = a.gate_mode == KDA_GATE_RAW
                           ? reinterpret_cast<const void *>(chunk_prepare_kernel<KDA_GATE_RAW>)
                           : reinterpret_cast<const void *>(chunk_prepare_kernel<KDA_GATE_LOG>);
    // K1 over chunks [lo, hi)
    auto launch_prep = [&](int lo, int hi, hipStream_t s) {
        if (hi <= lo) {
            return true;
        }
        int rg = ring, l = lo, h = hi, sw = 0;
        void *params[] = {&kargs, &ws, &rg, &l, &h, &sw};
        return hipLaunchKernel(prep, dim3(static_cast<unsigned>(static_cast<int64_t>(hi - lo) * a.num_heads)),
                               dim3(kThreads), params, 0, s) == hipSuccess;
    };
    // K2 over all chunks (seg false) or the segment [lo, hi)
    auto launch_scan = [&](bool seg, int lo, int hi) {
        const char *cws = ws;
        int rg = ring, l = lo, h = hi;
        void *params[] = {&kargs, &cws, &rg, &l, &h};
        return hipLaunchKernel(scan_kernel(nt, seg), dim3(static_cast<unsigned>(blocks)), dim3(kScanThreads),
                               params, 0, st) == hipSuccess;
    };
    if (win <= 0) {
        if (pers) {
            const char *cws = ws;
            int rg = ring, l = 0, h = 0;
            void *params[] = {&kargs, &cws, &rg, &l, &h};
            return launch_prep(0, nrec, st) &&
                           hipLaunchKernel(reinterpret_cast<const void *>(chunk_scan_kernel<2, false, false, true>),
                                           dim3(static_cast<unsigned>(teams * (8 / nt))), dim3(kScanThreads), params,
                                           0, st) == hipSuccess
                       ? KDA_OK
                       : KDA_ERR_LAUNCH;
        }
        return launch_prep(0, nrec, st) && launch_scan(false, 0, 0) ? KDA_OK : KDA_ERR_LAUNCH;
    }
    // one sequence; segments cover the chunks T tokens can hold (a shorter
    // sequence leaves its trailing segments empty: their workgroups return).
    // The first segment holds `first` chunks, the others `win`.
    const int nch_max = chunk_bound(a.num_tokens);
    const int first = first_seg > 0 ? first_seg : win;
    const int nseg = nch_max <= first ? 1 : 1 + (nch_max - first + win - 1) / win;
    auto seg_lo = [&](int s) { return s == 0 ? 0 : first + (s - 1) * win; };
    auto seg_hi = [&](int s) { return first + s * win < nch_max ? first + s * win : nch_max; };
    SideStream side;
    if (pipeline && nt == 1 && ring >= 2 * win && side_stream(st, side)) {
        // st:   K1(0) | [wait done1(s)] go(s) K2(s) ...
        // side:        [wait go(s)] K1(s+1) done1(s+1) ...
        // K1(s+1) is released together with the scan of segment s (go(s) is
        // recorded just before it), never earlier: a scan workgroup needs a
        // CU of its own, and K1 workgroups released ahead of the scan would
        // fill every CU first. go(s) follows K2(s-1) on st, so the ring half
        // K1(s+1) rewrites has been read. A side stream that another thread's
        // graph capture has pulled in is not used.
        std::lock_guard<std::mutex> lock(*side.order);
        hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(side.stream, &cap) == hipSuccess && cap == hipStreamCaptureStatusNone) {
            if (!launch_prep(seg_lo(0), seg_hi(0), st)) {
                return KDA_ERR_LAUNCH;
            }
            for (int s = 0; s < nseg; ++s) {
                hipEvent_t go = side.done2[s & 1];
                if (s >= 1 && hipStreamWaitEvent(st, side.done1[s & 1], 0) != hipSuccess) {
                    return KDA_ERR_LAUNCH;
                }
                if (s + 1 < nseg &&
                    (hipEventRecord(go, st) != hipSuccess || hipStreamWaitEvent(side.stream, go, 0) != hipSuccess ||
                     !launch_prep(seg_lo(s + 1), seg_hi(s + 1), side.stream) ||
                     hipEventRecord(side.done1[(s + 1) & 1], side.stream) != hipSuccess)) {
                    return KDA_ERR_LAUNCH;
                }
                if (!launch_scan(true, seg_lo(s), seg_hi(s))) {
                    return KDA_ERR_LAUNCH;
                }
            }
            return KDA_OK;
        }
        (void)hipGetLastError();
    }
    for (int s = 0; s < nseg; ++s) {
        if (!launch_prep(seg_lo(s), seg_hi(s), st) || !launch_scan(true, seg_lo(s), seg_hi(s))) {
            return KDA_ERR_LAUNCH;
        }
    }
    return KDA_OK;
}

// The affine form of one sequence, all on `st`: K1 over every chunk, the
// first pass (segment 0 from the pool, the later segments from zero and from
// the identity), the serial combine, the parallel correction of the later
// segments' outputs.
int launch_affine(const KdaChunkArgs &a, char *ws, hipStream_t st, int P, int W) {
    KdaChunkArgs kargs = a;
    const int H = a.num_heads;
    const int nrec = max_chunks(a.num_tokens, 1);
    const int nch_max = chunk_bound(a.num_tokens);
    const int64_t blocks = scan_blocks(static_cast<int64_t>(H) * (2 * P - 1), 1);
    if (static_cast<int64_t>(nrec) * H > 0x7fffffff || blocks > 0x7fffffff) {
        return KDA_ERR_INVALID_ARGUMENT;
    }
    const void *prep = a.gate_mode == KDA_GATE_RAW
                           ? reinterpret_cast<const void *>(chunk_prepare_kernel<KDA_GATE_RAW>)
                           : reinterpret_cast<const void *>(chunk_prepare_kernel<KDA_GATE_LOG>);
    // every chunk, numbered in segments of W chunks (P W >= nrec - 1 >= the chunks)
    int ring = nrec, lo = 0, hi = nch_max, order = W;
    void *pparams[] = {&kargs, &ws, &ring, &lo, &hi, &order};
    if (hipLaunchKernel(prep, dim3(static_cast<unsigned>(static_cast<int64_t>(P) * W * H)), dim3(kThreads), pparams,
                        0, st) != hipSuccess) {
        return KDA_ERR_LAUNCH;
    }
    const char *cws = ws;
    int sp = P, sw = W;
    void *sparams[] = {&kargs, &cws, &ring, &sp, &sw};
    if (hipLaunchKernel(scan_kernel_affine(), dim3(static_cast<unsigned>(blocks)), dim3(kScanThreads), sparams, 0,
                        st) != hipSuccess) {
        return KDA_ERR_LAUNCH;
    }
    void *cparams[] = {&kargs, &ws, &sp, &sw};
    if (hipLaunchKernel(reinterpret_cast<const void *>(chunk_affine_combine_kernel), dim3(static_cast<unsigned>(8 * H)),
                        dim3(kAffThreads), cparams, 0, st) != hipSuccess) {
        return KDA_ERR_LAUNCH;
    }
    const int64_t later = static_cast<int64_t>(P - 1) * ((W + kAffCorrectChunks - 1) / kAffCorrectChunks) * H;
    if (nch_max > W && later > 0 &&
        hipLaunchKernel(reinterpret_cast<const void *>(chunk_affine_correct_kernel), dim3(static_cast<unsigned>(later)),
                        dim3(kAffThreads), cparams, 0, st) != hipSuccess) {
        return KDA_ERR_LAUNCH;
    }
    return KDA_OK;
}

// The no-allocation entry point's scratch: one array per device, held until
// the process ends. Host code never uses the array's name as an address: the
// device address is resolved once per device with hipGetSymbolAddress (that
// device current) and kept here.
static __device__ __align__(256) char scratch[KDA_NOALLOC_SCRATCH_BYTES];

// The device address of `scratch` on the device `st` runs on, or null.
char *scratch_address(hipStream_t st) {
    static std::mutex mu;
    static char *addr[64] = {};
    hipDevice_t dev = 0;
    if (hipStreamGetDevice(st, &dev) != hipSuccess) {
        (void)hipGetLastError();
        if (hipGetDevice(&dev) != hipSuccess) {
            return nullptr;
        }
    }
    if (dev < 0 || dev >= 64) {
        return nullptr;
    }
    std::lock_guard<std::mutex> lock(mu);
    if (addr[dev] == nullptr) {
        int cur = 0;
        if (hipGetDevice(&cur) != hipSuccess) {
            return nullptr;
        }
        void *ptr = nullptr;
        const bool ok = hipSetDevice(dev) == hipSuccess &&
                        hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch)) == hipSuccess && ptr != nullptr;
        (void)hipSetDevice(cur);
        if (!ok) {
            (void)hipGetLastError();
            return nullptr;
        }
        addr[dev] = static_cast<char *>(ptr);
    }
    return addr[dev];
}

}  // namespace chunk
}  // namespace kda

extern "C" int kda_chunk_launch(const KdaChunkArgs *args, void *workspace, size_t workspace_bytes,
                                void *stream) {
    using namespace kda::chunk;
    const int rc = check_args(args);
    if (rc != KDA_OK || args->num_seqs == 0) {
        return rc;
    }
    const KdaChunkArgs &a = *args;
    if (workspace == nullptr || !aligned(workspace, 256)) {
        return KDA_ERR_WORKSPACE;
    }
    char *ws = static_cast<char *>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int T = a.num_tokens;
    const int H = a.num_heads;
    if (a.num_seqs == 1) {
        int W = 0;
        const int P = affine_segments(T, H, device_cus(st), W);
        if (P > 0 && workspace_bytes >= aff_layout(T, H, P).total) {
            return launch_affine(a, ws, st, P, W);
        }
    }
    if (workspace_bytes >= classic_bytes(T, a.num_seqs, H)) {
        if (windowed_shape(T, a.num_seqs, H)) {
            const int w = window_chunks(T);
            return launch(a, ws, st, 2 * w, w, true, first_segment(T));
        }
        return launch(a, ws, st, max_chunks(T, a.num_seqs), 0, false);
    }
    // a smaller workspace: one sequence in segments that fit it
    if (a.num_seqs == 1) {
        const int w = fit_window(T, H, workspace_bytes);
        if (w > 0) {
            return launch(a, ws, st, w, w, false);
        }
    }
    return KDA_ERR_WORKSPACE;
}

extern "C" int kda_chunk_launch_noalloc(const KdaChunkArgs *args, void *stream) {
    using namespace kda::chunk;
    const int rc = check_args(args);
    if (rc != KDA_OK || args->num_seqs == 0) {
        return rc;
    }
    const KdaChunkArgs &a = *args;
    const int T = a.num_tokens;
    const int H = a.num_heads;
    const bool whole = layout(T, a.num_seqs, H).total <= KDA_NOALLOC_SCRATCH_BYTES;
    const int w = whole || a.num_seqs != 1 ? 0 : fit_window(T, H, KDA_NOALLOC_SCRATCH_BYTES);
    if (!whole && w == 0) {
        return KDA_ERR_TOO_LARGE;
    }
    hipStream_t st = static_cast<hipStream_t>(stream);
    char *ws = scratch_address(st);
    if (ws == nullptr) {
        return KDA_ERR_LAUNCH;
    }
    return whole ? launch(a, ws, st, max_chunks(T, a.num_seqs), 0, false) : launch(a, ws, st, w, w, false);
}
