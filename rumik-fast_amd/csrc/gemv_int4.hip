// Batch-1 int4 group-128 GEMV for gfx950: y[n] = sum_g scale[n,g] * sum_{k in g} code[n,k] x[k] + min[n,g] * sum_{k in g} x[k]
// (the affine identity of the reference, kernels/int4_gemv.py:1-4; CUDA version kernels/cuda_gemv.py:38-115).
//
// Design (bandwidth-bound; one pass over the weights):
//   * A "team" of KS waves owns R rows. Thread t of the team (t < 64*KS) owns the 32-column chunks
//     c = t + j*64*KS (j < NJ). Each chunk of one row is one 16-byte load (global_load_dwordx4, non-temporal), so
//     a wave instruction streams 1 KiB of codes of one row: fully coalesced 128-byte lines.
//   * x is staged once per wave, in registers: the 32 values of each owned chunk as 16 fp16 pairs in the order
//     (x0,x4),(x1,x5),(x2,x6),(x3,x7) per 8 columns, plus their fp32 sum. It is reused for all R rows.
//   * Dequant in registers, exact: (w & 0x000F000F) | 0x64006400 is the fp16 pair (1024 + c0, 1024 + c4) (fp16
//     1024.0 = 0x6400 has a mantissa LSB worth 1); a packed fp16 add of -1024 leaves (c0, c4) exactly. The high
//     nibbles give 1024 + 16c, brought back to c by one exact packed fma (x 1/16, -64); the same for w >> 8.
//     v_dot2_f32_f16 multiplies each code pair with the matching x pair and accumulates in fp32, so every product
//     is exact and only the fp32 sums round (13 VALU ops per 8 weights).
//   * Per (row, chunk): acc += scale * dot + min * xsum, in fp32.
//   * Rows are reduced over the wave with a transposed butterfly (R + 6 exchanges for R rows, DPP inside 16-lane
//     rows), then over the KS waves of a team through LDS.
#include "internal.h"
#include "dequant.h"

namespace {

constexpr int kMaxThreads = 1024;

// Dot of one 16-byte code chunk (32 codes) with its x pairs.
RK_DEV float chunk_dot(u4_t w, const uint32_t (&xp)[16]) {
    const h2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    const h2_t s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2_t m64 = {(_Float16)-64.f, (_Float16)-64.f};
    float acc0 = 0.f, acc1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = w[i], b = a >> 8;
        h2_t c04 = as_h2((a & 0x000F000Fu) | 0x64006400u) + m1024;
        h2_t c15 = as_h2((a & 0x00F000F0u) | 0x64006400u) * s16 + m64;
        h2_t c26 = as_h2((b & 0x000F000Fu) | 0x64006400u) + m1024;
        h2_t c37 = as_h2((b & 0x00F000F0u) | 0x64006400u) * s16 + m64;
        acc0 = dot2(c04, as_h2(xp[4 * i + 0]), acc0);
        acc1 = dot2(c15, as_h2(xp[4 * i + 1]), acc1);
        acc0 = dot2(c26, as_h2(xp[4 * i + 2]), acc0);
        acc1 = dot2(c37, as_h2(xp[4 * i + 3]), acc1);
    }
    return acc0 + acc1;
}

// the GEMV of block `blk` (rows [blk * teams * R, ...)); `red`: LDS for the KS-way reduction
template <int R, int KS, int NJ>
RK_DEV void gemv_int4_block(const void* __restrict__ x, int xdt, const uint8_t* __restrict__ q,
                            const uint16_t* __restrict__ sc, const uint16_t* __restrict__ mn, void* __restrict__ y,
                            int ydt, int N, int K, int blk, float (*red)[R]) {
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int team = wave / KS;
    const int kw = wave - team * KS;
    const int teams = blockDim.x / (64 * KS);
    const int t = kw * 64 + lane;
    const int nch = K >> 5;
    const int ng = K >> 7;
    const int row0 = (blk * teams + team) * R;  // teams past N (last block only) clamp and store nothing

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;

    // K is walked in passes of 64*KS*NJ chunks (one pass whenever the plan allows it)
    for (int c0 = 0; c0 < nch; c0 += 64 * KS * NJ) {
        // ---- loads, in the order they are consumed: x (from L2), the scales / mins, then R rows x NJ chunks of
        // codes. Every load is unconditional (chunks past K re-read the last chunk, rows past N the last row) so the
        // compiler can wait for each one alone; the duplicates meet zeroed x and add nothing.
        XChunk xc[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) load_x_raw(x, min(c0 + t + j * 64 * KS, nch - 1), xc[j]);
        uint16_t s16[R][NJ], m16[R][NJ];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, N - 1);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int c = min(c0 + t + j * 64 * KS, nch - 1);
                const size_t gi = (size_t)row * ng + (c >> 2);
                s16[r][j] = sc[gi];
                m16[r][j] = mn[gi];
            }
        }
        u4_t w[R][NJ];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, N - 1);  // rows past N re-read the last row; their result is dropped
            const u4_t* qr = reinterpret_cast<const u4_t*>(q + (size_t)row * (size_t)(K >> 1));
#pragma unroll
            for (int j = 0; j < NJ; ++j) w[r][j] = __builtin_nontemporal_load(qr + min(c0 + t + j * 64 * KS, nch - 1));
        }

        // ---- x chunks as dequant-ordered pairs (zero past K)
        uint32_t xp[NJ][16];
        float xs[NJ];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            process_x_chunk(xc[j], xdt, xp[j], xs[j]);
            if (c0 + t + j * 64 * KS >= nch) {
#pragma unroll
                for (int e = 0; e < 16; ++e) xp[j][e] = 0u;
                xs[j] = 0.f;
            }
        }

        // ---- dequant + dot + group affine
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float a = acc[r];
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const float d = chunk_dot(w[r][j], xp[j]);
                const float sv = f16_bits_to_f32(s16[r][j]);
                const float mv = f16_bits_to_f32(m16[r][j]);
                a = __builtin_fmaf(d, sv, __builtin_fmaf(mv, xs[j], a));
            }
            acc[r] = a;
        }
    }

    // ---- reduce over the wave, then over the KS waves of the team
    wave_reduce_rows<R>(acc);
    const bool writer = (lane & (64 / R - 1)) == 0;
    const int rr = row_of_lane<R>(lane);
    if constexpr (KS == 1) {
        if (writer && row0 + rr < N) store_act(y, ydt, (size_t)(row0 + rr), acc[0]);
    } else {
        if (writer) red[wave][rr] = acc[0];
        __syncthreads();
        if (kw == 0 && lane < R && row0 + lane < N) {
            float v = 0.f;
#pragma unroll
            for (int k = 0; k < KS; ++k) v += red[team * KS + k][lane];
            store_act(y, ydt, (size_t)(row0 + lane), v);
        }
    }
}

template <int R, int KS, int NJ>
__global__ __launch_bounds__(kMaxThreads) void gemv_int4_kernel(const void* __restrict__ x, int xdt,
                                                                const uint8_t* __restrict__ q,
                                                                const uint16_t* __restrict__ sc,
                                                                const uint16_t* __restrict__ mn,
                                                                void* __restrict__ y, int ydt, int N, int K) {
    __shared__ float red[kMaxThreads / 64][R];
    gemv_int4_block<R, KS, NJ>(x, xdt, q, sc, mn, y, ydt, N, K, blockIdx.x, red);
}

// Two independent GEMVs in one launch (blocks [0, nb1) the first, the rest the second), each with its own plan;
// both run with the same block size. One launch instead of two saves a launch gap and one ramp / drain of the
// memory stream (the o and down projections of a layer both wait only on the attention and the MLP activation).
struct GemvArgs {
    const void* x;
    const uint8_t* q;
    const uint16_t *s, *m;
    void* y;
    int N, K, xdt, ydt;
};

template <int R1, int KS1, int NJ1, int R2, int KS2, int NJ2>
__global__ __launch_bounds__(kMaxThreads) void gemv_int4_pair_kernel(GemvArgs a, GemvArgs b, int nb1) {
    __shared__ float red1[kMaxThreads / 64][R1];
    __shared__ float red2[kMaxThreads / 64][R2];
    if ((int)blockIdx.x < nb1)
        gemv_int4_block<R1, KS1, NJ1>(a.x, a.xdt, a.q, a.s, a.m, a.y, a.ydt, a.N, a.K, blockIdx.x, red1);
    else
        gemv_int4_block<R2, KS2, NJ2>(b.x, b.xdt, b.q, b.s, b.m, b.y, b.ydt, b.N, b.K, blockIdx.x - nb1, red2);
}

template <int R, int KS, int NJ>
hipError_t launch(const void* x, int xdt, const uint8_t* q, const uint16_t* s, const uint16_t* m, void* y, int ydt,
                  int N, int K, int waves, hipStream_t st) {
    const int teams = waves / KS;
    const int rows_per_block = teams * R;
    const int blocks = (N + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((gemv_int4_kernel<R, KS, NJ>), dim3(blocks), dim3(waves * 64), 0, st, x, xdt, q, s, m,
                       y, ydt, N, K);
    return hipGetLastError();
}

template <int R, int KS>
hipError_t by_nj(int nj, const void* x, int xdt, const uint8_t* q, const uint16_t* s, const uint16_t* m, void* y,
                 int ydt, int N, int K, int waves, hipStream_t st) {
    switch (nj) {
        case 1: return launch<R, KS, 1>(x, xdt, q, s, m, y, ydt, N, K, waves, st);
        case 2: return launch<R, KS, 2>(x, xdt, q, s, m, y, ydt, N, K, waves, st);
        case 3: return launch<R, KS, 3>(x, xdt, q, s, m, y, ydt, N, K, waves, st);
        case 4: return launch<R, KS, 4>(x, xdt, q, s, m, y, ydt, N, K, waves, st);
        default: return hipErrorInvalidValue;
    }
}

template <int R>
hipError_t by_ks(int ks, int nj, const void* x, int xdt, const uint8_t* q, const uint16_t* s, const uint16_t* m,
                 void* y, int ydt, int N, int K, int waves, hipStream_t st) {
    switch (ks) {
        case 1: return by_nj<R, 1>(nj, x, xdt, q, s, m, y, ydt, N, K, waves, st);
        case 2: return by_nj<R, 2>(nj, x, xdt, q, s, m, y, ydt, N, K, waves, st);
        case 4: return by_nj<R, 4>(nj, x, xdt, q, s, m, y, ydt, N, K, waves, st);
        case 8: return by_nj<R, 8>(nj, x, xdt, q, s, m, y, ydt, N, K, waves, st);
        default: return hipErrorInvalidValue;
    }
}

}  // namespace

// Launch plan for one call (host side). Returns RK_OK or RK_ERR_BLOCK / RK_ERR_SHAPE.
struct Int4Plan {
    int waves, rows, ks, nj;
};

static int plan_int4(int N, int K, int waves, int rows, Int4Plan* p) {
    const int nch = K / 32;
    // tuned defaults (hipGraph-timed on MI355X, weights rotated past the MALL): short rows (K <= 4096) one wave per
    // row set, 4 waves per block, 4 rows per wave once N >= 3072 (qkv 3072 x 2048: 3.45 us) and 2 below, so the
    // 2048-row o projection still fills 256 blocks (3.08 us vs 3.36 with 4 rows); long rows (down, K = 11008) 2 waves
    // of 2 rows splitting K in two (5.79 us vs 6.25 with 4 waves)
    int w = waves ? waves : (nch <= 128 ? 4 : 2);
    int r = rows ? rows : (nch <= 128 ? (N >= 3072 ? 4 : 2) : 2);
    if (!(w == 1 || w == 2 || w == 4 || w == 8 || w == 16)) return RK_ERR_BLOCK;
    if (!(r == 1 || r == 2 || r == 4 || r == 8)) return RK_ERR_BLOCK;
    int ks = nch <= 128 ? 1 : 4;
    while (ks < 8 && (nch + 64 * ks - 1) / (64 * ks) > 4) ks *= 2;
    if (ks > w) ks = w;  // a small explicit block splits K over all of its waves
    int nj = (nch + 64 * ks - 1) / (64 * ks);
    if (nj > 4) nj = 4;  // longer rows take several passes over K
    p->waves = w;
    p->rows = r;
    p->ks = ks;
    p->nj = nj;
    return RK_OK;
}

int gemv_int4_valu_launch(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                          const uint16_t* min, void* y, int y_dtype, int N, int K, int waves, int rows,
                          rk_stream_t stream) {
    if (!x || !q || !scale || !min || !y) return RK_ERR_NULL;
    if (N <= 0 || K <= 0 || K % 128 != 0) return RK_ERR_SHAPE;
    if (x_dtype != RK_F16 && x_dtype != RK_BF16) return RK_ERR_DTYPE;
    if (y_dtype != RK_F16 && y_dtype != RK_BF16 && y_dtype != RK_F32) return RK_ERR_DTYPE;
    if (((uintptr_t)x & 15) || ((uintptr_t)q & 15)) return RK_ERR_ALIGN;
    Int4Plan p;
    int st = plan_int4(N, K, waves, rows, &p);
    if (st != RK_OK) return st;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t e;
    switch (p.rows) {
        case 1: e = by_ks<1>(p.ks, p.nj, x, x_dtype, q, scale, min, y, y_dtype, N, K, p.waves, s); break;
        case 2: e = by_ks<2>(p.ks, p.nj, x, x_dtype, q, scale, min, y, y_dtype, N, K, p.waves, s); break;
        case 4: e = by_ks<4>(p.ks, p.nj, x, x_dtype, q, scale, min, y, y_dtype, N, K, p.waves, s); break;
        default: e = by_ks<8>(p.ks, p.nj, x, x_dtype, q, scale, min, y, y_dtype, N, K, p.waves, s); break;
    }
    return e == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

// o-like (K <= 4096: 4 waves x 2 rows, one pass) + down-like (K <= 16384: 4 waves = 2 teams of 2 splitting K, 2 rows
// each) in one launch; other shapes run as two launches of the single-GEMV plans.
int gemv_int4_pair_launch(const void* x1, int x1_dtype, const uint8_t* q1, const uint16_t* s1,
                          const uint16_t* m1, void* y1, int y1_dtype, int N1, int K1, const void* x2,
                          int x2_dtype, const uint8_t* q2, const uint16_t* s2, const uint16_t* m2, void* y2,
                          int y2_dtype, int N2, int K2, rk_stream_t stream) {
    if (!x1 || !q1 || !s1 || !m1 || !y1 || !x2 || !q2 || !s2 || !m2 || !y2) return RK_ERR_NULL;
    if (N1 <= 0 || K1 <= 0 || K1 % 128 || N2 <= 0 || K2 <= 0 || K2 % 128) return RK_ERR_SHAPE;
    for (int dt : {x1_dtype, x2_dtype})
        if (dt != RK_F16 && dt != RK_BF16) return RK_ERR_DTYPE;
    for (int dt : {y1_dtype, y2_dtype})
        if (dt != RK_F16 && dt != RK_BF16 && dt != RK_F32) return RK_ERR_DTYPE;
    if (((uintptr_t)x1 | (uintptr_t)q1 | (uintptr_t)x2 | (uintptr_t)q2) & 15) return RK_ERR_ALIGN;
    const int nch1 = K1 / 32, nch2 = K2 / 32;
    if (nch1 <= 64 && nch2 > 128 && nch2 <= 512) {
        const GemvArgs a{x1, q1, s1, m1, y1, N1, K1, x1_dtype, y1_dtype};
        const GemvArgs b{x2, q2, s2, m2, y2, N2, K2, x2_dtype, y2_dtype};
        const int nb1 = (N1 + 7) / 8;   // 4 teams of 2 rows
        const int nb2 = (N2 + 3) / 4;   // 2 teams of 2 rows
        hipStream_t st = reinterpret_cast<hipStream_t>(stream);
        if (nch2 <= 384)
            hipLaunchKernelGGL((gemv_int4_pair_kernel<2, 1, 1, 2, 2, 3>), dim3(nb1 + nb2), dim3(256), 0, st, a, b, nb1);
        else
            hipLaunchKernelGGL((gemv_int4_pair_kernel<2, 1, 1, 2, 2, 4>), dim3(nb1 + nb2), dim3(256), 0, st, a, b, nb1);
        return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
    }
    int e = gemv_int4_valu_launch(x1, x1_dtype, q1, s1, m1, y1, y1_dtype, N1, K1, 0, 0, stream);
    if (e != RK_OK) return e;
    return gemv_int4_valu_launch(x2, x2_dtype, q2, s2, m2, y2, y2_dtype, N2, K2, 0, 0, stream);
}
