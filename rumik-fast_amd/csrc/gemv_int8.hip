// Batch-1 int8 GEMV with one scale per row (the audio head): y[n] = scale[n] * sum_k code[n,k] * x[k]
// (reference kernels/cuda_gemv.py:138-195; weights there are uint8 = int8 + 128 with an fp32 scale).
//
// Same structure as the int4 GEMV: a team of KS waves owns R rows, thread t owns the 16-column chunks
// c = t + j*64*KS, one 16-byte non-temporal load per (row, chunk); x is held in registers as natural fp16 pairs.
// Dequant, exact: v_perm_b32 places each byte u under 0x64 -> fp16 (1024 + u); a packed add of -1152 gives
// u - 128, the signed code (signed int8 input is first mapped to u = b ^ 0x80). Products and sums in fp32 via
// v_dot2_f32_f16; the row scale is applied once after the wave reduction.
#include "internal.h"

namespace {

constexpr int kMaxThreads = 1024;

RK_DEV void load_x16(const void* __restrict__ x, int xdt, int c, uint32_t (&xp)[8]) {
    const u4_t* xv = reinterpret_cast<const u4_t*>(x) + (size_t)c * 2;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        u4_t d = xv[i];
        if (xdt == RK_BF16) {
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t v = d[e];
                h2_t p;
                p.x = (_Float16)__builtin_bit_cast(float, v << 16);
                p.y = (_Float16)__builtin_bit_cast(float, v & 0xffff0000u);
                xp[4 * i + e] = as_u32(p);
            }
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) xp[4 * i + e] = d[e];
        }
    }
}

template <bool SIGNED>
RK_DEV float chunk_dot8(u4_t w, const uint32_t (&xp)[8]) {
    const h2_t m1152 = {(_Float16)-1152.f, (_Float16)-1152.f};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t v = w[i];
        if constexpr (SIGNED) v ^= 0x80808080u;
        h2_t c01 = as_h2(perm(0x64646464u, v, 0x04010400u)) + m1152;  // (code0, code1)
        h2_t c23 = as_h2(perm(0x64646464u, v, 0x04030402u)) + m1152;  // (code2, code3)
        a0 = dot2(c01, as_h2(xp[2 * i]), a0);
        a1 = dot2(c23, as_h2(xp[2 * i + 1]), a1);
    }
    return a0 + a1;
}

template <int R, int KS, int NJ, bool SIGNED>
__global__ __launch_bounds__(kMaxThreads) void gemv_int8_kernel(const void* __restrict__ x, int xdt,
                                                                const uint8_t* __restrict__ q,
                                                                const void* __restrict__ sc, int sdt,
                                                                void* __restrict__ y, int ydt, int N, int K) {
    __shared__ float red[kMaxThreads / 64][R];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int team = wave / KS;
    const int kw = wave - team * KS;
    const int teams = blockDim.x / (64 * KS);
    const int t = kw * 64 + lane;
    const int nch = K >> 4;
    const int row0 = (blockIdx.x * teams + team) * R;

    float acc[R];
#pragma unroll
    for (int r = 0; r < R; ++r) acc[r] = 0.f;
    for (int c0 = 0; c0 < nch; c0 += 64 * KS * NJ) {  // passes over K (one whenever the plan allows it)
        u4_t w[R][NJ];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int row = min(row0 + r, N - 1);
            const u4_t* qr = reinterpret_cast<const u4_t*>(q + (size_t)row * (size_t)K);
#pragma unroll
            for (int j = 0; j < NJ; ++j) {
                const int c = c0 + t + j * 64 * KS;
                if (c < nch) w[r][j] = __builtin_nontemporal_load(qr + c);
                else w[r][j] = u4_t{0u, 0u, 0u, 0u};
            }
        }
        uint32_t xp[NJ][8];
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
            const int c = c0 + t + j * 64 * KS;
            if (c < nch) {
                load_x16(x, xdt, c, xp[j]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) xp[j][e] = 0u;
            }
        }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float a = acc[r];
#pragma unroll
            for (int j = 0; j < NJ; ++j) a += chunk_dot8<SIGNED>(w[r][j], xp[j]);
            acc[r] = a;
        }
    }
    wave_reduce_rows<R>(acc);
    const bool writer = (lane & (64 / R - 1)) == 0;
    const int rr = row_of_lane<R>(lane);
    auto finish = [&](int row, float v) {
        const float s = sdt == RK_F32 ? reinterpret_cast<const float*>(sc)[row]
                                      : f16_bits_to_f32(reinterpret_cast<const uint16_t*>(sc)[row]);
        store_act(y, ydt, (size_t)row, v * s);
    };
    if constexpr (KS == 1) {
        if (writer && row0 + rr < N) finish(row0 + rr, acc[0]);
    } else {
        if (writer) red[wave][rr] = acc[0];
        __syncthreads();
        if (kw == 0 && lane < R && row0 + lane < N) {
            float v = 0.f;
#pragma unroll
            for (int k = 0; k < KS; ++k) v += red[team * KS + k][lane];
            finish(row0 + lane, v);
        }
    }
}

template <int R, int KS, int NJ, bool SIGNED>
hipError_t launch8(const void* x, int xdt, const uint8_t* q, const void* s, int sdt, void* y, int ydt, int N, int K,
                   int waves, hipStream_t st) {
    const int teams = waves / KS;
    const int rows_per_block = teams * R;
    const int blocks = (N + rows_per_block - 1) / rows_per_block;
    hipLaunchKernelGGL((gemv_int8_kernel<R, KS, NJ, SIGNED>), dim3(blocks), dim3(waves * 64), 0, st, x, xdt, q, s,
                       sdt, y, ydt, N, K);
    return hipGetLastError();
}

template <int R, int KS, bool SIGNED>
hipError_t by_nj8(int nj, const void* x, int xdt, const uint8_t* q, const void* s, int sdt, void* y, int ydt, int N,
                  int K, int waves, hipStream_t st) {
    switch (nj) {
        case 1: return launch8<R, KS, 1, SIGNED>(x, xdt, q, s, sdt, y, ydt, N, K, waves, st);
        case 2: return launch8<R, KS, 2, SIGNED>(x, xdt, q, s, sdt, y, ydt, N, K, waves, st);
        case 3: return launch8<R, KS, 3, SIGNED>(x, xdt, q, s, sdt, y, ydt, N, K, waves, st);
        case 4: return launch8<R, KS, 4, SIGNED>(x, xdt, q, s, sdt, y, ydt, N, K, waves, st);
        default: return hipErrorInvalidValue;
    }
}

template <bool SIGNED>
hipError_t by_plan8(int rows, int ks, int nj, const void* x, int xdt, const uint8_t* q, const void* s, int sdt,
                    void* y, int ydt, int N, int K, int waves, hipStream_t st) {
#define RK_CASE(RR, KK) \
    if (rows == RR && ks == KK) return by_nj8<RR, KK, SIGNED>(nj, x, xdt, q, s, sdt, y, ydt, N, K, waves, st);
    RK_CASE(1, 1) RK_CASE(2, 1) RK_CASE(4, 1) RK_CASE(8, 1)
    RK_CASE(1, 2) RK_CASE(2, 2) RK_CASE(4, 2) RK_CASE(8, 2)
    RK_CASE(1, 4) RK_CASE(2, 4) RK_CASE(4, 4) RK_CASE(8, 4)
    RK_CASE(1, 8) RK_CASE(2, 8) RK_CASE(4, 8) RK_CASE(8, 8)
#undef RK_CASE
    return hipErrorNotSupported;
}

}  // namespace

int gemv_int8_rows_launch(const void* x, int x_dtype, const void* q, int q_kind, const void* scale,
                          int s_dtype, void* y, int y_dtype, int N, int K, int waves, int rows, rk_stream_t stream) {
    if (!x || !q || !scale || !y) return RK_ERR_NULL;
    if (N <= 0 || K <= 0 || K % 16 != 0) return RK_ERR_SHAPE;
    if (x_dtype != RK_F16 && x_dtype != RK_BF16) return RK_ERR_DTYPE;
    if (s_dtype != RK_F16 && s_dtype != RK_F32) return RK_ERR_DTYPE;
    if (y_dtype != RK_F16 && y_dtype != RK_BF16 && y_dtype != RK_F32) return RK_ERR_DTYPE;
    if (q_kind != RK_Q_S8 && q_kind != RK_Q_U8) return RK_ERR_DTYPE;
    if (((uintptr_t)x & 15) || ((uintptr_t)q & 15)) return RK_ERR_ALIGN;
    const int nch = K / 16;
    int w = waves ? waves : 4;
    int r = rows ? rows : (nch <= 256 ? 2 : 1);
    if (!(w == 1 || w == 2 || w == 4 || w == 8 || w == 16)) return RK_ERR_BLOCK;
    if (!(r == 1 || r == 2 || r == 4 || r == 8)) return RK_ERR_BLOCK;
    int ks = nch <= 256 ? 1 : 4;
    while (ks < 8 && (nch + 64 * ks - 1) / (64 * ks) > 4) ks *= 2;
    if (ks > w) ks = w;
    int nj = (nch + 64 * ks - 1) / (64 * ks);
    if (nj > 4) nj = 4;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t e = q_kind == RK_Q_S8
                       ? by_plan8<true>(r, ks, nj, x, x_dtype, (const uint8_t*)q, scale, s_dtype, y, y_dtype, N, K, w, s)
                       : by_plan8<false>(r, ks, nj, x, x_dtype, (const uint8_t*)q, scale, s_dtype, y, y_dtype, N, K, w, s);
    if (e == hipErrorNotSupported) return RK_ERR_BLOCK;
    return e == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
