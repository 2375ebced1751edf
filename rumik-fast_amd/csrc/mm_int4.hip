// int4 group-128 matrix product for the prefill on gfx950 matrix cores:
//   Y[m,n] = sum_g ( scale[n,g] * sum_{k in g} X[m,k] code[n,k] + min[n,g] * sum_{k in g} X[m,k] )
// (reference kernels/mm_int4.py:24-46: per group, a tensor-core product on the raw codes plus the group affine).
//
// Tiling: a block of 4 waves (2 x 2) owns a (2*WM*16) x (2*WN*16) tile of Y; a wave owns WM x WN MFMA tiles of
// 16 x 16 (v_mfma_f32_16x16x32_f16: A[i][k] lane i+16*(k/8) element k%8, B[k][j] lane j+16*(k/8), D[i][j] lane
// j+16*(i/4) element i%4). Lane l = (j = l%16, s = l/16):
//   * B (codes): lane loads 16 bytes of W row n0+j at byte 64g + 16s -> 4 dwords = the B fragments of the group's
//     4 MFMAs; exact 1024-magic dequant to fp16 in the order (c0,c4),(c1,c5),(c2,c6),(c3,c7) per dword;
//   * A (X): lane loads 64 contiguous bytes of X row m0+j at column 128g + 32s and permutes each 16 bytes into the
//     same order, so A and B agree on every K index;
//   * per group: C = sum of 4 MFMAs from zero, then acc = scale * C + xsum * min in fp32 (xsum[g][m] precomputed
//     per block in LDS; a lane's 4 D rows are 4 consecutive m, one ds_read_b128).
// Codes never leave int4 in HBM; every product is exact, sums are fp32.
#include "common.h"

namespace {

RK_DEV uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

struct DqConsts {
    uint32_t lo_mask, hi_mask, magic;
};

RK_DEV h8_t dequant8(uint32_t w, const DqConsts& k) {
    const h2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    const h2_t s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2_t m64 = {(_Float16)-64.f, (_Float16)-64.f};
    const uint32_t b = w >> 8;
    const h2_t p0 = as_h2((w & k.lo_mask) | k.magic) + m1024;
    const h2_t p1 = as_h2((w & k.hi_mask) | k.magic) * s16 + m64;
    const h2_t p2 = as_h2((b & k.lo_mask) | k.magic) + m1024;
    const h2_t p3 = as_h2((b & k.hi_mask) | k.magic) * s16 + m64;
    h8_t r;
    r[0] = p0.x; r[1] = p0.y; r[2] = p1.x; r[3] = p1.y;
    r[4] = p2.x; r[5] = p2.y; r[6] = p3.x; r[7] = p3.y;
    return r;
}

// 8 consecutive activations (one 16-byte load) -> A fragment (x0,x4,x1,x5,x2,x6,x3,x7) as fp16
RK_DEV h8_t afrag(u4_t d, int xdt) {
    uint32_t h[4];
    if (xdt == RK_BF16) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f[2 * e] = __builtin_bit_cast(float, d[e] << 16);
            f[2 * e + 1] = __builtin_bit_cast(float, d[e] & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            h2_t p;
            p.x = (_Float16)f[e];
            p.y = (_Float16)f[e + 4];
            h[e] = as_u32(p);
        }
    } else {
        h[0] = perm(d.z, d.x, 0x05040100u);
        h[1] = perm(d.z, d.x, 0x07060302u);
        h[2] = perm(d.w, d.y, 0x05040100u);
        h[3] = perm(d.w, d.y, 0x07060302u);
    }
    return __builtin_bit_cast(h8_t, u4_t{h[0], h[1], h[2], h[3]});
}

// xsum[g][r] = fp32 sum of X[m0 + r, 128g .. 128g+127] for the block's BM rows (rows past M read row M-1)
RK_DEV void row_group_sums(const void* __restrict__ X, int xdt, int ldx, int M, int K, int m0, int BM,
                           float* __restrict__ xsum) {
    const int NG = K >> 7;
    // one thread per (row, group) pair, 16-byte loads along the group
    for (int p = threadIdx.x; p < BM * NG; p += blockDim.x) {
        const int g = p / BM, r = p - g * BM;
        const int m = min(m0 + r, M - 1);
        const u4_t* src = reinterpret_cast<const u4_t*>(reinterpret_cast<const uint16_t*>(X) + (size_t)m * ldx + 128 * g);
        float s = 0.f;
        for (int i = 0; i < 16; ++i) {
            const u4_t d = src[i];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                if (xdt == RK_BF16) {
                    s += __builtin_bit_cast(float, d[e] << 16) + __builtin_bit_cast(float, d[e] & 0xffff0000u);
                } else {
                    const h2_t v = as_h2(d[e]);
                    s += (float)v.x + (float)v.y;
                }
            }
        }
        xsum[g * BM + r] = s;
    }
}

template <int WM, int WN>
__global__ __launch_bounds__(256) void mm_int4_kernel(const void* __restrict__ X, int xdt, int ldx,
                                                      const uint8_t* __restrict__ q, const uint16_t* __restrict__ sc,
                                                      const uint16_t* __restrict__ mn, void* __restrict__ Y, int ydt,
                                                      int ldy, int M, int N, int K) {
    constexpr int BM = 2 * WM * 16, BN = 2 * WN * 16;
    extern __shared__ __align__(16) uint8_t smem[];
    float* xsum = reinterpret_cast<float*>(smem);  // [NG][BM]
    const int NG = K >> 7;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int j = lane & 15, s = lane >> 4;
    const int mb = blockIdx.y * BM, nb = blockIdx.x * BN;
    const int m0 = mb + wm * WM * 16, n0 = nb + wn * WN * 16;

    row_group_sums(X, xdt, ldx, M, K, mb, BM, xsum);
    __syncthreads();

    const DqConsts kc = {opaque(0x000F000Fu), opaque(0x00F000F0u), opaque(0x64006400u)};
    const uint16_t* xrow[WM];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
        xrow[mt] = reinterpret_cast<const uint16_t*>(X) + (size_t)min(m0 + mt * 16 + j, M - 1) * ldx + 32 * s;
    const uint8_t* qrow[WN];
    const uint16_t* srow[WN];
    const uint16_t* mrow[WN];
#pragma unroll
    for (int nt = 0; nt < WN; ++nt) {
        const int n = min(n0 + nt * 16 + j, N - 1);
        qrow[nt] = q + (size_t)n * (size_t)(K >> 1) + 16 * s;
        srow[nt] = sc + (size_t)n * NG;
        mrow[nt] = mn + (size_t)n * NG;
    }

    f4_t acc[WM][WN];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) acc[mt][nt] = f4_t{0.f, 0.f, 0.f, 0.f};

    for (int g = 0; g < NG; ++g) {
        u4_t wq[WN];
        uint16_t sv[WN], mv[WN];
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) {
            wq[nt] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(qrow[nt] + (size_t)g * 64));
            sv[nt] = srow[nt][g];
            mv[nt] = mrow[nt][g];
        }
        u4_t xa[WM][4];
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int t = 0; t < 4; ++t) xa[mt][t] = reinterpret_cast<const u4_t*>(xrow[mt] + 128 * g)[t];
        h8_t A[WM][4], B[WN][4];
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int t = 0; t < 4; ++t) A[mt][t] = afrag(xa[mt][t], xdt);
#pragma unroll
        for (int nt = 0; nt < WN; ++nt)
#pragma unroll
            for (int t = 0; t < 4; ++t) B[nt][t] = dequant8(wq[nt][t], kc);
#pragma unroll
        for (int mt = 0; mt < WM; ++mt) {
            // this lane's 4 D rows are m0 + mt*16 + 4s + e: their group sums are 4 consecutive floats
            const f4_t xs = *reinterpret_cast<const f4_t*>(xsum + g * BM + wm * WM * 16 + mt * 16 + 4 * s);
#pragma unroll
            for (int nt = 0; nt < WN; ++nt) {
                f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < 4; ++t) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt][t], B[nt][t], c, 0, 0, 0);
                const float scl = f16_bits_to_f32(sv[nt]), mnv = f16_bits_to_f32(mv[nt]);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[mt][nt][e] = __builtin_fmaf(c[e], scl, __builtin_fmaf(xs[e], mnv, acc[mt][nt][e]));
            }
        }
    }

#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) {
            const int n = n0 + nt * 16 + j;
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = m0 + mt * 16 + 4 * s + e;
                if (m < M) store_act(Y, ydt, (size_t)m * ldy + n, acc[mt][nt][e]);
            }
        }
}

template <int WM, int WN>
hipError_t launch_mm(const void* X, int xdt, int ldx, const uint8_t* q, const uint16_t* s, const uint16_t* m, void* Y,
                     int ydt, int ldy, int M, int N, int K, hipStream_t st) {
    constexpr int BM = 2 * WM * 16, BN = 2 * WN * 16;
    const size_t lds = (size_t)(K / 128) * BM * 4;
    dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL((mm_int4_kernel<WM, WN>), grid, dim3(256), lds, st, X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K);
    return hipGetLastError();
}

}  // namespace

extern "C" int rk_mm_int4_g128(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
                               const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K,
                               rk_stream_t stream) {
    if (!X || !q || !scale || !min || !Y) return RK_ERR_NULL;
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0 || ldx < K || ldy < N) return RK_ERR_SHAPE;
    if (x_dtype != RK_F16 && x_dtype != RK_BF16) return RK_ERR_DTYPE;
    if (y_dtype != RK_F16 && y_dtype != RK_BF16 && y_dtype != RK_F32) return RK_ERR_DTYPE;
    if (((uintptr_t)X & 15) || ((uintptr_t)q & 15) || (ldx % 8)) return RK_ERR_ALIGN;
    hipStream_t s = reinterpret_cast<hipStream_t>(stream);
    hipError_t e;
    // short prompts: 32-row blocks (memory-bound, keep the grid wide); longer: 64 x 64 blocks
    if (M <= 32) e = launch_mm<1, 2>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, s);
    else e = launch_mm<2, 2>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, s);
    return e == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
