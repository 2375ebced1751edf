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
#include <mutex>
#include <type_traits>

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

    // one group's operands; the next group's are loaded while the current one computes (software pipelining)
    struct Stage {
        u4_t wq[WN];
        uint16_t sv[WN], mv[WN];
        u4_t xa[WM][4];
    };
    auto load = [&](Stage& st, int g) {
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) {
            st.sv[nt] = srow[nt][g];
            st.mv[nt] = mrow[nt][g];
        }
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int t = 0; t < 4; ++t) st.xa[mt][t] = reinterpret_cast<const u4_t*>(xrow[mt] + 128 * g)[t];
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) st.wq[nt] = reinterpret_cast<const u4_t*>(qrow[nt] + (size_t)g * 64)[0];
    };
    auto compute = [&](const Stage& st, int g) {
        h8_t A[WM][4], B[WN][4];
#pragma unroll
        for (int mt = 0; mt < WM; ++mt)
#pragma unroll
            for (int t = 0; t < 4; ++t) A[mt][t] = afrag(st.xa[mt][t], xdt);
#pragma unroll
        for (int nt = 0; nt < WN; ++nt)
#pragma unroll
            for (int t = 0; t < 4; ++t) B[nt][t] = dequant8(st.wq[nt][t], kc);
#pragma unroll
        for (int mt = 0; mt < WM; ++mt) {
            // this lane's 4 D rows are m0 + mt*16 + 4s + e: their group sums are 4 consecutive floats
            const f4_t xs = *reinterpret_cast<const f4_t*>(xsum + g * BM + wm * WM * 16 + mt * 16 + 4 * s);
#pragma unroll
            for (int nt = 0; nt < WN; ++nt) {
                f4_t c = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int t = 0; t < 4; ++t) c = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt][t], B[nt][t], c, 0, 0, 0);
                const float scl = f16_bits_to_f32(st.sv[nt]), mnv = f16_bits_to_f32(st.mv[nt]);
#pragma unroll
                for (int e = 0; e < 4; ++e) acc[mt][nt][e] = __builtin_fmaf(c[e], scl, __builtin_fmaf(xs[e], mnv, acc[mt][nt][e]));
            }
        }
    };
    Stage cur, nxt;
    load(cur, 0);
    int g = 0;
    for (; g + 1 < NG; ++g) {
        load(nxt, g + 1);
        compute(cur, g);
        cur = nxt;
    }
    compute(cur, g);

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

// ---------------------------------------------------------------------------------------------- LDS-tiled kernel
// Block = 4 waves (2 x 2), tile BM x BN = (2*WM*16) x (2*WN*16). Per 128-column K step (one quantization group) the
// One K step (128-column group) of a block tile staged in LDS, double-buffered: the X rows as fp16 MFMA A
// fragments (dequant pair order), the code rows dequantised to exact fp16 codes as B fragments. MFMA t of a step covers columns 32s + 8t .. + 7 of the group in lane group s, as in the
// GEMV kernels.
template <int BM, int BN>
struct MmStage {
    // a[m tile][t][slot]: the A fragment of MFMA t for 16 rows; lane (row i, quarter s) sits in slot
    // 16 s + (i ^ (4 s + t)), so that both the 16-lane reads of a quarter and the writes of one row's 16 chunks
    // (all s, t) touch 16 distinct 16-byte bank groups
    uint4 a[BM / 16][4][64];
    uint4 b[BN / 16][4][64];  // b[n tile][t][lane]: lane (column j, quarter s)
};

// Block tile BM x BN = (2 WM 16) x (2 WN 16) with eight waves in two roles. Waves 0..3 (2 x 2) each hold WM x WN
// 16 x 16 MFMA tiles: per 128-column group g (one K step) they run 4 x WM x WN MFMAs from LDS stage g % 2 into
// per-step sums c, 4 x WM more against an all-ones B for the rows' sums of X over the group (exact products, fp32
// accumulation, already in the accumulator layout), and apply the group's affine, acc += c * scale[n] +
// rowsum(X)[m] * min[n] (fp32, as the reference's Triton kernel does). Waves 4..7 stage: they keep the X rows and
// code rows of the next two steps in registers and, during step g, convert step g + 1 into the other LDS stage
// (X -> fp16 fragments, codes -> exact fp16). One barrier per step; the two roles run on every SIMD at once, so
// the staging conversions overlap the MFMAs instead of following them.
// Split K (splits > 1): block (tile, split) covers groups [split NG / splits, (split + 1) NG / splits) and writes
// its fp32 sums to part[split][M][N] for mm_splitk_reduce; with splits == 1 the block writes Y directly.
// BF16: activations are bf16 (else fp16), a template parameter so the staging has no per-chunk dtype branches
template <int WM, int WN, bool BF16>
__global__ __launch_bounds__(512) void mm_int4_lds_kernel(const void* __restrict__ X, int ldx,
                                                          const uint8_t* __restrict__ q, const uint16_t* __restrict__ sc,
                                                          const uint16_t* __restrict__ mn, void* __restrict__ Y,
                                                          int ydt, int ldy, int M, int N, int K,
                                                          float* __restrict__ part, int splits) {
    constexpr int BM = 2 * WM * 16, BN = 2 * WN * 16;
    constexpr int XCH = BM * 16 / 256;  // 16-byte X chunks per staging thread per step (row r, 8-column block c)
    constexpr int WCH = BN * 4 / 256;   // 16-byte code chunks per staging thread per step (row n, quarter s)
    static_assert(XCH >= 1 && WCH >= 1, "tile too small for 256 staging threads");
    using Stage = MmStage<BM, BN>;
    extern __shared__ __align__(16) uint8_t smem[];
    Stage* stg = reinterpret_cast<Stage*>(smem);  // [2]
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform: role branches are scalar
    const bool stager = wave >= 4;
    const int sid = tid - 256;  // staging thread index (stager waves)
    const int wm = (wave & 3) >> 1, wn = wave & 1;
    // 1-D grid: workgroups go round-robin to the 8 XCDs, so virtual id (L % 8) * (G / 8) + L / 8 gives each XCD a
    // contiguous range, walked row block fastest: the row blocks sharing one code tile run together on one L2
    const int G = gridDim.x, L = blockIdx.x, GY = (M + BM - 1) / BM;
    const int Lv = (G % 8 == 0) ? (L % 8) * (G / 8) + L / 8 : L;
    const int split = Lv % splits, tile = Lv / splits;
    const int mb = (tile % GY) * BM, nb = (tile / GY) * BN;
    const int NGT = K >> 7;                                                   // groups of a row
    const int g0 = split * NGT / splits, NG = (split + 1) * NGT / splits - g0;  // this block's groups
    uint32_t* smw = reinterpret_cast<uint32_t*>(stg + 2);  // [BN][NG]: scale | min << 16 of the block's rows

    for (int i = tid; i < BN * NG; i += 512) {
        const int n = min(nb + i / NG, N - 1), g = g0 + i % NG;
        smw[i] = (uint32_t)sc[(size_t)n * NGT + g] | ((uint32_t)mn[(size_t)n * NGT + g] << 16);
    }
    // staging slots: X chunk i -> row r = idx / 16, 8-column block c = idx % 16 (a row's 256 bytes in 16
    // consecutive lanes); code chunk i -> row r = idx % 16 + 16 (idx / 64),
    // quarter s = idx / 16 % 4 (16 consecutive lanes write one quarter of 16 rows: no bank conflict)
    struct Regs {
        u4_t xr[XCH], wr[WCH];
    };
    auto load = [&](Regs& R, int g) {
        auto& xr = R.xr; auto& wr = R.wr;
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int idx = sid + 256 * i, r = idx >> 4, c = idx & 15;
            const int m = min(mb + r, M - 1);
            xr[i] = *reinterpret_cast<const u4_t*>(reinterpret_cast<const uint16_t*>(X) + (size_t)m * ldx +
                                                   128 * (g0 + g) + 8 * c);
        }
#pragma unroll
        for (int i = 0; i < WCH; ++i) {
            const int idx = sid + 256 * i, r = (idx & 15) | ((idx >> 6) << 4), qq = (idx >> 4) & 3;
            const int n = min(nb + r, N - 1);
            wr[i] = *reinterpret_cast<const u4_t*>(q + (size_t)n * (size_t)(K >> 1) + 64 * (g0 + g) + 16 * qq);
        }
    };
    auto store = [&](const Regs& R, Stage& st) {
        const DqConsts kc = {opaque(0x000F000Fu), opaque(0x00F000F0u), opaque(0x64006400u)};
        const auto& xr = R.xr; const auto& wr = R.wr;
#pragma unroll
        for (int i = 0; i < XCH; ++i) {
            const int idx = sid + 256 * i, r = idx >> 4, c = idx & 15;
            // 8-column block c = 32s + 8t: quarter s = c / 4, MFMA t = c % 4, swizzle 4 s + t = c
            st.a[r >> 4][c & 3][16 * (c >> 2) + ((r & 15) ^ c)] =
                __builtin_bit_cast(uint4, afrag(xr[i], BF16 ? RK_BF16 : RK_F16));
        }
#pragma unroll
        for (int i = 0; i < WCH; ++i) {
            const int idx = sid + 256 * i, r = (idx & 15) | ((idx >> 6) << 4), qq = (idx >> 4) & 3;
#pragma unroll
            for (int t = 0; t < 4; ++t)
                st.b[r >> 4][t][(r & 15) + 16 * qq] = __builtin_bit_cast(uint4, dequant8(wr[i][t], kc));
        }
    };

    // The two roles run separate loops with the same number of barriers (two before the K loop, one per step), so
    // neither holds the other's registers.
    if (stager) {
        Regs R0, R1;  // two steps in flight: step g + 2 is loaded while step g + 1 is converted
        load(R0, 0);
        load(R1, min(1, NG - 1));
        __syncthreads();  // smw
        store(R0, stg[0]);
        __syncthreads();
        // during step g: reload Rn (it held step g, already in LDS) with step g + 2, store step g + 1 (in Rs since
        // one step ago) into the other stage, last read by the MFMA waves one step ago, before the barrier
        auto step = [&](int g, Regs& Rn, const Regs& Rs) {
            load(Rn, min(g + 2, NG - 1));  // unconditional (the last steps reload the last group, unused): a
                                           // conditional load would make the compiler wait for every load in flight
            if (g + 1 < NG) store(Rs, stg[(g + 1) & 1]);
            __syncthreads();
        };
        int g = 0;
        for (; g + 1 < NG; g += 2) {  // unrolled by two so each register set has a fixed role
            step(g, R0, R1);
            step(g + 1, R1, R0);
        }
        if (g < NG) step(g, R0, R1);
        return;
    }

    f4_t acc[WM][WN];
#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) acc[mt][nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    // A fragment slot of this lane for MFMA t (the swizzle of the stores)
    int aslot[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) aslot[t] = 16 * (lane >> 4) + ((lane & 15) ^ (4 * (lane >> 4) + t));
    __syncthreads();  // smw
    __syncthreads();  // stage 0
    const h8_t ones = {1, 1, 1, 1, 1, 1, 1, 1};
    for (int g = 0; g < NG; ++g) {
        const Stage& st = stg[g & 1];
        f4_t c[WM][WN], xs[WM];
#pragma unroll
        for (int mt = 0; mt < WM; ++mt) {
            xs[mt] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int nt = 0; nt < WN; ++nt) c[mt][nt] = f4_t{0.f, 0.f, 0.f, 0.f};
        }
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            h8_t A[WM], B[WN];
#pragma unroll
            for (int mt = 0; mt < WM; ++mt) A[mt] = __builtin_bit_cast(h8_t, st.a[wm * WM + mt][t][aslot[t]]);
#pragma unroll
            for (int nt = 0; nt < WN; ++nt) B[nt] = __builtin_bit_cast(h8_t, st.b[wn * WN + nt][t][lane]);
#pragma unroll
            for (int mt = 0; mt < WM; ++mt) {
#pragma unroll
                for (int nt = 0; nt < WN; ++nt)
                    c[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt], B[nt], c[mt][nt], 0, 0, 0);
                xs[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mt], ones, xs[mt], 0, 0, 0);
            }
        }
        // D[i][j] in lane j + 16 (i / 4), element i % 4: column n = tile + lane % 16, rows 4 (lane / 16) + e
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) {
            const uint32_t w = smw[((wn * WN + nt) * 16 + (lane & 15)) * NG + g];
            const float scl = f16_bits_to_f32((uint16_t)w), mnv = f16_bits_to_f32((uint16_t)(w >> 16));
#pragma unroll
            for (int mt = 0; mt < WM; ++mt)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    acc[mt][nt][e] = __builtin_fmaf(c[mt][nt][e], scl, __builtin_fmaf(xs[mt][e], mnv, acc[mt][nt][e]));
        }
        __syncthreads();
    }

#pragma unroll
    for (int mt = 0; mt < WM; ++mt)
#pragma unroll
        for (int nt = 0; nt < WN; ++nt) {
            const int n = nb + (wn * WN + nt) * 16 + (lane & 15);
            if (n >= N) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int m = mb + (wm * WM + mt) * 16 + 4 * (lane >> 4) + e;
                if (m >= M) continue;
                if (splits == 1)
                    store_act(Y, ydt, (size_t)m * ldy + n, acc[mt][nt][e]);
                else
                    part[((size_t)split * M + m) * N + n] = acc[mt][nt][e];
            }
        }
}

// ---------------------------------------------------------------------------------------------- prepared-X kernel
// Two launches, for the workspace entry on shapes with enough column blocks to fill the chip:
//   mm_xprep_kernel: X once into the workspace, in the MFMA A-fragment order of dequant8's code order (fp16), plus
//     the fp32 sum of each row over each group;
//   mm_int4_prep_kernel<MT>: blocks of 16 MT rows x 128 columns, eight waves, wave w owning column tile w (16
//     columns) for all rows. Every K step (one group) is copied straight from memory into a three-slot LDS ring
//     with global_load_lds_dwordx4 (16 bytes per lane, no staging waves, no register round trip): the block's X
//     fragments, its 128 code rows, the rows' sums. The block's scale and min rows are copied once into LDS. A
//     wave dequantises its own columns (no column is converted twice) and runs 4 MT MFMAs per step.
// The copies are ordered by explicit vmcnt waits: each wave waits for its own copies of step g, then a barrier
// makes every wave's copies of step g visible and certifies that every wave has left step g - 1, whose slot the
// copies of step g + 2 then fill.

// s_waitcnt vmcnt(n) alone (gfx9 encoding: vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt left at their maxima)
#define RK_VMCNT(n) __builtin_amdgcn_s_waitcnt(((n) & 15) | (((n) >> 4) << 14) | (7 << 4) | (15 << 8))

// Xp[mt][g][t][lane] (16 bytes): afrag of X[16 mt + j][128 g + 32 s + 8 t .. + 7], lane = j + 16 s (rows past M are
// zero); xs[g][m] = fp32 sum of X[m][128 g .. 128 g + 127]. One thread per 16-byte chunk (m, g, c = 4 s + t); block
// b = (m tile, group) covers the 16 rows' 16 chunks of one group, so it writes one whole 4 KiB fragment block.
template <bool BF16>
__global__ __launch_bounds__(256) void mm_xprep_kernel(const void* __restrict__ X, int ldx, int M, int Mp, int K,
                                                       uint4* __restrict__ Xp, float* __restrict__ xs) {
    const int NG = K >> 7;
    const int c = threadIdx.x & 15;                               // chunk within the row's group
    const int g = blockIdx.x % NG, m = (blockIdx.x / NG) * 16 + (threadIdx.x >> 4);  // grid: Mp / 16 * NG blocks
    u4_t d = {0u, 0u, 0u, 0u};
    if (m < M)
        d = *reinterpret_cast<const u4_t*>(reinterpret_cast<const uint16_t*>(X) + (size_t)m * ldx + 128 * g + 8 * c);
    const int s = c >> 2, t = c & 3;
    Xp[(((size_t)(m >> 4) * NG + g) * 4 + t) * 64 + (m & 15) + 16 * s] =
        __builtin_bit_cast(uint4, afrag(d, BF16 ? RK_BF16 : RK_F16));
    float f = 0.f;
    if (BF16) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            f += __builtin_bit_cast(float, d[e] << 16) + __builtin_bit_cast(float, d[e] & 0xffff0000u);
    } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const h2_t v = as_h2(d[e]);
            f += (float)v.x + (float)v.y;
        }
    }
    f += dpp<0xB1>(f);   // the row's 16 chunks sit in one 16-lane DPP row
    f += dpp<0x4E>(f);
    f += dpp<0x141>(f);
    f += dpp<0x140>(f);
    if (c == 0) xs[(size_t)g * Mp + m] = f;
}

template <int MT>
struct PrepStage {
    uint4 x[MT][4][64];  // [m tile][MFMA t][lane (row j, quarter s)]
    uint4 w[8][64];      // [column tile][lane (column j, quarter s)]: bytes 16 s .. 16 s + 15 of the column's group
};
static_assert(sizeof(PrepStage<3>) == (3 * 4 + 8) * 64 * 16, "stage layout: x then w, no padding");
constexpr int kPrepRing = 3;  // X / code slots: steps g, g + 1 (in flight), g + 2 (being copied)
constexpr int kPrepXsRing = 4;  // row-sum slots live one step longer: step g - 1's are read in step g

template <int MT>
size_t mm_prep_lds_bytes(int ng) {
    return kPrepRing * sizeof(PrepStage<MT>) + kPrepXsRing * 128 * 4 + (size_t)2 * 128 * ng * 2;
}

// One block: rows mb .. mb + 16 MT - 1, columns nb .. nb + 127. Requires (N * NG) % 8 == 0 (the scale / min arrays
// end on a 16-byte boundary) and 16-byte aligned scale / min arrays; the host checks both.
template <int MT>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(1, 2)))
void mm_int4_prep_kernel(const uint4* __restrict__ Xp, const float* __restrict__ xsg, int Mp,
                         const uint8_t* __restrict__ q, const uint16_t* __restrict__ sc,
                         const uint16_t* __restrict__ mn, void* __restrict__ Y, int ydt, int ldy, int M, int N,
                         int K) {
    constexpr int BM = 16 * MT;
    constexpr int XPW = (MT * 4 + 7) / 8;  // X tile copies per wave per step (surplus slots repeat the last tile)
    using Stage = PrepStage<MT>;
    extern __shared__ __align__(16) uint8_t smem[];
    Stage* stg = reinterpret_cast<Stage*>(smem);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // 1-D grid, XCD-grouped as in mm_int4_lds_kernel: the row blocks of one column block run on one L2
    const int G = gridDim.x, L = blockIdx.x, GY = (Mp + BM - 1) / BM;
    const int Lv = (G % 8 == 0) ? (L % 8) * (G / 8) + L / 8 : L;
    const int mb = (Lv % GY) * BM, nb = (Lv / GY) * 128;
    const int NG = K >> 7;
    const int mts = min(MT, (Mp - mb) >> 4);  // m tiles of this block present in Xp
    float* xsr = reinterpret_cast<float*>(stg + kPrepRing);              // [kPrepXsRing][128]
    uint16_t* tsc = reinterpret_cast<uint16_t*>(xsr + kPrepXsRing * 128);  // [128][NG]
    uint16_t* tmn = tsc + 128 * NG;
    const int jn = lane & 15, sq = lane >> 4;

    // the block's scale and min rows ([n][g], contiguous), 16-byte copies clamped inside the arrays
    {
        const int nch = 16 * NG;                                        // 16-byte chunks per table
        const int lastc = (int)(((size_t)N * NG * 2) / 16) - 1;
        const size_t c0 = (size_t)nb * NG / 8;
        for (int b0 = wave * 64; b0 < nch; b0 += 512) {
            const int ci = min((int)(c0 + b0 + lane), lastc);
            if (b0 + lane < nch) {  // lanes past the table copy nothing
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4*>(sc) + ci,
                                                 reinterpret_cast<uint4*>(tsc) + b0, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint4*>(mn) + ci,
                                                 reinterpret_cast<uint4*>(tmn) + b0, 16, 0, 0);
            }
        }
    }
    // a step's copies per wave: X tiles i = wave + 8 k (m tile i / 4, t = i % 4), code tile `wave`, and 64 row sums
    // (waves 0 and 1)
    const uint8_t* wsrc = q + (size_t)min(nb + 16 * wave + jn, N - 1) * (size_t)(K >> 1) + 16 * sq;
    // copy destinations are addressed from the LDS base, not through the MT-dependent stage type: a dependent LDS
    // operand keeps the host pass from instantiating the kernel (its launch stub would be missing)
    auto issue = [&](int g) {
        uint4* slot = reinterpret_cast<uint4*>(smem + (size_t)(g % kPrepRing) * sizeof(Stage));  // Stage::x, Stage::w
#pragma unroll
        for (int k = 0; k < XPW; ++k) {
            const int i = min(wave + 8 * k, MT * 4 - 1), mt = i >> 2, t = i & 3;
            __builtin_amdgcn_global_load_lds(Xp + (((size_t)(mb / 16 + min(mt, mts - 1)) * NG + g) * 4 + t) * 64 + lane,
                                             slot + (mt * 4 + t) * 64, 16, 0, 0);
        }
        __builtin_amdgcn_global_load_lds(wsrc + 64 * g, slot + MT * 4 * 64 + wave * 64, 16, 0, 0);
        if (wave < 2)
            __builtin_amdgcn_global_load_lds(xsg + (size_t)g * Mp + min(mb + 64 * wave + lane, Mp - 1),
                                             xsr + (g % kPrepXsRing) * 128 + 64 * wave, 4, 0, 0);
    };

    f4_t acc[MT], c[MT];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) acc[mt] = f4_t{0.f, 0.f, 0.f, 0.f};
    const DqConsts kc = {opaque(0x000F000Fu), opaque(0x00F000F0u), opaque(0x64006400u)};
    const int col = 16 * wave + jn;
#pragma unroll
    for (int p = 0; p < kPrepRing - 1; ++p) issue(min(p, NG - 1));
    // the epilogue's arguments come in before the loop: a scalar load still in flight would turn every LDS wait
    // of the loop into lgkmcnt(0) (scalar loads complete out of order)
    asm volatile("" ::"s"(Y), "s"(ydt), "s"(ldy), "s"(M), "s"(N));
    for (int g = 0; g < NG; ++g) {
        // newer than this wave's copies of step g: its copies of step g + 1 (XPW + 1, or XPW + 2 with row sums)
        if (wave < 2) RK_VMCNT(XPW + 2); else RK_VMCNT(XPW + 1);
        __builtin_amdgcn_s_barrier();
        issue(min(g + kPrepRing - 1, NG - 1));  // into the slot of step g - 1 (clamped: the last steps repeat)
        const Stage& st = stg[g % kPrepRing];
        const u4_t wq = __builtin_bit_cast(u4_t, st.w[wave][lane]);
        // X fragments of MFMA step t + 1 are read while step t's MFMAs run
        h8_t Xa[MT], Xb[MT];
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) Xa[mt] = __builtin_bit_cast(h8_t, st.x[mt][0][lane]);
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            h8_t* Xc = (t & 1) ? Xb : Xa;
            h8_t* Xn = (t & 1) ? Xa : Xb;
            if (t < 3) {
#pragma unroll
                for (int mt = 0; mt < MT; ++mt) Xn[mt] = __builtin_bit_cast(h8_t, st.x[mt][t + 1][lane]);
            }
            const h8_t Wf = dequant8(wq[t], kc);
#pragma unroll
            for (int mt = 0; mt < MT; ++mt)
                c[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Xc[mt], Wf, t == 0 ? f4_t{0.f, 0.f, 0.f, 0.f} : c[mt],
                                                             0, 0, 0);
        }
        // D[i][j]: row 4 (lane / 16) + e of m tile mt, column lane % 16 of the wave's tile; group affine in fp32
        const float scl = f16_bits_to_f32(tsc[col * NG + g]), mnv = f16_bits_to_f32(tmn[col * NG + g]);
        const float* xs = xsr + (g % kPrepXsRing) * 128;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            const f4_t xv = *reinterpret_cast<const f4_t*>(&xs[mt * 16 + 4 * sq]);
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[mt][e] = __builtin_fmaf(c[mt][e], scl, __builtin_fmaf(xv[e], mnv, acc[mt][e]));
        }
    }
    RK_VMCNT(0);
    __builtin_amdgcn_s_barrier();  // every wave has left the ring: it becomes the output transpose buffer

    // the wave's BM x 16 tile through LDS ([BM][17] fp32), then 16-byte row pieces: lane -> row 32 i + lane / 2,
    // columns 8 (lane % 2) .. + 7
    float* tb = reinterpret_cast<float*>(smem) + wave * (BM * 17);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int e = 0; e < 4; ++e) tb[(mt * 16 + 4 * sq + e) * 17 + jn] = acc[mt][e];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave reads back only its own tile
    const int n0 = nb + 16 * wave;
    const bool vec_ok = (((uintptr_t)Y | (size_t)ldy * (ydt == RK_F32 ? 4 : 2)) & (ydt == RK_F32 ? 15 : 7)) == 0;
#pragma unroll
    for (int i = 0; i < (BM + 31) / 32; ++i) {
        const int r = 32 * i + (lane >> 1), cc = 8 * (lane & 1);
        const int m = mb + r, n = n0 + cc;
        if (r >= BM || m >= M || n >= N) continue;
        const float* p = tb + r * 17 + cc;
        const size_t o = (size_t)m * ldy + n;
        if (n + 7 < N && vec_ok) {
            if (ydt == RK_F32) {
                *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(Y) + o) = f4_t{p[0], p[1], p[2], p[3]};
                *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(Y) + o + 4) = f4_t{p[4], p[5], p[6], p[7]};
            } else if (ydt == RK_F16) {
                const h8_t h = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
                                (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
                *reinterpret_cast<h8_t*>(reinterpret_cast<uint16_t*>(Y) + o) = h;
            } else {
                u4_t b;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    b[e] = (uint32_t)f32_to_bf16_bits(p[2 * e]) | ((uint32_t)f32_to_bf16_bits(p[2 * e + 1]) << 16);
                *reinterpret_cast<u4_t*>(reinterpret_cast<uint16_t*>(Y) + o) = b;
            }
        } else {
            for (int e = 0; e < 8 && n + e < N; ++e) store_act(Y, ydt, o + e, p[e]);
        }
    }
}

// the three block heights the plan uses; explicit instantiation also emits their host launch stubs
#define RK_PREP_INST(MT)                                                                                          \
    template __global__ void mm_int4_prep_kernel<MT>(const uint4* __restrict__, const float* __restrict__, int,    \
                                                     const uint8_t* __restrict__, const uint16_t* __restrict__,     \
                                                     const uint16_t* __restrict__, void* __restrict__, int, int,    \
                                                     int, int, int);
RK_PREP_INST(3)
RK_PREP_INST(4)
RK_PREP_INST(8)
#undef RK_PREP_INST

// ------------------------------------------------------------------------------- prepared-X kernel, wide waves
// mm_int4_wide_kernel: the prepared X of mm_xprep_kernel, blocks of 128 rows x 128 columns with four waves in a
// 2 x 2 layout, wave (wm, wn) owning rows 64 wm .. + 63 and columns 64 wn .. + 63 (4 x 4 MFMA tiles), two blocks
// per CU:
//   * each X fragment read from LDS feeds four MFMAs (the fragment reads set the pace of the one-column-tile
//     layout); each code column is dequantised by the two waves that share it;
//   * codes go straight into registers, two steps ahead; X copies go into a two-slot LDS ring with
//     global_load_lds, one barrier per step;
//   * the min term sum_g xs[m][g] min[n][g] is each accumulator's starting value, computed on the matrix cores in
//     fp32 (v_mfma_f32_16x16x4f32, four groups per instruction) while the first copies land, from row sums copied
//     into the ring slot that step 0 leaves free; the per-step affine is one FMA per output (scale);
//   * the two blocks of a CU pass their barriers independently, so one block's affine, waits and barrier overlap
//     the other block's MFMAs.
// The ring slot of step g + 1 is filled after the barrier of step g, which every wave passes only once it has
// left step g - 1 (the slot's previous step).
constexpr int kWideRing = 2;
constexpr int kWideSlot = 8 * 4 * 64 * 16;              // one step's X fragments: 8 m tiles x 4 MFMA steps
constexpr int kWideOut = 4 * 64 * 65 * 4;               // epilogue transpose, per wave [64][65] fp32
constexpr int kWideArea = kWideOut > kWideRing * kWideSlot ? kWideOut : kWideRing * kWideSlot;

// ngs: the most groups one block takes (its split of K)
size_t mm_wide_lds_bytes(int ngs) { return (size_t)kWideArea + (size_t)2 * 128 * ngs * 2; }

// split sp of `splits` over the K / 128 groups, in whole pairs of groups: first group and count
__host__ __device__ inline void wide_split(int NG, int splits, int sp, int& g_lo, int& ngs) {
    const int P = NG >> 1, p_lo = sp * P / splits, p_hi = (sp + 1) * P / splits;
    g_lo = 2 * p_lo;
    ngs = 2 * (p_hi - p_lo);
}

// The ring's barrier: this wave's copies older than its newest `vm` loads are done and its LDS reads are done
// (lgkmcnt(0): the copies issued after the barrier refill the slot the last reads came from); the asm statements
// keep the compiler from moving LDS accesses across it (s_barrier itself is no memory operation).
template <int VM>
RK_DEV void wide_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt((VM & 15) | (7 << 4) | (0 << 8) | ((VM >> 4) << 14));  // vmcnt(VM) lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// Block = (tile, split): with splits > 1 each block takes an even range of >= 4 groups (wide_split) and writes
// its fp32 partial sums to part[split][M][N] (mm_splitk_reduce adds them in split order); with splits = 1 it takes
// all groups and writes Y. Requires K / 128 even, every split's group count >= 4 and <= kWideMaxGroups, and 4-byte
// aligned scale / min arrays; the host checks all of them.
constexpr int kWideMaxGroups = 26;  // LDS: 2 x 128 x 26 fp16 of tables beside the 66.5 KiB area stays <= 80 KiB

__global__ __launch_bounds__(256, 2) void mm_int4_wide_kernel(const uint4* __restrict__ Xp,
                                                              const float* __restrict__ xsg, int Mp,
                                                              const uint8_t* __restrict__ q,
                                                              const uint16_t* __restrict__ sc,
                                                              const uint16_t* __restrict__ mn, void* __restrict__ Y,
                                                              int ydt, int ldy, int M, int N, int K, int splits) {
    constexpr int BM = 128;
    extern __shared__ __align__(16) uint8_t smem[];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave & 1, wn = wave >> 1;
    // 1-D grid, XCD-grouped: the row blocks of one column block (and split) run on one L2
    const int G = gridDim.x, L = blockIdx.x, GY = (Mp + BM - 1) / BM;
    const int Lv = (G % 8 == 0) ? (L % 8) * (G / 8) + L / 8 : L;
    const int T = G / splits, sp = Lv / T, tl = Lv - sp * T;
    const int mb = (tl % GY) * BM, nb = (tl / GY) * 128;
    const int NG = K >> 7;
    int g_lo, ngs;  // this block's groups g_lo .. g_lo + ngs - 1
    wide_split(NG, splits, sp, g_lo, ngs);
    const int mts = min(8, (Mp - mb) >> 4);  // m tiles of this block present in Xp
    uint16_t* tsc = reinterpret_cast<uint16_t*>(smem + kWideArea);  // [128][ngs]
    uint16_t* tmn = tsc + 128 * ngs;
    float* xsl = reinterpret_cast<float*>(smem + kWideSlot);  // row sums [g][128] in ring slot 1 until step 0
    const int jn = lane & 15, sq = lane >> 4;

    // the block's scale and min entries ([n][g] for its groups: 4-byte copies, as g_lo and NG are even; columns
    // past N repeat the last) and row sums
    {
        const int hw = ngs >> 1, nd = 128 * hw;  // dwords per column, per table
        for (int b0 = wave * 64; b0 < nd; b0 += 256) {
            const int i = b0 + lane, c = i / hw, d = i - c * hw;
            const size_t src = ((size_t)min(nb + c, N - 1) * NG + g_lo) / 2 + d;
            if (i < nd) {
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(sc) + src,
                                                 reinterpret_cast<uint32_t*>(tsc) + b0, 4, 0, 0);
                __builtin_amdgcn_global_load_lds(reinterpret_cast<const uint32_t*>(mn) + src,
                                                 reinterpret_cast<uint32_t*>(tmn) + b0, 4, 0, 0);
            }
        }
        // xs[g][mb .. mb + 127] (rows past Mp repeat its last 4: their sums are never stored), 32 chunks a group
        for (int b0 = wave * 64; b0 < 32 * ngs; b0 += 256) {
            const int c = b0 + lane, g = c >> 5, r4 = min(c & 31, 4 * mts - 1);
            if (c < 32 * ngs)
                __builtin_amdgcn_global_load_lds(
                    reinterpret_cast<const uint4*>(xsg + (size_t)(g_lo + g) * Mp + mb) + r4,
                    reinterpret_cast<uint4*>(xsl) + b0, 16, 0, 0);
        }
    }
    // step g's X fragments i = wave + 4 k (m tile i / 4, MFMA step t = i % 4) into ring slot `sl`
    auto issue_x = [&](int g, int sl) {
        uint4* slot = reinterpret_cast<uint4*>(smem + (size_t)sl * kWideSlot);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int i = wave + 4 * k, mt = i >> 2, t = i & 3;
            __builtin_amdgcn_global_load_lds(
                Xp + (((size_t)(mb / 16 + min(mt, mts - 1)) * NG + g_lo + g) * 4 + t) * 64 + lane,
                slot + (mt * 4 + t) * 64, 16, 0, 0);
        }
    };
    // this lane's code bytes: column nb + 64 wn + 16 nt + jn (clamped), bytes 16 sq .. + 15 of each group. The
    // addresses pass through a volatile asm statement, which stays behind the X copies issued before it, so the
    // code loads follow those copies (the wait counts rely on that order; plain loads of read-only memory would
    // otherwise be free to move ahead of them).
    const uint8_t* wsrc[4];
#pragma unroll
    for (int nt = 0; nt < 4; ++nt) wsrc[nt] = q + (size_t)min(nb + 64 * wn + 16 * nt + jn, N - 1) * (size_t)(K >> 1) + 16 * sq;
    using gu4 = const __attribute__((address_space(1))) u4_t;
    auto load_w = [&](int g, u4_t (&w)[4]) {
        uint64_t a[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) a[nt] = (uint64_t)(wsrc[nt] + 64 * (g_lo + g));
        asm volatile("" : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]));
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) w[nt] = *(gu4*)a[nt];
    };

    issue_x(0, 0);
    u4_t wa[4], wb[4];  // codes of the even / odd steps
    load_w(0, wa);
    load_w(1, wb);
    // the epilogue's arguments come in before the loop (a scalar load in flight would turn the loop's LDS waits
    // into lgkmcnt(0))
    asm volatile("" ::: "memory");
    asm volatile("" ::"s"(Y), "s"(ydt), "s"(ldy), "s"(M), "s"(N));

    // the min term as the accumulators' start: tables and row sums landed (older than the 16 loads above)
    wide_barrier<16>();
    f4_t acc[4][4];
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) acc[mt][nt] = f4_t{0.f, 0.f, 0.f, 0.f};
    for (int qq = 0; qq < ngs; qq += 4) {
        const int gl = qq + sq;
        float mv[4], xa[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) mv[nt] = gl < ngs ? f16_bits_to_f32(tmn[(64 * wn + 16 * nt + jn) * ngs + gl]) : 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt) xa[mt] = gl < ngs ? xsl[gl * 128 + 64 * wm + 16 * mt + jn] : 0.f;
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int nt = 0; nt < 4; ++nt)
                acc[mt][nt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xa[mt], mv[nt], acc[mt][nt], 0, 0, 0);
    }

    const DqConsts kc = {opaque(0x000F000Fu), opaque(0x00F000F0u), opaque(0x64006400u)};
    // one K step (slot sl = g % 2): this wave's codes of step g are in w; on return they hold step g + 2's. Every
    // step issues the same loads in the same order (the last steps repeat the last group's, into the free slot and
    // the consumed registers), so one wait count fits every step: when step g starts, the loads newer than its X
    // copies and codes are step g + 1's codes (4 loads).
    auto step = [&](int g, int sl, u4_t (&w)[4], auto last) {
        wide_barrier<4>();
        if constexpr (!decltype(last)::value) issue_x(min(g + 1, ngs - 1), sl ^ 1);  // into step g - 1's slot
        const uint4* slot = reinterpret_cast<const uint4*>(smem + (size_t)sl * kWideSlot);
        h8_t A[4][4];  // the wave's 4 m tiles x 4 MFMA steps
#pragma unroll
        for (int mt = 0; mt < 4; ++mt)
#pragma unroll
            for (int t = 0; t < 4; ++t) A[mt][t] = __builtin_bit_cast(h8_t, slot[((4 * wm + mt) * 4 + t) * 64 + lane]);
        float sv[4];
#pragma unroll
        for (int nt = 0; nt < 4; ++nt) sv[nt] = f16_bits_to_f32(tsc[(64 * wn + 16 * nt + jn) * ngs + g]);
        // column tiles in pairs: dequantise the pair's codes, then per m tile pair the 4 MFMA steps on 2 x 2 tiles
        // (four independent chains) and their affine
#pragma unroll
        for (int np = 0; np < 4; np += 2) {
            h8_t B[2][4];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int t = 0; t < 4; ++t) B[j][t] = dequant8(w[np + j][t], kc);
            if constexpr (!decltype(last)::value)
                if (np == 2) load_w(min(g + 2, ngs - 1), w);
#pragma unroll
            for (int mp = 0; mp < 4; mp += 2) {
                f4_t c[2][2];
#pragma unroll
                for (int t = 0; t < 4; ++t)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
#pragma unroll
                        for (int j = 0; j < 2; ++j)
                            c[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[mp + i][t], B[j][t],
                                                                            t == 0 ? f4_t{0.f, 0.f, 0.f, 0.f} : c[i][j],
                                                                            0, 0, 0);
                // D[i][j]: row 4 (lane / 16) + e of the m tile, column lane % 16 of the tile: scale in fp32
#pragma unroll
                for (int i = 0; i < 2; ++i)
#pragma unroll
                    for (int j = 0; j < 2; ++j)
#pragma unroll
                        for (int e = 0; e < 4; ++e)
                            acc[mp + i][np + j][e] = __builtin_fmaf(c[i][j][e], sv[np + j], acc[mp + i][np + j][e]);
            }
        }
    };
    // NG is even. Step 0 runs before the loop: the code loads above may be issued in any order, and a code register
    // possibly in flight at the loop's first wait would make the compiler's waits in every iteration vmcnt(0); from
    // step 1 on the load order is the loop's own. The last step, after the loop, issues no loads.
    using more = std::integral_constant<bool, false>;
    __builtin_assume(ngs >= 4);  // the loop runs at least once (the host checks)
    step(0, 0, wa, more{});
    for (int g = 1; g + 1 < ngs; g += 2) {
        step(g, 1, wb, more{});
        step(g + 1, 0, wa, more{});
    }
    step(ngs - 1, 1, wb, std::integral_constant<bool, true>{});
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0 | (7 << 4) | (0 << 8));  // vmcnt(0) lgkmcnt(0): copies landed, ring reads done
    __builtin_amdgcn_s_barrier();                           // every wave has left the ring
    asm volatile("" ::: "memory");

    // the wave's 64 x 64 tile through LDS ([64][65] fp32), then 16-byte row pieces: lane -> row 8 i + lane / 8,
    // columns 8 (lane % 8) .. + 7
    float* tb = reinterpret_cast<float*>(smem) + wave * (64 * 65);
#pragma unroll
    for (int mt = 0; mt < 4; ++mt)
#pragma unroll
        for (int nt = 0; nt < 4; ++nt)
#pragma unroll
            for (int e = 0; e < 4; ++e) tb[(mt * 16 + 4 * sq + e) * 65 + 16 * nt + jn] = acc[mt][nt][e];
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): the wave reads back only its own tile
    const int m0 = mb + 64 * wm, n0 = nb + 64 * wn;
    if (splits > 1) Y = reinterpret_cast<float*>(Y) + (size_t)sp * M * ldy;  // this split's partial sums
    const bool vec_ok = (((uintptr_t)Y | (size_t)ldy * (ydt == RK_F32 ? 4 : 2)) & (ydt == RK_F32 ? 15 : 7)) == 0;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int r = 8 * i + (lane >> 3), cc = 8 * (lane & 7);
        const int m = m0 + r, n = n0 + cc;
        if (m >= M || n >= N) continue;
        const float* p = tb + r * 65 + cc;
        const size_t o = (size_t)m * ldy + n;
        if (n + 7 < N && vec_ok) {
            if (ydt == RK_F32) {
                *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(Y) + o) = f4_t{p[0], p[1], p[2], p[3]};
                *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(Y) + o + 4) = f4_t{p[4], p[5], p[6], p[7]};
            } else if (ydt == RK_F16) {
                const h8_t h = {(_Float16)p[0], (_Float16)p[1], (_Float16)p[2], (_Float16)p[3],
                                (_Float16)p[4], (_Float16)p[5], (_Float16)p[6], (_Float16)p[7]};
                *reinterpret_cast<h8_t*>(reinterpret_cast<uint16_t*>(Y) + o) = h;
            } else {
                u4_t b;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    b[e] = (uint32_t)f32_to_bf16_bits(p[2 * e]) | ((uint32_t)f32_to_bf16_bits(p[2 * e + 1]) << 16);
                *reinterpret_cast<u4_t*>(reinterpret_cast<uint16_t*>(Y) + o) = b;
            }
        } else {
            for (int e = 0; e < 8 && n + e < N; ++e) store_act(Y, ydt, o + e, p[e]);
        }
    }
}

// ---------------------------------------------------------------------------------------------- small-M stream
// For M <= 16 MT rows (MT <= 3) and K <= 2048 X is small enough to stay in registers: a block of eight waves holds X
// as MFMA A fragments for the whole launch, wave w owning <= 2 of the <= 16 groups, and
// streams 16-column tiles of codes past them (D tiles of codes in flight per wave: all of a block's tiles when it
// has <= 8). Per tile a wave dequantises
// its groups' codes once (16 bytes per lane per group: column j = lane % 16, bytes 16 s .. 16 s + 15 of the group,
// s = lane / 16, as in the tile kernels), runs 4 MT MFMAs per group and applies the group's scale in fp32; the
// eight waves' sums meet in LDS (two buffers, one barrier per tile), wave mt < MT adds them in wave order together
// with the tile's min term (sum over groups of rowsum * min, fp32 MFMAs) into the block's output stage, and the
// block stores its tiles at the end as 16-byte row pieces. Weights are read exactly once; X once per block.
// The tile loop has no conditional memory instruction: every step issues the same two code loads (clamped to the
// block's last tile; the surplus re-reads hit the L2) and computes (steps past the block's tiles compute on the
// clamped codes and are never stored), and the global stores come after the loop. The compiler's vmcnt waits
// then stay exact; a conditional load or store in the loop makes it wait for everything in flight.
constexpr int kStreamWaves = 8;
constexpr int kStreamMaxGroups = 16;  // K <= 2048: two groups per wave
constexpr int kStreamBlocks = 256;    // one block per CU
constexpr int kStreamTab = 4;         // scale / min table entries copied per thread (tables <= 2048 entries)

// A build option (RK_STREAM_TRACE; off in the product library, where RK_STR is empty): wall-clock stamps per (block,
// wave, event) in scalar registers, stored at the end of the launch to the buffer rk_stream_trace_set names
// ([block][8 waves][16 events] uint64, 100 MHz ticks), which the host reads after the launch.
// Events: 0 start, 1 prologue loads issued, 2 X fragments and row sums done, 3 tables in LDS (barrier passed),
// 4 / 5 tile 0 computed / reduced (its barrier passed), 6 / 7 tile 1, 8 / 9 the block's last tile, 10 loop done,
// 11 stores issued, 12 stores complete.
#ifdef RK_STREAM_TRACE
__device__ unsigned long long* g_stream_trace;
#define RK_STR(i) (T_[i] = wall_clock64())
#else
#define RK_STR(i) ((void)0)
#endif

template <int MT>
constexpr size_t stream_red_bytes() { return (size_t)2 * kStreamWaves * MT * 64 * sizeof(f4_t); }
constexpr size_t kStreamXsBytes = (size_t)kStreamMaxGroups * 64 * sizeof(float);  // row sums [group][row]

// grid, prefetch depth and LDS sizes of one shape (K <= 2048): NT tiles per block, D tiles in flight
struct StreamShape {
    int BPC, D, NT, NG;
};
inline StreamShape stream_shape(int N, int K) {
    const int T = (N + 15) / 16;
    const int NT = (T + kStreamBlocks - 1) / kStreamBlocks;
    // every code tile of a block in flight from the start when it has <= 8 (depths 1 2 3 4 6 8 are built)
    const int D = NT <= 4 ? NT : NT <= 6 ? 6 : NT <= 8 ? 8 : 4;
    return {(T + NT - 1) / NT, D, NT, K / 128};
}
template <int MT>
size_t mm_stream_lds_bytes(const StreamShape& sh) {
    return stream_red_bytes<MT>() + kStreamXsBytes + (size_t)sh.NT * MT * 64 * sizeof(f4_t) +
           (size_t)2 * 16 * sh.NT * sh.NG * 2;
}

// Block b: tiles b NT .. b NT + NT - 1 (fewer in the last block) of the T = ceil(N / 16) column tiles.
template <int MT, int D, bool BF16>
__global__ __launch_bounds__(512) void mm_int4_stream_kernel(const uint16_t* __restrict__ X, int ldx,
                                                             const uint8_t* __restrict__ q,
                                                             const uint16_t* __restrict__ sc,
                                                             const uint16_t* __restrict__ mn, void* __restrict__ Y,
                                                             int ydt, int ldy, int M, int N, int K, int NT) {
    extern __shared__ __align__(16) uint8_t smem[];
    f4_t* red = reinterpret_cast<f4_t*>(smem);                                       // [2][8][MT][64]
    float* xsl = reinterpret_cast<float*>(smem + stream_red_bytes<MT>());            // [16][64]
    f4_t* outb = reinterpret_cast<f4_t*>(smem + stream_red_bytes<MT>() + kStreamXsBytes);  // [NT][MT][64]
    uint16_t* tsc = reinterpret_cast<uint16_t*>(outb + (size_t)NT * MT * 64);
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int jn = lane & 15, sq = lane >> 4;
    const int NG = K >> 7, T = (N + 15) >> 4, KB = K >> 1;
    const int b = blockIdx.x, ngc = NG;
    const int t0 = b * NT, ntl = min(NT, T - t0);
    const int wl0 = wave * ngc / kStreamWaves, GW = (wave + 1) * ngc / kStreamWaves - wl0;  // 0, 1 or 2 groups
    const int wg0 = wl0;
    const int rows = min(16 * ntl, N - 16 * t0);                                    // the block's weight rows
    uint16_t* tmn = tsc + rows * ngc;
#ifdef RK_STREAM_TRACE
    uint64_t T_[16] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
#endif
    RK_STR(0);

    // codes of tile i (clamped to the block's last tile); both group slots are always loaded (a wave with fewer
    // groups re-reads its first)
    const int g1 = GW > 1 ? 64 : 0;
    const uint8_t* qb = q + 64 * min(wg0, NG - 1) + 16 * sq;
    auto issue = [&](int i, u4_t (&w)[2]) {
        const int n = min(16 * (t0 + min(i, ntl - 1)) + jn, N - 1);
        const uint8_t* src = qb + (size_t)n * KB;
        w[0] = *reinterpret_cast<const u4_t*>(src);
        w[1] = *reinterpret_cast<const u4_t*>(src + g1);
    };
    // the block's scale / min rows: kStreamTab entries per thread and table (issued before
    // X: they come from HBM, X mostly from the L2)
    uint16_t tv[2][kStreamTab];
#pragma unroll
    for (int k = 0; k < kStreamTab; ++k) {
        const int p = min(tid + 512 * k, rows * ngc - 1);
        const int r = p / ngc, gi = p - r * ngc;
        const size_t o = (size_t)(16 * t0 + r) * NG + gi;
        tv[0][k] = sc[o];
        tv[1][k] = mn[o];
    }
    // X of the wave's groups, raw; lanes of rows past M and waves' absent groups load nothing (zeros)
    u4_t xr[2][MT][4];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
#pragma unroll
            for (int t = 0; t < 4; ++t) xr[i][mt][t] = u4_t{0u, 0u, 0u, 0u};
            if (i < GW && 16 * mt + jn < M) {
                const u4_t* src = reinterpret_cast<const u4_t*>(X + (size_t)(16 * mt + jn) * ldx + 128 * (wg0 + i) + 32 * sq);
#pragma unroll
                for (int t = 0; t < 4; ++t) xr[i][mt][t] = src[t];
            }
        }
    // then the first D tiles' codes (issued after X, so that waiting for X does not wait for them)
    u4_t wq[D][2];
#pragma unroll
    for (int d = 0; d < D; ++d) issue(d, wq[d]);
    RK_STR(1);

    // X fragments, and the rows' sums per group on the matrix cores (X against an all-ones B: exact fp16 products,
    // fp32 sums, in the accumulator layout: lane l holds rows 4 (l / 16) + e) into xsl[local group][row]
    h8_t xf[2][MT][4];
    const h8_t ones = {(_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f,
                       (_Float16)1.f, (_Float16)1.f, (_Float16)1.f, (_Float16)1.f};
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
            f4_t rs = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                xf[i][mt][t] = afrag(xr[i][mt][t], BF16 ? RK_BF16 : RK_F16);
                rs = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[i][mt][t], ones, rs, 0, 0, 0);
            }
            if (i < GW && jn == 0) *reinterpret_cast<f4_t*>(&xsl[(wl0 + i) * 64 + 16 * mt + 4 * sq]) = rs;
        }
    }
    RK_STR(2);
#pragma unroll
    for (int k = 0; k < kStreamTab; ++k) {
        const int p = tid + 512 * k;
        if (p < rows * ngc) {
            tsc[p] = tv[0][k];
            tmn[p] = tv[1][k];
        }
    }
    __syncthreads();  // tables and row sums in LDS
    RK_STR(3);
    // the min term sum_g xs[m][g] min[n][g] of m tile `wave` is added by that wave at the reduction, on the matrix
    // cores in fp32 (v_mfma_f32_16x16x4f32, four groups per instruction: A lane l = xs[row l % 16][group 4 q +
    // l / 16], B lane l = min[column l % 16][group 4 q + l / 16], zero past the last group)
    float xsa[4];
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
        const int gl = 4 * qq + sq;
        xsa[qq] = (wave < MT && gl < ngc) ? xsl[gl * 64 + 16 * min(wave, MT - 1) + jn] : 0.f;
    }

    const DqConsts kc = {opaque(0x000F000Fu), opaque(0x00F000F0u), opaque(0x64006400u)};
    const int steps = (ntl + D - 1) / D * D;  // the last D-step may run up to D - 1 clamped, unstored tiles
    for (int base = 0; base < steps; base += D) {
#pragma unroll
        for (int d = 0; d < D; ++d) {
            const int i = base + d;
            f4_t acc[MT];
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) acc[mt] = f4_t{0.f, 0.f, 0.f, 0.f};
            const int r = min(16 * i + jn, rows - 1);  // this lane's weight row (column of Y) within the block
#pragma unroll
            for (int gi = 0; gi < 2; ++gi) {
                if (gi >= GW) break;
                f4_t c[MT];
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const h8_t Wf = dequant8(wq[d][gi][t], kc);
#pragma unroll
                    for (int mt = 0; mt < MT; ++mt)
                        c[mt] = __builtin_amdgcn_mfma_f32_16x16x32_f16(xf[gi][mt][t], Wf,
                                                                     t == 0 ? f4_t{0.f, 0.f, 0.f, 0.f} : c[mt], 0, 0, 0);
                }
                const float scl = f16_bits_to_f32(tsc[r * ngc + wl0 + gi]);
#pragma unroll
                for (int mt = 0; mt < MT; ++mt)
#pragma unroll
                    for (int e = 0; e < 4; ++e) acc[mt][e] = __builtin_fmaf(c[mt][e], scl, acc[mt][e]);
            }
            issue(i + D, wq[d]);
#ifdef RK_STREAM_TRACE
            if (i == 0) RK_STR(4);
            if (i == 1) RK_STR(6);
            if (i == ntl - 1) RK_STR(8);
#endif
            f4_t* rb = red + (size_t)(i & 1) * kStreamWaves * MT * 64;
#pragma unroll
            for (int mt = 0; mt < MT; ++mt) rb[(wave * MT + mt) * 64 + lane] = acc[mt];
            __syncthreads();
#ifdef RK_STREAM_TRACE
            if (i == 0) RK_STR(5);
            if (i == 1) RK_STR(7);
            if (i == ntl - 1) RK_STR(9);
#endif
            if (wave < MT && i < ntl) {  // 64 MT threads: (m tile = wave, lane), the waves' sums in wave order
                f4_t v = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int qq = 0; qq < 4; ++qq) {
                    const int gl = 4 * qq + sq;
                    const float mnv = gl < ngc ? f16_bits_to_f32(tmn[r * ngc + gl]) : 0.f;
                    v = __builtin_amdgcn_mfma_f32_16x16x4f32(xsa[qq], mnv, v, 0, 0, 0);
                }
#pragma unroll
                for (int w = 0; w < kStreamWaves; ++w) {
                    const f4_t u = rb[(w * MT + wave) * 64 + lane];
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] += u[e];
                }
                outb[(i * MT + wave) * 64 + lane] = v;
            }
        }
    }
    __syncthreads();
    RK_STR(10);
    // the block's tiles as 8-column row pieces: piece (row m, tile i, half h) = Y[m][16 (t0 + i) + 8 h .. + 7];
    // outb[i][mt][lane l][e] holds Y row 16 mt + 4 (l / 16) + e, column 16 (t0 + i) + l % 16
    const bool vec_ok = (((uintptr_t)Y | (size_t)ldy * (ydt == RK_F32 ? 4 : 2)) & (ydt == RK_F32 ? 15 : 7)) == 0;
    for (int it = tid; it < M * ntl * 2; it += 512) {
        const int m = it / (ntl * 2), rest = it - m * ntl * 2, i = rest >> 1, h = rest & 1;
        const int mt = m >> 4, sqm = (m >> 2) & 3, e = m & 3;
        const float* src = reinterpret_cast<const float*>(outb + (size_t)(i * MT + mt) * 64 + 16 * sqm + 8 * h) + e;
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = src[4 * j];
        const int n = 16 * (t0 + i) + 8 * h;
        if (n >= N) continue;
        const size_t o = (size_t)m * ldy + n;
        if (n + 7 < N && vec_ok) {
            if (ydt == RK_F32) {
                *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(Y) + o) = f4_t{v[0], v[1], v[2], v[3]};
                *reinterpret_cast<f4_t*>(reinterpret_cast<float*>(Y) + o + 4) = f4_t{v[4], v[5], v[6], v[7]};
            } else if (ydt == RK_F16) {
                const h8_t hv = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3],
                                 (_Float16)v[4], (_Float16)v[5], (_Float16)v[6], (_Float16)v[7]};
                *reinterpret_cast<h8_t*>(reinterpret_cast<uint16_t*>(Y) + o) = hv;
            } else {
                u4_t bv;
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    bv[j] = (uint32_t)f32_to_bf16_bits(v[2 * j]) | ((uint32_t)f32_to_bf16_bits(v[2 * j + 1]) << 16);
                *reinterpret_cast<u4_t*>(reinterpret_cast<uint16_t*>(Y) + o) = bv;
            }
        } else {
            for (int j = 0; j < 8 && n + j < N; ++j) store_act(Y, ydt, o + j, v[j]);
        }
    }
#ifdef RK_STREAM_TRACE
    RK_STR(11);
    __builtin_amdgcn_s_waitcnt(0);
    RK_STR(12);
    if (g_stream_trace && lane == 0)
        for (int k = 0; k < 16; ++k) g_stream_trace[((size_t)b * kStreamWaves + wave) * 16 + k] = T_[k];
#endif
}

// workspace of the prepared-X plan: Xp (Mp K fp16) then xs (NG Mp fp32)
inline size_t mm_prep_ws_bytes(int M, int K) {
    const size_t Mp = (size_t)(M + 15) / 16 * 16;
    return Mp * (size_t)K * 2 + (size_t)(K / 128) * Mp * 4;
}

template <int MT>
hipError_t launch_mm_prep(const void* X, int xdt, int ldx, const uint8_t* q, const uint16_t* s, const uint16_t* m,
                          void* Y, int ydt, int ldy, int M, int N, int K, void* ws, hipStream_t st) {
    constexpr int BM = 16 * MT;
    const int NG = K / 128, Mp = (M + 15) / 16 * 16;
    uint4* Xp = static_cast<uint4*>(ws);
    float* xs = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + (size_t)Mp * K * 2);
    const dim3 pg((unsigned)(Mp / 16 * NG));  // one block per (m tile, group)
    if (xdt == RK_BF16)
        hipLaunchKernelGGL((mm_xprep_kernel<true>), pg, dim3(256), 0, st, X, ldx, M, Mp, K, Xp, xs);
    else
        hipLaunchKernelGGL((mm_xprep_kernel<false>), pg, dim3(256), 0, st, X, ldx, M, Mp, K, Xp, xs);
    const dim3 grid(((N + 127) / 128) * ((Mp + BM - 1) / BM));
    hipLaunchKernelGGL((mm_int4_prep_kernel<MT>), grid, dim3(512), mm_prep_lds_bytes<MT>(NG), st, Xp, xs, Mp, q, s, m,
                       Y, ydt, ldy, M, N, K);
    return hipGetLastError();
}

// Y[m, n] = sum over splits of part[split][m][n] (fixed order), in Y's dtype
__global__ __launch_bounds__(256) void mm_splitk_reduce(const float* __restrict__ part, int splits,
                                                        void* __restrict__ Y, int ydt, int ldy, int M, int N) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x, MN = (size_t)M * N;
    if (i >= MN) return;
    float v = 0.f;
    for (int k = 0; k < splits; ++k) v += part[k * MN + i];
    store_act(Y, ydt, (i / N) * ldy + i % N, v);
}

// the same four outputs per thread (16-byte loads of each split), for N % 4 == 0 and a 16-byte aligned part
__global__ __launch_bounds__(256) void mm_splitk_reduce4(const float* __restrict__ part, int splits,
                                                         void* __restrict__ Y, int ydt, int ldy, int M, int N) {
    const size_t i = ((size_t)blockIdx.x * 256 + threadIdx.x) * 4, MN = (size_t)M * N;
    if (i >= MN) return;
    f4_t v = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < splits; ++k) {
        const f4_t p = *reinterpret_cast<const f4_t*>(part + k * MN + i);
#pragma unroll
        for (int e = 0; e < 4; ++e) v[e] += p[e];
    }
    const size_t o = (i / N) * ldy + i % N;
#pragma unroll
    for (int e = 0; e < 4; ++e) store_act(Y, ydt, o + e, v[e]);
}

// The wide-wave plan: X prepared into the workspace, then (tile, split) blocks; with splits > 1 the fp32 partial
// sums follow the prepared X in the workspace and mm_splitk_reduce adds them in split order.
size_t mm_wide_part_offset(int M, int K) { return (mm_prep_ws_bytes(M, K) + 255) / 256 * 256; }

hipError_t launch_mm_wide(const void* X, int xdt, int ldx, const uint8_t* q, const uint16_t* s, const uint16_t* m,
                          void* Y, int ydt, int ldy, int M, int N, int K, int splits, void* ws, hipStream_t st) {
    const int NG = K / 128, Mp = (M + 15) / 16 * 16;
    uint4* Xp = static_cast<uint4*>(ws);
    float* xs = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + (size_t)Mp * K * 2);
    const dim3 pg((unsigned)(Mp / 16 * NG));  // one block per (m tile, group)
    if (xdt == RK_BF16)
        hipLaunchKernelGGL((mm_xprep_kernel<true>), pg, dim3(256), 0, st, X, ldx, M, Mp, K, Xp, xs);
    else
        hipLaunchKernelGGL((mm_xprep_kernel<false>), pg, dim3(256), 0, st, X, ldx, M, Mp, K, Xp, xs);
    const int tiles = ((N + 127) / 128) * ((Mp + 127) / 128);
    int g_lo, ngs;
    wide_split(NG, splits, splits - 1, g_lo, ngs);  // the last split has the most groups
    const size_t lds = mm_wide_lds_bytes(ngs);
    if (splits == 1) {
        hipLaunchKernelGGL(mm_int4_wide_kernel, dim3(tiles), dim3(256), lds, st, Xp, xs, Mp, q, s, m, Y, ydt, ldy,
                           M, N, K, 1);
    } else {
        float* part = reinterpret_cast<float*>(static_cast<uint8_t*>(ws) + mm_wide_part_offset(M, K));
        hipLaunchKernelGGL(mm_int4_wide_kernel, dim3(tiles * splits), dim3(256), lds, st, Xp, xs, Mp, q, s, m,
                           (void*)part, (int)RK_F32, N, M, N, K, splits);
        const size_t mn = (size_t)M * N;
        if (N % 4 == 0)
            hipLaunchKernelGGL(mm_splitk_reduce4, dim3((unsigned)((mn / 4 + 255) / 256)), dim3(256), 0, st, part,
                               splits, Y, ydt, ldy, M, N);
        else
            hipLaunchKernelGGL(mm_splitk_reduce, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, part, splits,
                               Y, ydt, ldy, M, N);
    }
    return hipGetLastError();
}

template <int MT, int D>
hipError_t launch_mm_stream_md(const void* X, int xdt, int ldx, const uint8_t* q, const uint16_t* s,
                               const uint16_t* m, void* Y, int ydt, int ldy, int M, int N, int K, hipStream_t st) {
    const StreamShape sh = stream_shape(N, K);
    const size_t lds = mm_stream_lds_bytes<MT>(sh);
    const uint16_t* x = static_cast<const uint16_t*>(X);
    if (xdt == RK_BF16)
        hipLaunchKernelGGL((mm_int4_stream_kernel<MT, D, true>), dim3(sh.BPC), dim3(512), lds, st, x, ldx, q, s, m,
                           Y, ydt, ldy, M, N, K, sh.NT);
    else
        hipLaunchKernelGGL((mm_int4_stream_kernel<MT, D, false>), dim3(sh.BPC), dim3(512), lds, st, x, ldx, q, s, m,
                           Y, ydt, ldy, M, N, K, sh.NT);
    return hipGetLastError();
}

template <int MT>
hipError_t launch_mm_stream_mt(const void* X, int xdt, int ldx, const uint8_t* q, const uint16_t* s,
                               const uint16_t* m, void* Y, int ydt, int ldy, int M, int N, int K, hipStream_t st) {
    switch (stream_shape(N, K).D) {
        case 1: return launch_mm_stream_md<MT, 1>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
        case 2: return launch_mm_stream_md<MT, 2>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
        case 3: return launch_mm_stream_md<MT, 3>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
        case 4: return launch_mm_stream_md<MT, 4>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
        case 6: return launch_mm_stream_md<MT, 6>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
        default: return launch_mm_stream_md<MT, 8>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
    }
}

hipError_t launch_mm_stream(const void* X, int xdt, int ldx, const uint8_t* q, const uint16_t* s, const uint16_t* m,
                            void* Y, int ydt, int ldy, int M, int N, int K, hipStream_t st) {
    if (M <= 16) return launch_mm_stream_mt<1>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
    if (M <= 32) return launch_mm_stream_mt<2>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
    return launch_mm_stream_mt<3>(X, xdt, ldx, q, s, m, Y, ydt, ldy, M, N, K, st);
}

template <int WM, int WN>
size_t mm_lds_bytes(int ng) {  // ng: groups of one block
    constexpr int BM = 2 * WM * 16, BN = 2 * WN * 16;
    return 2 * sizeof(MmStage<BM, BN>) + (size_t)BN * ng * 4;
}

template <int WM, int WN>
hipError_t launch_mm_lds(const void* X, int xdt, int ldx, const uint8_t* q, const uint16_t* s, const uint16_t* m,
                         void* Y, int ydt, int ldy, int M, int N, int K, float* part, int splits, hipStream_t st) {
    constexpr int BM = 2 * WM * 16, BN = 2 * WN * 16;
    const size_t lds = mm_lds_bytes<WM, WN>((K / 128 + splits - 1) / splits);
    dim3 grid(((N + BN - 1) / BN) * ((M + BM - 1) / BM) * splits);
    if (xdt == RK_BF16)
        hipLaunchKernelGGL((mm_int4_lds_kernel<WM, WN, true>), grid, dim3(512), lds, st, X, ldx, q, s, m, Y, ydt, ldy,
                           M, N, K, part, splits);
    else
        hipLaunchKernelGGL((mm_int4_lds_kernel<WM, WN, false>), grid, dim3(512), lds, st, X, ldx, q, s, m, Y, ydt,
                           ldy, M, N, K, part, splits);
    if (splits > 1) {
        const size_t mn = (size_t)M * N;
        hipLaunchKernelGGL(mm_splitk_reduce, dim3((unsigned)((mn + 255) / 256)), dim3(256), 0, st, part, splits, Y,
                           ydt, ldy, M, N);
    }
    return hipGetLastError();
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

namespace {

constexpr size_t kLdsMax = 160 * 1024;

// Kernel choice for one shape. With a caller's workspace (rk_mm_int4_g128_ws) and enough 128-column blocks to give
// most CUs one (cfg 3 / 4 / 5: the prepared-X kernel with 128 / 64 / 48-row blocks; its workspace holds the prepared
// X; cfg 7 ahead of them for M > 64 when K / 128 is even and >= 4: the wide-wave kernel, two blocks per CU, split
// over K when its tiles are few). Otherwise 128 x 128 tiles (cfg 1) when that still gives every CU a block, else 64 x 64 tiles (cfg 2), split
// over K when a workspace or the fixed scratch is allowed and the tiles alone leave CUs idle (each split keeps >= 4
// groups); cfg 0 is the register-staged kernel, for K too long to stage one block's scales in LDS.
struct MmPlan {
    int cfg, splits;
    size_t ws;  // workspace bytes: fp32 partials (cfg 2 with splits > 1) or the prepared X (cfg 3 - 5)
};

enum MmMode { kMmPlain = 0, kMmWorkspace = 1, kMmScratch = 2 };  // rk_mm_int4_g128, _ws, _noalloc
constexpr long kPrepMinBlocks = 160;  // measured: below this the tile kernels' extra blocks win

// M <= 48 and K <= 2048: the stream kernel (cfg 6) when its tables fit in LDS. Longer K was measured split into
// chunks of 16 groups with fp32 partial sums: slower than the tile kernels' split over K (M = 34, 2048 x 11008:
// 17.0 us against 15.3), so those shapes keep the tile plans.
MmPlan mm_stream_plan(int M, int N, int K, int mode) {
    if (M > 48 || K > 128 * kStreamMaxGroups) return {-1, 0, 0};
    const StreamShape sh = stream_shape(N, K);
    const size_t lds = M <= 16 ? mm_stream_lds_bytes<1>(sh) : M <= 32 ? mm_stream_lds_bytes<2>(sh) : mm_stream_lds_bytes<3>(sh);
    if (lds > kLdsMax || 16L * sh.NT * sh.NG > 512L * kStreamTab) return {-1, 0, 0};
    (void)mode;  // no workspace: the same plan for every entry
    return {6, 1, 0};
}

MmPlan mm_plan(int M, int N, int K, int mode);

// The wide-wave plan (cfg 7) for M > 64 and an even group count >= 4: splits over K (whole pairs of groups, >= 4
// groups and <= kWideMaxGroups each) only when the 128 x 128 tiles alone leave the chip's two-blocks-per-CU slots
// mostly idle, M >= 256 and K / 128 > 16; used when tiles x splits reaches kPrepMinBlocks. The workspace holds the prepared X, the partial
// sums when split, and at least what the tile plan that unaligned scale / min arrays fall back to needs.
constexpr long kWideSlots = 512;  // two blocks per CU on 256 CUs
MmPlan mm_wide_plan(int M, int N, int K) {
    const int NG = K / 128, P = NG / 2;
    const long Mp = (M + 15) / 16 * 16;
    const long tiles = (long)((N + 127) / 128) * ((Mp + 127) / 128);
    const int smin = (P + kWideMaxGroups / 2 - 1) / (kWideMaxGroups / 2);
    if (tiles >= kPrepMinBlocks && smin > 1) return {-1, 0, 0};  // enough tiles: no split just to fit the tables
    // few tiles: the split's fp32 partial sums (S x M x N) and the reduce launch paid off only for long K at large M
    // (measured: 512 x 2048 x 11008 58 us against 75 on the tile plan; 512 x 3072 x 2048 34 against 24,
    // 128 x 2048 x 11008 32 against 26)
    if (tiles < kPrepMinBlocks && (M < 256 || NG <= 16)) return {-1, 0, 0};
    int S = smin;
    if (tiles < kPrepMinBlocks) S = std::max<long>(smin, std::min<long>((kWideSlots + tiles / 2) / tiles, P / 2));
    if (S > P / 2 || tiles * S < kPrepMinBlocks) return {-1, 0, 0};
    size_t ws = S > 1 ? mm_wide_part_offset(M, K) + (size_t)S * M * N * sizeof(float) : mm_prep_ws_bytes(M, K);
    ws = std::max(ws, mm_plan(M, N, K, kMmScratch).ws);
    return {7, S, ws};
}

MmPlan mm_plan(int M, int N, int K, int mode) {
    const int NG = K / 128;
    const MmPlan sp = mm_stream_plan(M, N, K, mode);
    if (sp.cfg == 6) return sp;
    if (mode == kMmWorkspace && M > 64 && NG % 2 == 0 && NG >= 4) {
        const MmPlan w = mm_wide_plan(M, N, K);
        if (w.cfg == 7) return w;
    }
    if (mode == kMmWorkspace && ((long)N * NG) % 8 == 0) {
        const int mt = M <= 48 ? 3 : M <= 64 ? 4 : 8;
        const long Mp = (M + 15) / 16 * 16;
        const long blocks = (long)((N + 127) / 128) * ((Mp + 16 * mt - 1) / (16 * mt));
        const size_t lds = mt == 3 ? mm_prep_lds_bytes<3>(NG) : mt == 4 ? mm_prep_lds_bytes<4>(NG) : mm_prep_lds_bytes<8>(NG);
        if (blocks >= kPrepMinBlocks && lds <= kLdsMax) return {mt == 8 ? 3 : mt == 4 ? 4 : 5, 1, mm_prep_ws_bytes(M, K)};
    }
    const bool allow_ws = mode != kMmPlain;
    const long big = (long)((N + 127) / 128) * ((M + 127) / 128);
    if (M > 64 && big >= 256 && mm_lds_bytes<4, 4>(NG) <= kLdsMax) return {1, 1, 0};
    const long small = (long)((N + 63) / 64) * ((M + 63) / 64);
    int splits = 1;
    if (allow_ws && small < 256) splits = (int)std::max(1L, std::min((256 + small - 1) / small, (long)(NG / 4)));
    while (allow_ws && mm_lds_bytes<2, 2>((NG + splits - 1) / splits) > kLdsMax && splits < NG) ++splits;
    if (mm_lds_bytes<2, 2>((NG + splits - 1) / splits) > kLdsMax) return {0, 1, 0};
    return {2, splits, splits > 1 ? (size_t)splits * M * N * sizeof(float) : 0};
}

int mm_check(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale, const uint16_t* min,
             const void* Y, int y_dtype, int ldy, int M, int N, int K) {
    if (!X || !q || !scale || !min || !Y) return RK_ERR_NULL;
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0 || ldx < K || ldy < N) return RK_ERR_SHAPE;
    if (x_dtype != RK_F16 && x_dtype != RK_BF16) return RK_ERR_DTYPE;
    if (y_dtype != RK_F16 && y_dtype != RK_BF16 && y_dtype != RK_F32) return RK_ERR_DTYPE;
    if (((uintptr_t)X & 15) || ((uintptr_t)q & 15) || (ldx % 8)) return RK_ERR_ALIGN;
    return RK_OK;
}

int mm_run(const MmPlan& p, const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
           const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K, void* ws, hipStream_t s) {
    hipError_t e;
    if (p.cfg == 1)
        e = launch_mm_lds<4, 4>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, nullptr, 1, s);
    else if (p.cfg == 2)
        e = launch_mm_lds<2, 2>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, static_cast<float*>(ws),
                                p.splits, s);
    else if (p.cfg == 3)
        e = launch_mm_prep<8>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, ws, s);
    else if (p.cfg == 4)
        e = launch_mm_prep<4>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, ws, s);
    else if (p.cfg == 5)
        e = launch_mm_prep<3>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, ws, s);
    else if (p.cfg == 6)
        e = launch_mm_stream(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, s);
    else if (p.cfg == 7)
        e = launch_mm_wide(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, p.splits, ws, s);
    else
        e = launch_mm<2, 2>(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, s);
    return e == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

}  // namespace

// ---------------------------------------------------------------------------------------------- fixed scratch
// The split-K partial sums of rk_mm_int4_g128_noalloc live here instead of in a caller's workspace: one array per
// GPU, held until the process ends. In host code `scratch` is only a stand-in for the symbol; its device address
// on each GPU comes from hipGetSymbolAddress (scratch_ptr) and only that address is passed to kernels.
static __device__ __align__(256) float scratch[RK_MM_SCRATCH_BYTES / sizeof(float)];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
float* g_scratch[kMaxDevices];  // device address of `scratch` per device (null until that device's first call)

// the current device's address of `scratch`, looked up once per device with that device current
int scratch_ptr(float** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return RK_ERR_LAUNCH;
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch[dev]) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return RK_ERR_LAUNCH;
        g_scratch[dev] = static_cast<float*>(p);
    }
    *out = g_scratch[dev];
    return RK_OK;
}

}  // namespace

extern "C" int rk_mm_int4_g128(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
                               const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K,
                               rk_stream_t stream) {
    const int st = mm_check(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K);
    if (st != RK_OK) return st;
    return mm_run(mm_plan(M, N, K, kMmPlain), X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, nullptr,
                  reinterpret_cast<hipStream_t>(stream));
}

extern "C" int rk_mm_int4_plan(int M, int N, int K, int use_workspace, int* kernel, int* splits) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0) return RK_ERR_SHAPE;
    const MmPlan p = mm_plan(M, N, K, use_workspace != 0 ? kMmWorkspace : kMmPlain);
    static const int kCode[8] = {RK_MM_REGS,   RK_MM_TILE128, RK_MM_TILE64, RK_MM_PREP128,
                                 RK_MM_PREP64, RK_MM_PREP48,  RK_MM_STREAM, RK_MM_WIDE128};
    if (kernel) *kernel = kCode[p.cfg];
    if (splits) *splits = p.splits;
    return RK_OK;
}

extern "C" size_t rk_mm_int4_workspace_bytes(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || K % 128 != 0) return 0;
    return mm_plan(M, N, K, kMmWorkspace).ws;
}

extern "C" int rk_mm_int4_g128_ws(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
                                  const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K,
                                  void* workspace, size_t workspace_bytes, rk_stream_t stream) {
    const int st = mm_check(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K);
    if (st != RK_OK) return st;
    MmPlan p = mm_plan(M, N, K, kMmWorkspace);
    // the prepared-X kernels copy the scale / min rows in 16-byte pieces (the wide-wave kernel in 4-byte pieces);
    // other arrays take the tile plan, whose workspace the plan's size covers
    if (((p.cfg == 3 || p.cfg == 4 || p.cfg == 5) && (((uintptr_t)scale | (uintptr_t)min) & 15)) ||
        (p.cfg == 7 && (((uintptr_t)scale | (uintptr_t)min) & 3)))
        p = mm_plan(M, N, K, kMmScratch);
    if (p.ws > 0 && (!workspace || workspace_bytes < p.ws)) return RK_ERR_SHAPE;
    if (p.ws > 0 && ((uintptr_t)workspace & 15)) return RK_ERR_ALIGN;
    return mm_run(p, X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, workspace,
                  reinterpret_cast<hipStream_t>(stream));
}

extern "C" int rk_mm_int4_g128_noalloc(const void* X, int x_dtype, int ldx, const uint8_t* q, const uint16_t* scale,
                                       const uint16_t* min, void* Y, int y_dtype, int ldy, int M, int N, int K,
                                       rk_stream_t stream) {
    // every check comes before the device is touched: a rejected call launches nothing
    const int st = mm_check(X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K);
    if (st != RK_OK) return st;
    const MmPlan p = mm_plan(M, N, K, kMmScratch);
    if (p.ws > RK_MM_SCRATCH_BYTES) return RK_ERR_SCRATCH;
    float* part = nullptr;
    if (p.ws > 0) {
        const int e = scratch_ptr(&part);
        if (e != RK_OK) return e;
    }
    // the partial sums need no clearing: block (tile, split) writes every (m, n) of its tile for its split before
    // the reduction kernel, ordered after it on the stream, reads them
    return mm_run(p, X, x_dtype, ldx, q, scale, min, Y, y_dtype, ldy, M, N, K, part,
                  reinterpret_cast<hipStream_t>(stream));
}

#ifdef RK_STREAM_TRACE
// trace builds only: the stamp buffer of the stream kernel ([blocks][8][16] uint64, or NULL)
extern "C" __attribute__((visibility("default"))) int rk_stream_trace_set(unsigned long long* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_stream_trace), &buf, sizeof(buf)) == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
#endif
