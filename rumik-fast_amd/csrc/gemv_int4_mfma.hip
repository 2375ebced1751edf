// Batch-1 int4 group-128 GEMV on the matrix cores of gfx950 (the default GEMV path).
//
// y[n] = sum_g ( scale[n,g] * sum_{k in g} code[n,k] x[k] + min[n,g] * sum_{k in g} x[k] )
// (affine identity of the reference, kernels/int4_gemv.py:1-4; its CUDA kernel: kernels/cuda_gemv.py:38-115).
//
// Why MFMA for a GEMV: at ~7 TB/s a SIMD receives ~1 KB of codes every ~360 cycles. Doing the multiply-adds on
// the VALU (v_dot2_f32_f16) costs ~13 VALU ops per 8 codes plus a cross-lane reduction (measured: 129 VALU
// instructions per KB, VALU-bound at ~2.2 TB/s). Here the VALU only dequantizes (9 ops per 8 codes) and
// v_mfma_f32_16x16x32_f16 does the products and the reduction over K; only 1/16 of each MFMA is useful, but the
// matrix pipe has >10x headroom at this arithmetic intensity.
//
// Mapping (v_mfma_f32_16x16x32_f16: A[i][k] in lane i+16*(k/8) element k%8; B[k][j] in lane j+16*(k/8);
// D[i][j] in lane j+16*(i/4) element i%4 — checked on the hardware):
//   * a wave owns a tile of 16 rows; lane l works on row j = l%16 and on the 16-byte quarter s = l/16 of each
//     128-column group: one global_load_dwordx4 per (row, group), so a wave instruction reads 16 rows x 64 B;
//   * the 4 dwords of that quarter are the B fragments of 4 MFMAs (K-slice s): the 1024-magic dequant,
//     (w & 0x000F000F) | 0x64006400 = fp16 (1024 + c0, 1024 + c4), minus 1024 in packed fp16, gives exact codes
//     in the order (c0,c4),(c1,c5),(c2,c6),(c3,c7) (high nibbles: 1024 + 16c, times 1/16 minus 64);
//   * A holds x in the same permuted order, staged once per block in LDS as 16-byte fragments; every A row is
//     the same x, so every lane's D element 0 is its row's dot over the group (no cross-lane reduction);
//   * per group: acc += scale * dot + min * xsum_g, fp32; xsum_g comes from LDS;
//   * KS waves of a block split the groups of the same tile (fills the chip for N = 2048); partial sums are added
//     through LDS, lanes 0..15 of the first wave store.
#include "internal.h"


namespace {

constexpr int kGB = 8;  // groups per load batch (two batches in flight per wave)

// d = (a & mask) | bits. gfx9 VOP3 encodings take no literal constants, so with literal masks the compiler splits
// this into v_and + v_or; with the constants held in VGPRs (see opaque_vgpr) it emits one v_and_or_b32. The
// instruction itself stays compiler-generated, so MFMA/VALU hazard tracking still sees it.
RK_DEV uint32_t and_or(uint32_t a, uint32_t mask, uint32_t bits) { return (a & mask) | bits; }

// a constant the optimizer cannot see through: materialized once in a VGPR
RK_DEV uint32_t opaque_vgpr(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

struct Consts {
    uint32_t lo_mask, hi_mask, magic;
};

// one dword of codes (8 columns) -> B fragment (c0,c4,c1,c5,c2,c6,c3,c7) as exact fp16
RK_DEV h8_t dequant8(uint32_t w, const Consts& k) {
    const h2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    const h2_t s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2_t m64 = {(_Float16)-64.f, (_Float16)-64.f};
    const uint32_t b = w >> 8;
    const h2_t p0 = as_h2(and_or(w, k.lo_mask, k.magic)) + m1024;
    const h2_t p1 = as_h2(and_or(w, k.hi_mask, k.magic)) * s16 + m64;
    const h2_t p2 = as_h2(and_or(b, k.lo_mask, k.magic)) + m1024;
    const h2_t p3 = as_h2(and_or(b, k.hi_mask, k.magic)) * s16 + m64;
    h8_t r;
    r[0] = p0.x; r[1] = p0.y; r[2] = p1.x; r[3] = p1.y;
    r[4] = p2.x; r[5] = p2.y; r[6] = p3.x; r[7] = p3.y;
    return r;
}

// Stage x in LDS: fragment f = g*16 + t*4 + s holds the 8 values of columns 128g + 32s + 8t + (0,4,1,5,2,6,3,7)
// as fp16; xsum[g] = fp32 sum of the group's 128 values. Every thread of the block takes part.
// kXPre 8-column blocks per thread are loaded into registers before the weights (x_issue), so that staging them
// (stage_x) waits for x only: vector-memory results return in issue order. Longer x (more than kXPre blocks per
// thread) is loaded in the staging loop itself.
constexpr int kXPre = 2;

struct XRegs {
    u4_t d[kXPre];
};

RK_DEV void x_issue(const void* __restrict__ x, int K, XRegs& xr) {
    const int nb = K >> 3;
#pragma unroll
    for (int k = 0; k < kXPre; ++k)  // clamped, unconditional: a fixed number of loads in flight
        xr.d[k] = reinterpret_cast<const u4_t*>(x)[min((int)threadIdx.x + k * (int)blockDim.x, nb - 1)];
}

// one 8-column block: fp16 pairs in dequant order (or bf16 converted) + its fp32 sum -> LDS fragment; the
// 16 threads of a group then sum their parts inside a 16-lane DPP row
RK_DEV void stage_block(int i, int nb, int xdt, u4_t d, uint4* __restrict__ frag, float* __restrict__ xsum) {
    // the conversion runs unconditionally (only the LDS writes are guarded): a value used only under i < nb would let
    // the compiler sink its load behind the weight loads, and the staging would then wait for all of them
    const bool ok = i < nb;
    float sum = 0.f;
    uint32_t h[4];
    const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
    if (xdt == RK_BF16) {
        float f[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            f[2 * e] = __builtin_bit_cast(float, d[e] << 16);
            f[2 * e + 1] = __builtin_bit_cast(float, d[e] & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += f[e];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            h2_t p;
            p.x = (_Float16)f[e];
            p.y = (_Float16)f[e + 4];
            h[e] = as_u32(p);
        }
    } else {
        h[0] = perm(d.z, d.x, 0x05040100u);  // (x0, x4)
        h[1] = perm(d.z, d.x, 0x07060302u);  // (x1, x5)
        h[2] = perm(d.w, d.y, 0x05040100u);  // (x2, x6)
        h[3] = perm(d.w, d.y, 0x07060302u);  // (x3, x7)
#pragma unroll
        for (int e = 0; e < 4; ++e) sum = dot2(as_h2(d[e]), one, sum);
    }
    const int g = i >> 4, r = i & 15;  // column offset in the group: 8r = 32s + 8t
    const int s = r >> 2, t = r & 3;
    if (ok) frag[g * 16 + t * 4 + s] = make_uint4(h[0], h[1], h[2], h[3]);
    sum = ok ? sum : 0.f;
    sum += dpp<0x128>(sum);  // 16 consecutive threads hold one group: sum inside their 16-lane DPP row (row_ror:8)
    sum += dpp<0x124>(sum);  // row_ror:4
    sum += dpp<0x122>(sum);  // row_ror:2
    sum += dpp<0x121>(sum);  // row_ror:1
    if (ok && (i & 15) == 0) xsum[i >> 4] = sum;
}

// XREG (K / 8 <= kXPre * blockDim, chosen on the host): every block of x is in registers already. It is a template
// parameter so that the x loads are not sunk into a branch behind the weight loads.
template <bool XREG>
RK_DEV void stage_x(const void* __restrict__ x, int xdt, int K, const XRegs& xr, uint4* __restrict__ frag,
                    float* __restrict__ xsum) {
    const int nb = K >> 3;  // 8-column blocks
    if constexpr (XREG) {
        stage_block(threadIdx.x, nb, xdt, xr.d[0], frag, xsum);  // unguarded: its x load stays ahead of the weights
#pragma unroll
        for (int k = 1; k < kXPre; ++k)
            if (k * (int)blockDim.x < nb) stage_block(threadIdx.x + k * blockDim.x, nb, xdt, xr.d[k], frag, xsum);
    } else {
        for (int base = 0; base < nb; base += blockDim.x) {
            const int i = base + threadIdx.x;
            const u4_t d = i < nb ? reinterpret_cast<const u4_t*>(x)[i] : u4_t{0u, 0u, 0u, 0u};
            stage_block(i, nb, xdt, d, frag, xsum);
        }
    }
}

// codes and scales of up to kGB consecutive groups of one lane's row
struct Batch {
    u4_t w[kGB];
    uint16_t sv[kGB], mv[kGB];
};

// VEC_SM (16-byte aligned rows and batch starts, every batch full): one load for 8 scales, one for 8 mins
template <bool VEC_SM>
RK_DEV void load_batch_sm(Batch& b, const uint16_t* srow, const uint16_t* mrow, int gb, int g1) {
    if constexpr (VEC_SM) {
        const u4_t s8 = *reinterpret_cast<const u4_t*>(srow + gb);
        const u4_t m8 = *reinterpret_cast<const u4_t*>(mrow + gb);
#pragma unroll
        for (int e = 0; e < kGB; ++e) {
            b.sv[e] = (uint16_t)(s8[e >> 1] >> (16 * (e & 1)));
            b.mv[e] = (uint16_t)(m8[e >> 1] >> (16 * (e & 1)));
        }
    } else {
#pragma unroll
        for (int e = 0; e < kGB; ++e) {
            const int g = min(gb + e, g1 - 1);
            b.sv[e] = srow[g];
            b.mv[e] = mrow[g];
        }
    }
}

// Scales / mins first, then the codes in group order: the compute of group e then waits only for the loads up to
// its own (results return in issue order), so it starts while later groups are still in flight. Groups past g1
// reload group g1 - 1 (fixed load count; their results are never used).
template <bool VEC_SM>
RK_DEV void load_batch(Batch& b, const uint8_t* qrow, const uint16_t* srow, const uint16_t* mrow, int gb, int g1) {
    load_batch_sm<VEC_SM>(b, srow, mrow, gb, g1);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order: scales before codes
#pragma unroll
    for (int e = 0; e < kGB; ++e) {
        const int g = min(gb + e, g1 - 1);
        // plain (cached) loads: an instruction covers half of each row's 128-byte line and the next group's load the
        // other half, which then comes from L2 (measured faster than non-temporal loads)
        b.w[e] = *reinterpret_cast<const u4_t*>(qrow + (size_t)g * 64);
    }
}

// dequant + 4 MFMAs per group (each group waits only for its own codes; the next group's x fragments are read from
// LDS while the current group's MFMAs run), then the group affines into acc once the batch's scales / mins are in
// (whatever order the compiler issued them in): acc += scale * dot + min * xsum_g. FULL batches have no per-group
// checks.
template <bool FULL>
RK_DEV void compute_batch(const Batch& b, const uint4* frag, const float* xsum, int s, int gb, int g1,
                          const Consts& kc, float& acc) {
    float dg[kGB];
    h8_t A[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) A[t] = __builtin_bit_cast(h8_t, frag[min(gb, g1 - 1) * 16 + t * 4 + s]);
#pragma unroll
    for (int e = 0; e < kGB; ++e) {
        const int g = gb + e;
        h8_t An[4];
        if (e + 1 < kGB) {
#pragma unroll
            for (int t = 0; t < 4; ++t) An[t] = __builtin_bit_cast(h8_t, frag[min(g + 1, g1 - 1) * 16 + t * 4 + s]);
        }
        dg[e] = 0.f;
        if (FULL || g < g1) {
            f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t = 0; t < 4; ++t)
                d = __builtin_amdgcn_mfma_f32_16x16x32_f16(A[t], dequant8(b.w[e][t], kc), d, 0, 0, 0);
            dg[e] = d[0];
        }
        if (e + 1 < kGB) {
#pragma unroll
            for (int t = 0; t < 4; ++t) A[t] = An[t];
        }
    }
#pragma unroll
    for (int e = 0; e < kGB; ++e) {
        const int g = gb + e;
        if (FULL || g < g1) {
            acc = __builtin_fmaf(dg[e], f16_bits_to_f32(b.sv[e]), __builtin_fmaf(f16_bits_to_f32(b.mv[e]), xsum[g], acc));
        }
    }
}

// the value an output of dtype dt holds for v (what a later kernel reading it back would see)
RK_DEV float round_as(int dt, float v) {
    if (dt == RK_F16) return f16_bits_to_f32(f32_to_f16_bits(v));
    if (dt == RK_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    return v;
}

// Rows: the first `plain` rows of the matrix are ordinary outputs y[r]; with inter > 0 they are followed by
// `inter` gate rows and `inter` up rows, and tile plain_tiles + t holds gate rows 8t .. 8t+7 in its rows 0..7 and
// the matching up rows in rows 8..15, so its epilogue writes act[8t + j] = silu(gate) * up (the gate and up values
// rounded to ydt first, as a separate SiLU kernel reading them back would see them).
// 3 waves per SIMD (<= 168 VGPRs): the 688 blocks of the gate+up projection are all resident at once.
// PAIRED: the instance with gate / up tiles (a kernel of its own, so profiles tell the two launches apart).
template <int KS, bool VEC_SM, bool XREG, bool PAIRED>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(3))) void gemv_int4_mfma_kernel(const void* __restrict__ x, int xdt,
                                                              const uint8_t* __restrict__ q,
                                                              const uint16_t* __restrict__ sc,
                                                              const uint16_t* __restrict__ mn,
                                                              void* __restrict__ y, int ydt, int plain, int inter,
                                                              void* __restrict__ act, int K) {
    extern __shared__ __align__(16) uint8_t smem[];
    const int NG = K >> 7;
    uint4* frag = reinterpret_cast<uint4*>(smem);
    float* xsum = reinterpret_cast<float*>(smem + (size_t)K * 2);
    float* red = xsum + NG;  // [waves][16]

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int team = wave / KS, kw = wave - team * KS;
    const int teams = blockDim.x / (64 * KS);
    const int tile = blockIdx.x * teams + team;
    const int j = lane & 15, s = lane >> 4;
    const int plain_tiles = (plain + 15) / 16;
    const bool paired = PAIRED && tile >= plain_tiles;  // wave-uniform
    const int pc = min(8 * (tile - plain_tiles) + (j & 7), inter - 1);  // channel of a paired tile's row j
    // rows past the end re-read the last row of their part; never stored
    const int row = !paired ? min(tile * 16 + j, plain - 1) : plain + (j < 8 ? pc : inter + pc);
    const int gpw = (NG + KS - 1) / KS;         // groups per wave
    const int g0 = kw * gpw, g1 = min(NG, g0 + gpw);
    const uint8_t* qrow = q + (size_t)row * (size_t)(K >> 1) + 16 * s;
    const uint16_t* srow = sc + (size_t)row * NG;
    const uint16_t* mrow = mn + (size_t)row * NG;

    // x, then the first batch of scales and codes: the HBM latency of the weights overlaps the staging of x
    XRegs xr;
    if constexpr (XREG) x_issue(x, K, xr);
    __builtin_amdgcn_sched_barrier(0);  // keep the issue order: x before the weights
    Batch cur;
    load_batch<VEC_SM>(cur, qrow, srow, mrow, g0, g1);

    stage_x<XREG>(x, xdt, K, xr, frag, xsum);
    __syncthreads();

    const Consts kc = {opaque_vgpr(0x000F000Fu), opaque_vgpr(0x00F000F0u), opaque_vgpr(0x64006400u)};
    float acc = 0.f;
    if (g1 - g0 == kGB) {  // wave-uniform: one full batch, nothing more to load (straight-line waits)
        compute_batch<true>(cur, frag, xsum, s, g0, g1, kc, acc);
    } else for (int gb = g0; gb < g1; gb += kGB) {
        Batch nxt;
        const bool more = gb + kGB < g1;
        if (more) load_batch<VEC_SM>(nxt, qrow, srow, mrow, gb + kGB, g1);  // prefetch while computing
        if (gb + kGB <= g1) compute_batch<true>(cur, frag, xsum, s, gb, g1, kc, acc);
        else compute_batch<false>(cur, frag, xsum, s, gb, g1, kc, acc);
        if (more) cur = nxt;
    }

    // ---- combine the KS partial sums of the tile, lanes 0..15 store their row
    auto out = [&](float v) {  // lanes 0..15 of one wave, all active
        if (!paired) {
            const int r = tile * 16 + j;
            if (r < plain) store_act(y, ydt, (size_t)r, v);
        } else {
            const float u = round_as(ydt, __shfl_down(v, 8, 16));  // up row j + 8 -> lane j
            const float g = round_as(ydt, v);
            const int c = 8 * (tile - plain_tiles) + j;
            if (j < 8 && c < inter) store_act(act, ydt, (size_t)c, g / (1.0f + __expf(-g)) * u);
        }
    };
    if constexpr (KS == 1) {
        if (lane < 16) out(acc);
    } else {
        if (lane < 16) red[wave * 16 + lane] = acc;
        __syncthreads();
        if (kw == 0 && lane < 16) {
            float v = 0.f;
#pragma unroll
            for (int k = 0; k < KS; ++k) v += red[(team * KS + k) * 16 + lane];
            out(v);
        }
    }
}

template <int KS, bool VEC>
hipError_t launch_mfma(const void* x, int xdt, const uint8_t* q, const uint16_t* s, const uint16_t* m, void* y,
                       int ydt, int plain, int inter, void* act, int K, int teams, hipStream_t st) {
    const int tiles = (plain + 15) / 16 + (inter + 7) / 8;
    const int blocks = (tiles + teams - 1) / teams;
    const int threads = 64 * KS * teams;
    const size_t lds = (size_t)K * 2 + (size_t)(K / 128) * 4 + (size_t)teams * KS * 16 * 4;
#define RK_LAUNCH(XR, PR)                                                                                          \
    hipLaunchKernelGGL((gemv_int4_mfma_kernel<KS, VEC, XR, PR>), dim3(blocks), dim3(threads), lds, st, x, xdt, q, s, \
                       m, y, ydt, plain, inter, act, K)
    const bool xreg = K / 8 <= kXPre * threads;
    if (inter > 0) {
        if (xreg) RK_LAUNCH(true, true); else RK_LAUNCH(false, true);
    } else {
        if (xreg) RK_LAUNCH(true, false); else RK_LAUNCH(false, false);
    }
#undef RK_LAUNCH
    return hipGetLastError();
}

}  // namespace

// KS (waves per 16-row tile) and teams (tiles per block) for one call; blocks are 4 waves (KS * teams = 4, or
// the caller's `waves` when that is smaller). Default KS: the largest that leaves every wave at least 6 of the
// row's 128-column groups. Measured (16 rotated copies, hipGraph): 6-8 groups per wave (one load batch of kGB) are
// the fast range; 4 per wave and 16 or more per wave are both slow -- N = 8192 K = 2048 8.8 us with 4 per wave,
// 3.9 with 8; N = 32768 K = 2048 19.4 us with 16, 8.7 with 8; N = 16384 K = 4096 10.9 with 16, 8.8 with 8;
// N = 8192 K = 3072 7.7 with 6, 8.6 with 12; N = 22016 / 25088 K = 2048 (8 per wave) unchanged.
static void plan_mfma(int tiles, int K, int waves, int* ks_out, int* teams_out) {
    (void)tiles;
    const int NG = K / 128;
    const int w = waves ? waves : 4;
    int ks = 1;
    while (ks < w && ks * 2 <= NG && NG / (ks * 2) >= 6) ks *= 2;
    *ks_out = ks;
    *teams_out = w / ks;
}

static int gemv_mfma_run(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale, const uint16_t* min,
                         void* y, int y_dtype, int plain, int inter, void* act, int K, int waves, hipStream_t s) {
    if (K <= 0 || K % 128 != 0) return RK_ERR_SHAPE;
    if (x_dtype != RK_F16 && x_dtype != RK_BF16) return RK_ERR_DTYPE;
    if (y_dtype != RK_F16 && y_dtype != RK_BF16 && y_dtype != RK_F32) return RK_ERR_DTYPE;
    if (((uintptr_t)x & 15) || ((uintptr_t)q & 15)) return RK_ERR_ALIGN;
    if (waves && !(waves == 1 || waves == 2 || waves == 4 || waves == 8 || waves == 16)) return RK_ERR_BLOCK;
    if (waves > 4) waves = 4;  // blocks hold at most 4 waves here (each may use up to 168 VGPRs)
    if ((size_t)K * 2 + (size_t)(K / 128) * 4 + 16 * 16 * 4 > 160 * 1024) return RK_ERR_SHAPE;  // x must fit in LDS
    int ks, teams;
    plan_mfma((plain + 15) / 16 + (inter + 7) / 8, K, waves, &ks, &teams);
    const int NG = K / 128;
    // 16-byte scale / min loads need 16-byte aligned rows and batch starts
    const bool vec = NG % 8 == 0 && ((NG + ks - 1) / ks) % 8 == 0 && !((uintptr_t)scale & 15) && !((uintptr_t)min & 15);
    hipError_t e;
#define RK_KS(KK)                                                                                                  \
    case KK:                                                                                                       \
        e = vec ? launch_mfma<KK, true>(x, x_dtype, q, scale, min, y, y_dtype, plain, inter, act, K, teams, s)     \
                : launch_mfma<KK, false>(x, x_dtype, q, scale, min, y, y_dtype, plain, inter, act, K, teams, s);   \
        break;
    switch (ks) {
        RK_KS(1) RK_KS(2) RK_KS(4)
        default: return RK_ERR_BLOCK;
    }
#undef RK_KS
    return e == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

int gemv_int4_mfma_launch(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                          const uint16_t* min, void* y, int y_dtype, int N, int K, int waves, rk_stream_t stream) {
    if (!x || !q || !scale || !min || !y) return RK_ERR_NULL;
    if (N <= 0) return RK_ERR_SHAPE;
    return gemv_mfma_run(x, x_dtype, q, scale, min, y, y_dtype, N, 0, nullptr, K, waves,
                         reinterpret_cast<hipStream_t>(stream));
}

extern "C" int rk_gemv_int4_g128_silu(const void* x, int x_dtype, const uint8_t* q, const uint16_t* scale,
                                      const uint16_t* min, void* y, void* act, int y_dtype, int n_plain, int inter,
                                      int K, int waves, rk_stream_t stream) {
    if (!x || !q || !scale || !min || !act || (n_plain > 0 && !y)) return RK_ERR_NULL;
    if (n_plain < 0 || inter <= 0) return RK_ERR_SHAPE;
    return gemv_mfma_run(x, x_dtype, q, scale, min, y, y_dtype, n_plain, inter, act, K, waves,
                         reinterpret_cast<hipStream_t>(stream));
}
