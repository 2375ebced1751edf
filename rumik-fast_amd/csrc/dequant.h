// Exact int4 / int8 dequantization and small dot-product building blocks shared by the GEMV kernels, the prefill
// and the persistent decode kernel.
#pragma once

#include "common.h"

// A constant the optimizer cannot see through, materialized once in a VGPR. gfx9 VOP3 encodings take no literal
// operands, so (a & mask) | bits with literal masks becomes v_and + v_or; with the masks in VGPRs the compiler
// emits a single v_and_or_b32.
RK_DEV uint32_t opaque_vgpr(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

struct Int4Masks {
    uint32_t lo, hi, magic, magic64;
};

RK_DEV Int4Masks int4_masks() {
    return {opaque_vgpr(0x000F000Fu), opaque_vgpr(0x00F000F0u), opaque_vgpr(0x64006400u), opaque_vgpr(0x54005400u)};
}

// One dword of int4 codes (8 columns c0..c7, nibble i = column i) -> exact fp16 codes in the order
// (c0,c4),(c1,c5),(c2,c6),(c3,c7): (w & 0x000F000F) | 0x64006400 is the fp16 pair (1024 + c0, 1024 + c4) (1024.0
// has a mantissa LSB worth 1); a packed fp16 add of -1024 leaves the codes. The high nibbles give 1024 + 16c,
// brought back by one exact packed fma (x 1/16, -64).
RK_DEV void dequant_pairs(uint32_t w, const Int4Masks& k, h2_t (&p)[4]) {
    const h2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    const h2_t s16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const h2_t m64 = {(_Float16)-64.f, (_Float16)-64.f};
    const uint32_t b = w >> 8;
    p[0] = as_h2((w & k.lo) | k.magic) + m1024;
    p[1] = as_h2((w & k.hi) | k.magic) * s16 + m64;
    p[2] = as_h2((b & k.lo) | k.magic) + m1024;
    p[3] = as_h2((b & k.hi) | k.magic) * s16 + m64;
}

// the same as an MFMA B fragment (8 fp16)
RK_DEV h8_t dequant_frag(uint32_t w, const Int4Masks& k) {
    h2_t p[4];
    dequant_pairs(w, k, p);
    h8_t r;
    r[0] = p[0].x; r[1] = p[0].y; r[2] = p[1].x; r[3] = p[1].y;
    r[4] = p[2].x; r[5] = p[2].y; r[6] = p[3].x; r[7] = p[3].y;
    return r;
}

// The MFMA B fragment with the high-nibble codes left biased: (c0, c4), (64 + c1, 64 + c5), (c2, c6),
// (64 + c3, 64 + c7), all exact fp16. A high nibble sits at bits 4..7 of its half, which under the exponent of 64.0
// (0x5400, mantissa LSB worth 1/16) is worth exactly c: one v_and_or per pair, no fix-up (7 VALU per 8 codes
// instead of 9). Against A (the activations in the same order, unscaled) an MFMA gives sum_k x_k c_k +
// 64 sum_{k odd} x_k, the odd columns being those of the high nibbles: the caller subtracts 64 x (the sum of the
// odd-column activations). The products are exact in fp32; the bias is about 8x the mean code, so it adds a few
// fp32 ulps of a number of that size to each dot, far below the fp16 rounding of the result.
RK_DEV h8_t dequant_frag_hi64(uint32_t w, const Int4Masks& k) {
    const h2_t m1024 = {(_Float16)-1024.f, (_Float16)-1024.f};
    const uint32_t b = w >> 8;
    const h2_t p0 = as_h2((w & k.lo) | k.magic) + m1024, p1 = as_h2((w & k.hi) | k.magic64);
    const h2_t p2 = as_h2((b & k.lo) | k.magic) + m1024, p3 = as_h2((b & k.hi) | k.magic64);
    h8_t r;
    r[0] = p0.x; r[1] = p0.y; r[2] = p1.x; r[3] = p1.y;
    r[4] = p2.x; r[5] = p2.y; r[6] = p3.x; r[7] = p3.y;
    return r;
}

// 8 consecutive fp16 activations (x0..x7) -> pairs (x0,x4),(x1,x5),(x2,x6),(x3,x7), matching dequant_pairs
RK_DEV void pair_permute(u4_t d, uint32_t (&h)[4]) {
    h[0] = perm(d.z, d.x, 0x05040100u);
    h[1] = perm(d.z, d.x, 0x07060302u);
    h[2] = perm(d.w, d.y, 0x05040100u);
    h[3] = perm(d.w, d.y, 0x07060302u);
}

// sum(code * x) over one 16-byte chunk (32 codes) against its 16 permuted x pairs, fp32 accumulate (v_dot2)
RK_DEV float chunk_dot_int4(u4_t w, const uint32_t* xp, const Int4Masks& k) {
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h2_t p[4];
        dequant_pairs(w[i], k, p);
        a0 = dot2(p[0], as_h2(xp[4 * i + 0]), a0);
        a1 = dot2(p[1], as_h2(xp[4 * i + 1]), a1);
        a0 = dot2(p[2], as_h2(xp[4 * i + 2]), a0);
        a1 = dot2(p[3], as_h2(xp[4 * i + 3]), a1);
    }
    return a0 + a1;
}

// sum(code * x) over one 16-byte chunk of int8 codes (16 columns) against natural fp16 pairs (x0,x1),(x2,x3)...
// Each byte u is placed under 0x64 (fp16 1024 + u) by v_perm_b32; -1152 gives u - 128 exactly. SIGNED codes are
// first mapped to u = b ^ 0x80.
template <bool SIGNED>
RK_DEV float chunk_dot_int8(u4_t w, const uint32_t* xp) {
    const h2_t m1152 = {(_Float16)-1152.f, (_Float16)-1152.f};
    float a0 = 0.f, a1 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        uint32_t v = w[i];
        if constexpr (SIGNED) v ^= 0x80808080u;
        const h2_t c01 = as_h2(perm(0x64646464u, v, 0x04010400u)) + m1152;
        const h2_t c23 = as_h2(perm(0x64646464u, v, 0x04030402u)) + m1152;
        a0 = dot2(c01, as_h2(xp[2 * i]), a0);
        a1 = dot2(c23, as_h2(xp[2 * i + 1]), a1);
    }
    return a0 + a1;
}

// The 32 x values of chunk c (4 x 16 bytes), loaded raw: issued before the weights so that processing them waits for
// x only (vector-memory results return in issue order).
struct XChunk {
    u4_t d[4];
};
RK_DEV void load_x_raw(const void* __restrict__ x, int c, XChunk& xc) {
    const u4_t* xv = reinterpret_cast<const u4_t*>(x) + (size_t)c * 4;
#pragma unroll
    for (int i = 0; i < 4; ++i) xc.d[i] = xv[i];
}

// chunk c's x as 16 fp16 pairs in dequant order, and their fp32 sum
RK_DEV void process_x_chunk(const XChunk& xc, int xdt, uint32_t (&xp)[16], float& xs) {
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        u4_t d = xc.d[i];  // 8 consecutive 16-bit values: d.x = (x0,x1), d.y = (x2,x3), d.z = (x4,x5), d.w = (x6,x7)
        if (xdt == RK_BF16) {
            // bf16 -> fp32 (exact, summed) -> fp16 (round to nearest even) pairs
            float f[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                uint32_t v = d[e];
                f[2 * e] = __builtin_bit_cast(float, v << 16);
                f[2 * e + 1] = __builtin_bit_cast(float, v & 0xffff0000u);
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) s += f[e];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                h2_t p;
                p.x = (_Float16)f[e];
                p.y = (_Float16)f[e + 4];
                xp[4 * i + e] = as_u32(p);
            }
        } else {
            xp[4 * i + 0] = perm(d.z, d.x, 0x05040100u);  // (x0, x4)
            xp[4 * i + 1] = perm(d.z, d.x, 0x07060302u);  // (x1, x5)
            xp[4 * i + 2] = perm(d.w, d.y, 0x05040100u);  // (x2, x6)
            xp[4 * i + 3] = perm(d.w, d.y, 0x07060302u);  // (x3, x7)
            const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) s = dot2(as_h2(d[e]), one, s);
        }
    }
    xs = s;
}
