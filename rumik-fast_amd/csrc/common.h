// Shared device helpers for the gfx950 (CDNA4) kernels of the int4 decode path.
//
// Conventions used by every kernel in this directory:
//   * wave64 only (gfx950); block sizes are multiples of 64;
//   * activations are fp16 or bf16 (dtype code RK_F16 / RK_BF16), outputs fp16 / bf16 / fp32;
//   * the int4 format is the "rumik-int4-g128-minmax-v1" layout: qweight uint8 [N, K/2] with the low nibble
//     holding the even column, scale and min fp16 [N, K/128], w = code * scale + min.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/rumik_hip.h"

typedef _Float16 h2_t __attribute__((ext_vector_type(2)));
typedef _Float16 h4_t __attribute__((ext_vector_type(4)));
typedef _Float16 h8_t __attribute__((ext_vector_type(8)));
typedef float f4_t __attribute__((ext_vector_type(4)));
typedef float f16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u2_t __attribute__((ext_vector_type(2)));

#define RK_DEV __device__ __forceinline__

// ---------------------------------------------------------------- scalar conversions
RK_DEV float bf16_bits_to_f32(uint16_t b) { return __builtin_bit_cast(float, (uint32_t)b << 16); }

// fp32 -> bf16, round to nearest even (NaN kept quiet)
RK_DEV uint16_t f32_to_bf16_bits(float f) {
    uint32_t u = __builtin_bit_cast(uint32_t, f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
    u += 0x7fffu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

RK_DEV float f16_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
RK_DEV uint16_t f32_to_f16_bits(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// element `i` of an activation vector of dtype `dt` (RK_F16 / RK_BF16 / RK_F32) as fp32
RK_DEV float load_act(const void* p, int dt, size_t i) {
    if (dt == RK_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
    if (dt == RK_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

RK_DEV void store_act(void* p, int dt, size_t i, float v) {
    if (dt == RK_F16) ((uint16_t*)p)[i] = f32_to_f16_bits(v);
    else if (dt == RK_BF16) ((uint16_t*)p)[i] = f32_to_bf16_bits(v);
    else ((float*)p)[i] = v;
}

// ---------------------------------------------------------------- packed fp16 helpers
RK_DEV h2_t as_h2(uint32_t v) { return __builtin_bit_cast(h2_t, v); }
RK_DEV uint32_t as_u32(h2_t v) { return __builtin_bit_cast(uint32_t, v); }

// fp32 accumulate of a two-element fp16 dot product (v_dot2_f32_f16)
RK_DEV float dot2(h2_t a, h2_t b, float c) { return __builtin_amdgcn_fdot2(a, b, c, false); }

// byte permute (v_perm_b32): result byte i = byte sel_i of the 8-byte value {hi:lo}
RK_DEV uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) { return __builtin_amdgcn_perm(hi, lo, sel); }

// ---------------------------------------------------------------- cross-row exchange without LDS
// gfx950's v_permlane32_swap exchanges lanes 32..63 of one VGPR with lanes 0..31 of another (v_permlane16_swap:
// the odd 16-lane rows of one with the even rows of the other). With both operands holding v, the two results are
// v's lower and upper half, each in both halves; a + b is then v[i] + v[i ^ 32] in every lane, bit for bit what a
// __shfl_xor exchange gives (IEEE addition commutes), without the LDS round trip of ds_bpermute. Inline asm: this
// compiler's builtin drops the second result when it feeds float arithmetic. The s_nops give the wait states a
// VALU write needs before the swap reads it, and the swap's results before a VALU reads them.
template <int ROWS>
RK_DEV void swap_halves(float v, float& a, float& b) {
    static_assert(ROWS == 16 || ROWS == 32, "16- or 32-lane halves");
    int x = __builtin_bit_cast(int, v), y = x;
    if constexpr (ROWS == 32)
        asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
    else
        asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(x), "+v"(y));
    a = __builtin_bit_cast(float, x);
    b = __builtin_bit_cast(float, y);
}
// v of lane i ^ M for M = 1, 2, 4, 8, 16, 32 from VALU lane moves only (no LDS round trip): DPP quad permutes for
// 1 and 2, row_half_mirror (i -> 7 - i in each 8 lanes) followed by the quad reversal (i -> 3 - i in each 4) for 4,
// row_ror:8 inside the 16-lane rows for 8, and the lane swaps above for 16 and 32 (lane i keeps the half it lacks).
template <int M>
RK_DEV uint32_t xor_lanes(uint32_t v) {
    static_assert(M == 1 || M == 2 || M == 4 || M == 8 || M == 16 || M == 32, "lane distance");
    const int x = (int)v;
    if constexpr (M == 1) return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true);
    if constexpr (M == 2) return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true);
    if constexpr (M == 4)
        return (uint32_t)__builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF,
                                                  true);
    if constexpr (M == 8) return (uint32_t)__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true);
    if constexpr (M >= 16) {
        int a = x, b = x;
        if constexpr (M == 32)
            asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
        else
            asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
        return (uint32_t)((__lane_id() & M) ? a : b);  // a: the lower half's values, b: the upper half's
    }
    return v;
}

template <int M>
RK_DEV float sum_xor(float v) {  // v[i] + v[i ^ M], M = 16 or 32
    float a, b;
    swap_halves<M>(v, a, b);
    return a + b;
}
template <int M>
RK_DEV float max_xor(float v) {  // max(v[i], v[i ^ M]), M = 16 or 32
    float a, b;
    swap_halves<M>(v, a, b);
    return fmaxf(a, b);
}

// ---------------------------------------------------------------- wave64 reductions
// Full-wave sum; every lane ends with the total. Cross-row steps by lane swaps, DPP inside 16-lane rows.
RK_DEV float wave_sum(float v) {
    v = sum_xor<32>(v);
    v = sum_xor<16>(v);
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true));  // row_half_mirror
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true));   // quad xor 2
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true));   // quad xor 1
    v += __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true));  // row_mirror
    return v;
}

RK_DEV float wave_max(float v) {
    v = max_xor<32>(v);
    v = max_xor<16>(v);
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x141, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x4E, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0xB1, 0xF, 0xF, true)));
    v = fmaxf(v, __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), 0x140, 0xF, 0xF, true)));
    return v;
}

// value of another lane through a DPP lane pattern (no LDS traffic)
template <int CTRL>
RK_DEV float dpp(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}

// Exact butterfly partner (lane ^ M), used while rows are still being split between lanes.
template <int M>
RK_DEV float xor_lane(float v) {
    if constexpr (M == 1) return dpp<0xB1>(v);        // quad_perm [1,0,3,2]
    else if constexpr (M == 2) return dpp<0x4E>(v);   // quad_perm [2,3,0,1]
    else return __shfl_xor(v, M);
}

// Partner for a plain-sum step on lane bit log2(M): any lane that differs in that bit and agrees on all higher
// bits works, because the later steps cover the lower bits. Mirrors inside a 16-lane row stay on DPP.
template <int M>
RK_DEV float sum_partner(float v) {
    if constexpr (M == 8) return dpp<0x140>(v);       // row_mirror: lane i <- 15 - i
    else if constexpr (M == 4) return dpp<0x141>(v);  // row_half_mirror: lane i <- 7 - i (inside 8)
    else return xor_lane<M>(v);
}

template <int M, int R>
RK_DEV void reduce_step(float (&v)[R], int& n, int lane) {
    if (n > 1) {
        const int h = n / 2;
        const bool up = (lane & M) != 0;
#pragma unroll
        for (int i = 0; i < R / 2; ++i) {
            if (i < h) {
                // both values first, then the selects: a select between two elements of v itself can be folded
                // into one load at a lane-dependent index, which would move v to scratch memory
                const float lo = v[i], hi = v[i + h];
                const float keep = up ? hi : lo;
                const float send = up ? lo : hi;
                v[i] = keep + xor_lane<M>(send);
            }
        }
        n = h;
    } else {
        v[0] += sum_partner<M>(v[0]);
    }
}

// Reduce R per-lane partial sums (one per row) over the 64 lanes of a wave, R a power of two <= 64.
// Transposed butterfly: during the first log2(R) steps (lane bits 5, 4, ...) a lane keeps half of its remaining
// rows and adds its partner's copy of them, so a wave needs about R + 6 exchanges instead of 6R. On return v[0]
// holds the total of row row_of_lane<R>(lane); writer_lane<R>(r) is the lowest lane holding row r.
template <int R>
RK_DEV void wave_reduce_rows(float (&v)[R]) {
    static_assert(R >= 1 && R <= 64 && (R & (R - 1)) == 0, "R must be a power of two");
    const int lane = threadIdx.x & 63;
    int n = R;
    reduce_step<32>(v, n, lane);
    reduce_step<16>(v, n, lane);
    reduce_step<8>(v, n, lane);
    reduce_step<4>(v, n, lane);
    reduce_step<2>(v, n, lane);
    reduce_step<1>(v, n, lane);
}

// Row whose total lane `lane` holds after wave_reduce_rows<R>: the first log2(R) lane bits from bit 5 downwards,
// most significant first.
template <int R>
RK_DEV int row_of_lane(int lane) {
    int r = 0, n = R;
#pragma unroll
    for (int step = 0; step < 6; ++step) {
        if (n > 1) {
            r = r * 2 + ((lane >> (5 - step)) & 1);
            n /= 2;
        }
    }
    return r;
}

// Lowest lane holding row r's total (the writer lane): inverse of row_of_lane with the remaining bits zero.
template <int R>
RK_DEV int writer_lane(int r) {
    int lane = 0, n = R, bits = 0;
    while (n > 1) { n /= 2; ++bits; }
    for (int b = 0; b < bits; ++b) {
        int bit = (r >> (bits - 1 - b)) & 1;
        lane |= bit << (5 - b);
    }
    return lane;
}
