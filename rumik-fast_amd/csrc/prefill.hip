// Prompt prefill on gfx950: the reference's int4 prefill (engine/rumik_fused.py:54-78) between its mm_int4
// products, for T prompt rows at once:
//   embed_ln_rows   x[t] = dt(emb_q[ids[t]] * emb_s[ids[t]]); h[t] = LN(x[t]) * w      (rumik_int4.py:38-43)
//   post_rows       RoPE on q / k of row t at position p0 + t (interleaved pairs, rumik_int4.py:46-52), K / V
//                   into the layer's cache slot p0 + t, q to q_out, act = silu(gate) * up
//   prefill_attn    causal GQA attention of the T queries over cache slots 0 .. p0 + t (rumik_int4.py:163-171)
//   add_ln_rows     x[t] = dt(x[t] + a[t] + b[t]); h[t] = LN(x[t]) * w (the residual of the parallel block and
//                   the next layer's LayerNorm)
// Every stored activation is rounded once to the activation dtype, as in the decode glue.
//
// prefill_attn on the matrix cores (v_mfma_f32_16x16x32_f16; operand layouts: A[i][k] in lane i + 16 (k / 8),
// element k % 8; B[k][j] in lane j + 16 (k / 8); D[i][j] in lane j + 16 (i / 4), element i % 4). Block = (KV head
// g, a share of its query heads, tile of 16 queries); wave r = the share's head r. Per key block of 32 slots the
// block stages K [32 x 128] and V transposed [128 x 32] in LDS once for its heads; each wave computes S = Q K^T (2 x 4
// MFMAs), the causal mask and an online softmax in log2 units (lazy running max, see the key loop), stores P (fp16,
// the reference's tensor-core PV in 16-bit) to its LDS tile in the A layout and accumulates O += P V (8 MFMAs, fp32).
// The launch time is the longest query tile's key loop, whose steps are bound by the waves' VALU work (one or two
// waves per SIMD), so the loop keeps the per-score instruction count down: the row max is reduced across lanes only
// when a ballot says some score exceeds its row's running max by more than 8 (log2 units, a factor of 256), O is
// rescaled only then, the row sums stay per lane until the loop ends, and the causal mask is applied only on blocks
// that reach past the tile's first query.
#include "common.h"

#include <initializer_list>

namespace {

constexpr int kRowThreads = 256;
constexpr int kMaxPer = 32;  // H <= 8192
constexpr int kHD = 128;
constexpr int kKB = 32;      // keys per block step
constexpr int kQT = 16;      // queries per tile
#ifndef RK_ATTN_KS
#define RK_ATTN_KS 2
#endif
constexpr int kAttnKS = RK_ATTN_KS;  // key groups per attention block up to 384 keys (four past it; <= 4 heads per KV head)

RK_DEV float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

RK_DEV float round_act(float v, int dt) {
    if (dt == RK_F16) return (float)(_Float16)v;
    if (dt == RK_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    return v;
}

// LN of the block's register copy of one row, written to h (d = x - mean, h = d * rsqrt(mean(d^2) + eps) * w)
RK_DEV void ln_row(const float (&xv)[kMaxPer], const void* w, void* h, int dt, int H, float eps, float* red) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
        if (threadIdx.x + k * blockDim.x < (unsigned)H) s += xv[k];
    const float mean = block_sum(s, red) / (float)H;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k)
        if (threadIdx.x + k * blockDim.x < (unsigned)H) {
            const float d = xv[k] - mean;
            ss += d * d;
        }
    const float rstd = 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps);
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        if (i < H) store_act(h, dt, (size_t)i, (xv[k] - mean) * rstd * load_act(w, dt, (size_t)i));
    }
}

__global__ __launch_bounds__(kRowThreads) void embed_ln_rows_kernel(const int64_t* ids, const int8_t* eq,
                                                                    const uint16_t* es, const void* w, void* x,
                                                                    void* h, int dt, int H, float eps) {
    __shared__ float red[16];
    const int t = blockIdx.x;
    const int64_t id = ids[t];
    const float sc = f16_bits_to_f32(es[id]);
    const int8_t* row = eq + (size_t)id * H;
    float xv[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        xv[k] = 0.f;
        if (i < H) {
            xv[k] = round_act((float)row[i] * sc, dt);
            store_act(x, dt, (size_t)t * H + i, xv[k]);
        }
    }
    ln_row(xv, w, (char*)h + (size_t)t * H * (dt == RK_F32 ? 4 : 2), dt, H, eps, red);
}

__global__ __launch_bounds__(kRowThreads) void add_ln_rows_kernel(void* x, const void* a, const void* b,
                                                                  const void* w, void* h, int dt, int H, float eps) {
    __shared__ float red[16];
    const size_t r0 = (size_t)blockIdx.x * H;
    float xv[kMaxPer];
#pragma unroll
    for (int k = 0; k < kMaxPer; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        xv[k] = 0.f;
        if (i < H) {
            float v = load_act(x, dt, r0 + i) + load_act(a, dt, r0 + i);
            if (b) v += load_act(b, dt, r0 + i);
            xv[k] = round_act(v, dt);
            store_act(x, dt, r0 + i, xv[k]);
        }
    }
    ln_row(xv, w, (char*)h + r0 * (dt == RK_F32 ? 4 : 2), dt, H, eps, red);
}

// ---- 16-byte vector forms (fp16 / bf16 with H % 8 == 0 and 16-byte aligned rows): a thread holds 8-column chunks
// c = tid + 256 k of the row; every load of the row is issued before the first use. Same arithmetic as the scalar
// kernels above (sum in fp32, rounded once; LayerNorm statistics in fp32 over the rounded x).
constexpr int kVecPer = 4;  // 8-column chunks per thread: H <= 8192

template <bool BF16>
RK_DEV void unpack8(const u4_t& d, float (&f)[8]) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (BF16) {
            f[2 * e] = __builtin_bit_cast(float, d[e] << 16);
            f[2 * e + 1] = __builtin_bit_cast(float, d[e] & 0xffff0000u);
        } else {
            const h2_t v = as_h2(d[e]);
            f[2 * e] = (float)v.x;
            f[2 * e + 1] = (float)v.y;
        }
    }
}

template <bool BF16>
RK_DEV u4_t pack8(const float (&f)[8]) {
    u4_t d;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if constexpr (BF16)
            d[e] = (uint32_t)f32_to_bf16_bits(f[2 * e]) | ((uint32_t)f32_to_bf16_bits(f[2 * e + 1]) << 16);
        else
            d[e] = (uint32_t)f32_to_f16_bits(f[2 * e]) | ((uint32_t)f32_to_f16_bits(f[2 * e + 1]) << 16);
    }
    return d;
}

// LayerNorm of the thread's chunks (values v, valid chunks c < nc) -> h row (chunk-indexed)
template <bool BF16>
RK_DEV void ln_chunks(float (&v)[kVecPer][8], const u4_t (&wd)[kVecPer], u4_t* __restrict__ h4, int nc, int H,
                      float eps, float* red) {
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kVecPer; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[k][e];  // zero past the row
    const float mean = block_sum(s, red) / (float)H;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kVecPer; ++k)
        if ((int)threadIdx.x + 256 * k < nc)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float d = v[k][e] - mean;
                ss += d * d;
            }
    const float rstd = 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps);
#pragma unroll
    for (int k = 0; k < kVecPer; ++k) {
        const int c = threadIdx.x + 256 * k;
        if (c < nc) {
            float w[8], o[8];
            unpack8<BF16>(wd[k], w);
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = (v[k][e] - mean) * rstd * w[e];
            h4[c] = pack8<BF16>(o);
        }
    }
}

template <bool BF16>
__global__ __launch_bounds__(256) void add_ln_rows_vec_kernel(u4_t* __restrict__ x, const u4_t* __restrict__ a,
                                                              const u4_t* __restrict__ b, const u4_t* __restrict__ w,
                                                              u4_t* __restrict__ h, int H, float eps) {
    __shared__ float red[16];
    const int nc = H >> 3;
    const size_t r0 = (size_t)blockIdx.x * nc;
    u4_t xd[kVecPer], ad[kVecPer], bd[kVecPer], wd[kVecPer];
#pragma unroll
    for (int k = 0; k < kVecPer; ++k) {  // clamped, unconditional loads
        const int c = min((int)threadIdx.x + 256 * k, nc - 1);
        xd[k] = x[r0 + c];
        ad[k] = a[r0 + c];
        bd[k] = b ? b[r0 + c] : u4_t{0u, 0u, 0u, 0u};
        wd[k] = w[c];
    }
    float v[kVecPer][8];
#pragma unroll
    for (int k = 0; k < kVecPer; ++k) {
        const int c = threadIdx.x + 256 * k;
        float fx[8], fa[8], fb[8];
        unpack8<BF16>(xd[k], fx);
        unpack8<BF16>(ad[k], fa);
        unpack8<BF16>(bd[k], fb);
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] = c < nc ? round_act(fx[e] + fa[e] + fb[e], BF16 ? RK_BF16 : RK_F16) : 0.f;
        if (c < nc) x[r0 + c] = pack8<BF16>(v[k]);
    }
    ln_chunks<BF16>(v, wd, h + r0, nc, H, eps, red);
}

template <bool BF16>
__global__ __launch_bounds__(256) void embed_ln_rows_vec_kernel(const int64_t* ids, const int8_t* eq,
                                                                const uint16_t* es, const u4_t* __restrict__ w,
                                                                u4_t* __restrict__ x, u4_t* __restrict__ h, int H,
                                                                float eps) {
    __shared__ float red[16];
    const int nc = H >> 3;
    const size_t r0 = (size_t)blockIdx.x * nc;
    const int64_t id = ids[blockIdx.x];
    const float sc = f16_bits_to_f32(es[id]);
    const uint2* row = reinterpret_cast<const uint2*>(eq + (size_t)id * H);
    uint2 qd[kVecPer];
    u4_t wd[kVecPer];
#pragma unroll
    for (int k = 0; k < kVecPer; ++k) {
        const int c = min((int)threadIdx.x + 256 * k, nc - 1);
        qd[k] = row[c];
        wd[k] = w[c];
    }
    float v[kVecPer][8];
#pragma unroll
    for (int k = 0; k < kVecPer; ++k) {
        const int c = threadIdx.x + 256 * k;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int8_t q = (int8_t)(((e < 4 ? qd[k].x : qd[k].y) >> (8 * (e & 3))) & 0xFF);
            v[k][e] = c < nc ? round_act((float)q * sc, BF16 ? RK_BF16 : RK_F16) : 0.f;
        }
        if (c < nc) x[r0 + c] = pack8<BF16>(v[k]);
    }
    ln_chunks<BF16>(v, wd, h + r0, nc, H, eps, red);
}

// grid (T, NH + 2 NKV + ceil(inter / 256)), 64 threads: block (t, b) as post_kernel of the decode glue for row t
__global__ __launch_bounds__(64) void post_rows_kernel(const void* y, int ldy, int p0, const void* cos_t,
                                                       const void* sin_t, void* kc, void* vc, void* qo, void* act,
                                                       int dt, int NH, int NKV, int HD, int S, int inter, int rope) {
    const int t = blockIdx.x, b = blockIdx.y, tid = threadIdx.x;
    const int pos = p0 + t;
    const size_t yr = (size_t)t * ldy;
    if (b < NH + NKV) {
        for (int j = tid; j < HD / 2; j += 64) {
            const float xe = load_act(y, dt, yr + (size_t)b * HD + 2 * j);
            const float xo = load_act(y, dt, yr + (size_t)b * HD + 2 * j + 1);
            float oe = xe, oo = xo;
            if (rope) {
                const float c = load_act(cos_t, dt, (size_t)pos * HD + 2 * j);
                const float s = load_act(sin_t, dt, (size_t)pos * HD + 2 * j);
                oe = xe * c - xo * s;
                oo = xo * c + xe * s;
            }
            if (b < NH) {
                store_act(qo, dt, (size_t)t * NH * HD + (size_t)b * HD + 2 * j, oe);
                store_act(qo, dt, (size_t)t * NH * HD + (size_t)b * HD + 2 * j + 1, oo);
            } else {
                const size_t c0 = ((size_t)(b - NH) * S + pos) * HD;
                store_act(kc, dt, c0 + 2 * j, oe);
                store_act(kc, dt, c0 + 2 * j + 1, oo);
            }
        }
    } else if (b < NH + 2 * NKV) {
        const int hv = b - NH - NKV;
        for (int j = tid; j < HD; j += 64)
            store_act(vc, dt, ((size_t)hv * S + pos) * HD + j, load_act(y, dt, yr + (size_t)(NH + NKV + hv) * HD + j));
    } else {
        const size_t base = (size_t)(NH + 2 * NKV) * HD;
        for (int c = (b - NH - 2 * NKV) * 256 + tid; c < min(inter, (b - NH - 2 * NKV + 1) * 256); c += 64) {
            const float g = load_act(y, dt, yr + base + c), u = load_act(y, dt, yr + base + inter + c);
            store_act(act, dt, (size_t)t * inter + c, g / (1.0f + __expf(-g)) * u);
        }
    }
}

// post_rows on a 2-D grid (row t, part): one item per thread, so a short prompt still spreads over the chip (one
// block per row left 34 of 256 CUs busy at T = 34, each walking 25k values: 8.5 us). Parts [0, nqk): the q / k heads
// as 32-bit pairs (RoPE), 256 pairs per part; part nqk: v as 8-column chunks; parts after it: silu(gate) * up as
// 8-column chunks, 256 per part. Shapes with HD % 8 == 0, inter % 8 == 0 and 16-byte aligned rows.
constexpr int kPostPart = 256;

__host__ __device__ inline int post_qk_parts(int NH, int NKV, int HD) { return ((NH + NKV) * (HD / 2) + kPostPart - 1) / kPostPart; }
__host__ __device__ inline int post_act_parts(int inter) { return (inter / 8 + kPostPart - 1) / kPostPart; }

template <bool BF16>
__global__ __launch_bounds__(kPostPart) void post_rows_vec_kernel(const uint16_t* __restrict__ y, int ldy, int p0,
                                                                  const uint16_t* __restrict__ cos_t,
                                                                  const uint16_t* __restrict__ sin_t,
                                                                  uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                                  uint16_t* __restrict__ qo, uint16_t* __restrict__ act,
                                                                  int NH, int NKV, int HD, int S, int inter, int rope) {
    const int t = blockIdx.x, part = blockIdx.y, tid = threadIdx.x, pos = p0 + t;
    const uint16_t* yr = y + (size_t)t * ldy;
    const int dt = BF16 ? RK_BF16 : RK_F16;
    const int hp = HD / 2, nqk = post_qk_parts(NH, NKV, HD);
    const u4_t* y4 = reinterpret_cast<const u4_t*>(yr);
    if (part < nqk) {
        const int pi = part * kPostPart + tid;
        if (pi >= (NH + NKV) * hp) return;
        const int hd = pi / hp, j = pi - hd * hp;
        const uint32_t v = *reinterpret_cast<const uint32_t*>(yr + (size_t)hd * HD + 2 * j);
        const float xe = load_act(&v, dt, 0), xo = load_act(&v, dt, 1);
        float oe = xe, oo = xo;
        if (rope) {
            const float c = load_act(cos_t, dt, (size_t)pos * HD + 2 * j);
            const float sn = load_act(sin_t, dt, (size_t)pos * HD + 2 * j);
            oe = xe * c - xo * sn;
            oo = xo * c + xe * sn;
        }
        uint32_t o;
        store_act(&o, dt, 0, oe);
        store_act(&o, dt, 1, oo);
        uint16_t* dst = hd < NH ? qo + (size_t)t * NH * HD + (size_t)hd * HD + 2 * j
                                : kc + ((size_t)(hd - NH) * S + pos) * HD + 2 * j;
        *reinterpret_cast<uint32_t*>(dst) = o;
    } else if (part == nqk) {
        const int vb = (NH + NKV) * HD / 8, nv = NKV * HD / 8;
        for (int c = tid; c < nv; c += kPostPart) {
            const int hv = (8 * c) / HD, off = 8 * c - hv * HD;
            *reinterpret_cast<u4_t*>(vc + ((size_t)hv * S + pos) * HD + off) = y4[vb + c];
        }
    } else {
        const int gb = (NH + 2 * NKV) * HD / 8, ni = inter / 8;
        const int c = (part - nqk - 1) * kPostPart + tid;
        if (c >= ni) return;
        float g[8], u[8], o[8];
        unpack8<BF16>(y4[gb + c], g);
        unpack8<BF16>(y4[gb + ni + c], u);
#pragma unroll
        for (int e = 0; e < 8; ++e) o[e] = g[e] / (1.0f + __expf(-g[e])) * u[e];
        reinterpret_cast<u4_t*>(act + (size_t)t * inter)[c] = pack8<BF16>(o);
    }
}

// all-reduce over the 16 lanes of a DPP row (row_ror 8, 4, 2, 1)
RK_DEV float row16_max(float v) {
    v = fmaxf(v, dpp<0x128>(v));
    v = fmaxf(v, dpp<0x124>(v));
    v = fmaxf(v, dpp<0x122>(v));
    v = fmaxf(v, dpp<0x121>(v));
    return v;
}
RK_DEV float row16_sum(float v) {
    v += dpp<0x128>(v);
    v += dpp<0x124>(v);
    v += dpp<0x122>(v);
    v += dpp<0x121>(v);
    return v;
}

// grid (NKV * (NH / NKV) / REP, ceil(T / 16)), 64 * REP * KS threads: block x = (KV head g, share z) computes query
// heads g (NH / NKV) + z REP .. + REP - 1. q: [T, NH * 128] fp16 (RoPE applied); kc / vc: the layer's cache
// [NKV, S, 128] fp16 holding slots 0 .. p0 + T - 1; o: [T, NH * 128] fp16. Query t attends slots 0 .. p0 + t.
// Wave w = REP ks + r computes the share's query head r over the key blocks ks, ks + KS, ks + 2 KS, ... of the tile's
// range (KS wave groups walk the keys side by side, each with its own online softmax), and the KS partial results
// of a head are merged through LDS at the end. One step stages KS key blocks (one per group) in LDS.
template <int CH>
struct KVChunks {
    u4_t k[CH], v[CH];  // native vectors (HIP's uint4 is a struct with a union, which stays in scratch memory)
};

// Staging of one step's KS key blocks (K rows to Ks, V transposed to Vt[dim][key] so that a 16-byte MFMA fragment
// read holds 8 consecutive keys of one dim; each dim row rotated by 8 ((dim / 8) % 4) keys, vt_col, so the stores
// of one instruction spread over more banks). Slots past `last` re-read slot `last`: every load valid and
// unconditional, so the compiler waits for exactly the chunks it stores; those keys are masked out of S (P = 0).
// Two forms, by the 16-byte chunks (8 dims of one key) a thread holds per step:
// - QUAD (at least 4 chunks): a thread's chunks come as quads, 4 consecutive keys at the same 8 dims (quad qq of key
//   block kb = qd / 128: dims 8 (qq % 16), keys 4 (qq / 16) .. + 3; each of the quad's 4 loads is one 256-byte row
//   per 16 lanes, coalesced), and V goes to Vt as 8-byte words of 4 keys per dim: 8 stores per quad instead of 32
//   2-byte ones (those measured ~0.5 us per step of two key blocks, a third of the step). Vt rows of 80 bytes.
//   (Measured and not kept: lanes along the keys, 16 quads of one dim row per store instruction into unrotated rows,
//   which spreads the stores over all banks but splits every load over 16 half-lines: 15.6 against 14.8 us.)
// - CHUNK (fewer): chunk e (< KS * 512) is key block e / 512, key (e % 512) / 16, dims 8 (e % 16) (16 consecutive
//   lanes: one 256-byte row); V is stored 2 bytes at a time into rows of kKB keys.
constexpr float kLazyMax = 8.f;  // log2 units: a row's running max moves only when exceeded by more than this
constexpr int kKsPad = 8;  // K rows padded by 16 bytes: the QK fragment reads of 16 rows then spread over the banks
constexpr int kChunksPerKB = kKB * kHD / 8;  // 512
constexpr int kVtRow = kKB + 8;     // QUAD: halves per Vt row (80 bytes)
constexpr int kVtBlk = kHD * kVtRow;  // QUAD: halves per key block of Vt (the CHUNK form uses kHD * kKB of them)

// column of key j in transposed row d
RK_DEV int vt_col(int d, int j) { return (j + 8 * ((d >> 3) & 3)) & (kKB - 1); }
// offset in halves of key j of dim row d of Vt key block b (j a multiple of 4 for QUAD, of 8 for CHUNK)
template <bool QUAD>
RK_DEV int vt_off(int b, int d, int j) {
    if constexpr (QUAD)
        return b * kVtBlk + d * kVtRow + vt_col(d, j);
    else
        return (b * kHD + d) * kKB + vt_col(d, j);
}

template <int CH>
RK_DEV void kv_load(const uint16_t* kg, const uint16_t* vg, int s0, int last, KVChunks<CH>& c) {
#pragma unroll
    for (int u = 0; u < CH; ++u) {
        int j, d8;
        if constexpr (CH % 4 == 0) {
            const int qd = threadIdx.x + (u / 4) * blockDim.x, qq = qd % (kChunksPerKB / 4);
            j = (s0 + qd / (kChunksPerKB / 4)) * kKB + 4 * (qq / (kHD / 8)) + u % 4;
            d8 = (qq % (kHD / 8)) * 8;
        } else {
            const int e = threadIdx.x + u * blockDim.x;
            j = (s0 + e / kChunksPerKB) * kKB + (e % kChunksPerKB) / (kHD / 8);
            d8 = (e % (kHD / 8)) * 8;
        }
        c.k[u] = *reinterpret_cast<const u4_t*>(kg + (size_t)min(j, last) * kHD + d8);
        c.v[u] = *reinterpret_cast<const u4_t*>(vg + (size_t)min(j, last) * kHD + d8);
    }
}

template <int CH>
RK_DEV void kv_store(const KVChunks<CH>& c, uint16_t (*Ks)[kKB][kHD + kKsPad], uint16_t* Vt) {
    if constexpr (CH % 4 == 0) {
#pragma unroll
        for (int g = 0; g < CH / 4; ++g) {
            const int qd = threadIdx.x + g * blockDim.x, kb = qd / (kChunksPerKB / 4), qq = qd % (kChunksPerKB / 4);
            const int k4 = 4 * (qq / (kHD / 8)), d8 = (qq % (kHD / 8)) * 8;
#pragma unroll
            for (int u = 0; u < 4; ++u) *reinterpret_cast<u4_t*>(&Ks[kb][k4 + u][d8]) = c.k[4 * g + u];
#pragma unroll
            for (int w = 0; w < 4; ++w) {  // dims d8 + 2w (low halves) and d8 + 2w + 1 (high halves) of the 4 keys
                const uint32_t v0 = c.v[4 * g][w], v1 = c.v[4 * g + 1][w], v2 = c.v[4 * g + 2][w], v3 = c.v[4 * g + 3][w];
                const u2_t lo = {(v0 & 0xFFFFu) | (v1 << 16), (v2 & 0xFFFFu) | (v3 << 16)};
                const u2_t hi = {(v0 >> 16) | (v1 & 0xFFFF0000u), (v2 >> 16) | (v3 & 0xFFFF0000u)};
                *reinterpret_cast<u2_t*>(Vt + vt_off<true>(kb, d8 + 2 * w, k4)) = lo;
                *reinterpret_cast<u2_t*>(Vt + vt_off<true>(kb, d8 + 2 * w + 1, k4)) = hi;
            }
        }
    } else {
#pragma unroll
        for (int u = 0; u < CH; ++u) {
            const int e = threadIdx.x + u * blockDim.x, kb = e / kChunksPerKB, ep = e % kChunksPerKB;
            const int kj = ep / (kHD / 8), d8 = (ep % (kHD / 8)) * 8;
            *reinterpret_cast<u4_t*>(&Ks[kb][kj][d8]) = c.k[u];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                Vt[vt_off<false>(kb, d8 + 2 * w, kj)] = (uint16_t)c.v[u][w];
                Vt[vt_off<false>(kb, d8 + 2 * w + 1, kj)] = (uint16_t)(c.v[u][w] >> 16);
            }
        }
    }
}

// dynamic LDS of prefill_attn_kernel<REP, KS>: the staging (KS key blocks of K and transposed V, one P tile per
// wave), reused after the key loop for the merge (REP partial results of 16 x 128 fp32 plus m / l per row)
constexpr size_t attn_stage_bytes(int REP, int KS) {
    return (size_t)KS * kKB * (kHD + kKsPad) * 2 + (size_t)KS * kVtBlk * 2 + (size_t)REP * KS * kQT * kKB * 2;
}
constexpr size_t attn_merge_bytes(int REP) { return (size_t)REP * (64 * 32 + 2 * kQT) * 4; }
constexpr size_t attn_lds_bytes(int REP, int KS) {
    return attn_stage_bytes(REP, KS) > attn_merge_bytes(REP) ? attn_stage_bytes(REP, KS) : attn_merge_bytes(REP);
}

template <int REP, int KS>
__global__ __launch_bounds__(64 * REP * KS) __attribute__((amdgpu_waves_per_eu(1, 1))) void prefill_attn_kernel(const uint16_t* q, const uint16_t* kc,
                                                                      const uint16_t* vc, uint16_t* o, int T, int p0,
                                                                      int NH, int NKV, int S, float scale) {
    // REP: the query heads of one KV head this block computes (all NH / NKV of them, or a share: blockIdx.x then
    // names the KV head and the share)
    constexpr int CH = KS * kChunksPerKB / (64 * REP * KS);
    extern __shared__ __align__(16) uint8_t lds[];
    auto Ks = reinterpret_cast<uint16_t(*)[kKB][kHD + kKsPad]>(lds);
    constexpr bool QUAD = CH % 4 == 0;
    uint16_t* Vt = reinterpret_cast<uint16_t*>(lds + (size_t)KS * kKB * (kHD + kKsPad) * 2);
    uint16_t* Ps = reinterpret_cast<uint16_t*>(lds + (size_t)KS * kKB * (kHD + kKsPad) * 2 + (size_t)KS * kVtBlk * 2);
    const int shares = NH / NKV / REP;
    const int g = blockIdx.x / shares, q0 = blockIdx.y * kQT;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int r = w % REP, ks = w / REP;
    const int h = g * (NH / NKV) + (blockIdx.x % shares) * REP + r;
    const int li = lane & 15, lq = lane >> 4;  // A / B fragment: row or column li, k-group lq
    const float sl2 = scale * 1.44269504088896341f;  // scores in log2 units: P = 2^(s sl2 - m)
    const int ldq = NH * kHD;
    uint16_t* P = Ps + w * kQT * kKB;
    // Q fragments of this wave's head: query q0 + li, dims 32c + 8 lq .. + 8
    h8_t Qf[4];
    {
        const int qi = min(q0 + li, T - 1);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            Qf[c] = __builtin_bit_cast(h8_t, *reinterpret_cast<const uint4*>(q + (size_t)qi * ldq + h * kHD + 32 * c + 8 * lq));
    }
    // the Q loads go out before the K / V prefetch: results return in issue order, so the first step's S = Q K^T then
    // waits only for its own K / V block, not for the second set behind it
    __builtin_amdgcn_sched_barrier(0);
    f4_t O[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) O[c] = f4_t{0.f, 0.f, 0.f, 0.f};
    float m[4], l[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        m[e] = -INFINITY;
        l[e] = 0.f;
    }
    const uint16_t* kg = kc + (size_t)g * S * kHD;
    const uint16_t* vg = vc + (size_t)g * S * kHD;
    const int last = p0 + min(q0 + kQT, T) - 1;  // the last slot any query of the tile sees
    const int kb0 = 0, kb1 = last / kKB + 1;      // the tile's key blocks
    const int nsteps = (kb1 - kb0 + KS - 1) / KS;  // steps of KS key blocks
    // K / V of the next two steps are in flight in registers while a step is computed: set A holds the even steps,
    // set B the odd ones (the loop is unrolled by two so that neither is copied)
    KVChunks<CH> ka, kb;
    kv_load<CH>(kg, vg, kb0, last, ka);
    __builtin_amdgcn_sched_barrier(0);  // set A issued before set B (the order the steps consume them in)
    kv_load<CH>(kg, vg, kb0 + KS, last, kb);
    // one step (a macro, not a lambda: the register sets must stay promotable to registers). (Measured and not kept: a
    // double-buffered staging with one barrier per step, each wave storing step st + 1 while computing step st: no
    // faster, 15.1 against 14.8 us; the step is bound by the waves' own LDS traffic, not by the barrier.)
#define RK_ATTN_STEP(st, cur) \
    __syncthreads();  /* the previous step's K / V are no longer read */ \
    kv_store<CH>(cur, Ks, Vt); \
    __syncthreads(); \
    kv_load<CH>(kg, vg, kb0 + ((st) + 2) * KS, last, cur);  /* two steps ahead (clamped past the end) */ \
    if (kb0 + (st) * KS + ks < kb1) {  /* wave-uniform: this group's key block of the step exists */ \
        const int j0 = (kb0 + (st) * KS + ks) * kKB; \
        /* S = Q K^T for keys j0 + 16 hf + li (D layout: row 4 lq + e, key li) */ \
        /* all 8 K fragments are read before the first MFMA (the reads' latencies overlap instead of adding up) */ \
        h8_t Bk[2][4]; \
_Pragma("unroll") \
        for (int hf = 0; hf < 2; ++hf) \
_Pragma("unroll") \
            for (int c = 0; c < 4; ++c) \
                Bk[hf][c] = __builtin_bit_cast(h8_t, *reinterpret_cast<const uint4*>(&Ks[ks][16 * hf + li][32 * c + 8 * lq])); \
        __builtin_amdgcn_sched_group_barrier(0x100, 8, 0); \
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0); \
        f4_t Sd[2]; \
_Pragma("unroll") \
        for (int hf = 0; hf < 2; ++hf) { \
            f4_t d = {0.f, 0.f, 0.f, 0.f}; \
_Pragma("unroll") \
            for (int c = 0; c < 4; ++c) d = __builtin_amdgcn_mfma_f32_16x16x32_f16(Qf[c], Bk[hf][c], d, 0, 0, 0); \
            Sd[hf] = d; \
        } \
        /* scores in log2 units (scale * log2 e folded in); the causal mask only on blocks that reach past the */ \
        /* tile's first query (wave-uniform). Lazy running max: a row's m moves only when one of the block's */ \
        /* scores exceeds it by more than kLazyMax, so P = 2^(s - m) <= 2^kLazyMax (fp16 holds it at the same */ \
        /* relative precision); a lane-local compare and one ballot decide, and only then are the row maxima */ \
        /* reduced and O rescaled. l holds per-lane partial sums (reduced across the row after the key loop). */ \
        const bool diag = j0 + kKB - 1 > p0 + q0; \
        float sc0[4], sc1[4]; \
        bool big = false; \
_Pragma("unroll") \
        for (int e = 0; e < 4; ++e) { \
            sc0[e] = Sd[0][e] * sl2; \
            sc1[e] = Sd[1][e] * sl2; \
            if (diag) { \
                const int qpos = p0 + q0 + 4 * lq + e; \
                if (j0 + li > qpos) sc0[e] = -INFINITY; \
                if (j0 + 16 + li > qpos) sc1[e] = -INFINITY; \
            } \
            big = big || fmaxf(sc0[e], sc1[e]) > m[e] + kLazyMax; /* never for a masked score */ \
        } \
        float alpha[4] = {1.f, 1.f, 1.f, 1.f}; \
        const bool moved = __any(big); \
        if (moved) { \
_Pragma("unroll") \
            for (int e = 0; e < 4; ++e) { \
                const float mb = row16_max(fmaxf(sc0[e], sc1[e])); \
                if (mb > m[e] + kLazyMax) { \
                    alpha[e] = __builtin_amdgcn_exp2f(m[e] - mb);  /* m = -inf: 0 (O and l are still 0) */ \
                    m[e] = mb; \
                } \
            } \
        } \
_Pragma("unroll") \
        for (int e = 0; e < 4; ++e) { \
            const float p0v = m[e] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc0[e] - m[e]); \
            const float p1v = m[e] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sc1[e] - m[e]); \
            const _Float16 h0 = (_Float16)p0v, h1 = (_Float16)p1v; \
            l[e] = l[e] * alpha[e] + ((float)h0 + (float)h1); \
            P[(4 * lq + e) * kKB + li] = __builtin_bit_cast(uint16_t, h0); \
            P[(4 * lq + e) * kKB + 16 + li] = __builtin_bit_cast(uint16_t, h1); \
        } \
        if (moved) { \
_Pragma("unroll") \
            for (int c = 0; c < 8; ++c) \
_Pragma("unroll") \
                for (int e = 0; e < 4; ++e) O[c][e] *= alpha[e]; \
        } \
        __builtin_amdgcn_wave_barrier(); \
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront"); \
        /* O += P V: A = P[query li][keys 8 lq .. + 8], B = Vt[dim 16 c + li][keys 8 lq .. + 8] */ \
        const h8_t A = __builtin_bit_cast(h8_t, *reinterpret_cast<const uint4*>(&P[li * kKB + 8 * lq])); \
        h8_t Bv[8]; \
_Pragma("unroll") \
        for (int c = 0; c < 8; ++c) \
            Bv[c] = __builtin_bit_cast(h8_t, *reinterpret_cast<const uint4*>(Vt + vt_off<QUAD>(ks, 16 * c + li, 8 * lq))); \
        __builtin_amdgcn_sched_group_barrier(0x100, 9, 0); \
        __builtin_amdgcn_sched_group_barrier(0x008, 8, 0); \
_Pragma("unroll") \
        for (int c = 0; c < 8; ++c) O[c] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, Bv[c], O[c], 0, 0, 0); \
        __builtin_amdgcn_wave_barrier();  /* P is rewritten in the next step only after these reads */ \
    } \
    do {} while (0)
    // both steps of an iteration run unconditionally (a step past the tile's last key block stages clamped slots and
    // computes nothing): with the second step conditional, the compiler's counter waits at the loop head cannot tell
    // which loads are outstanding and wait for all of them, the set prefetched for the next step included
    for (int st = 0; st < nsteps; st += 2) {
        RK_ATTN_STEP(st, ka);
        RK_ATTN_STEP(st + 1, kb);
    }
#undef RK_ATTN_STEP
#pragma unroll
    for (int e = 0; e < 4; ++e) l[e] = row16_sum(l[e]);  // the row's partial sums across its 16 lanes
    // merge the KS partials of each head into group 0, one group at a time, in group order: (m, l, O) of group k
    // through LDS (lane-major O, m / l per row), then m' = max, l' = l a + l_k b, O' = O a + O_k b
    if constexpr (KS > 1) {
        float* mo = reinterpret_cast<float*>(lds) + (size_t)r * (64 * 32 + 2 * kQT);
        for (int k = 1; k < KS; ++k) {
            __syncthreads();  // the staging (or the previous round's values) is no longer read
            if (ks == k) {
#pragma unroll
                for (int c = 0; c < 8; ++c)
#pragma unroll
                    for (int e = 0; e < 4; ++e) mo[(c * 4 + e) * 64 + lane] = O[c][e];
                if (li == 0) {
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        mo[64 * 32 + 4 * lq + e] = m[e];
                        mo[64 * 32 + kQT + 4 * lq + e] = l[e];
                    }
                }
            }
            __syncthreads();
            if (ks == 0) {
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float mk = mo[64 * 32 + 4 * lq + e], lk = mo[64 * 32 + kQT + 4 * lq + e];
                    const float mn = fmaxf(m[e], mk);
                    const float a = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(m[e] - mn);  // m in log2 units
                    const float b = mn == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mk - mn);
                    l[e] = l[e] * a + lk * b;
                    m[e] = mn;
#pragma unroll
                    for (int c = 0; c < 8; ++c) O[c][e] = O[c][e] * a + mo[(c * 4 + e) * 64 + lane] * b;
                }
            }
        }
    }
    if (ks != 0) return;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int t = q0 + 4 * lq + e;
        if (t >= T) continue;
        const float inv = l[e] > 0.f ? 1.0f / l[e] : 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c)
            o[(size_t)t * ldq + h * kHD + 16 * c + li] = __builtin_bit_cast(uint16_t, (_Float16)(O[c][e] * inv));
    }
}

bool act_dt(int dt) { return dt == RK_F16 || dt == RK_BF16; }

// the vector row kernels: rows of H 2-byte values in 8-column chunks, every pointer 16-byte aligned
bool vec_rows(int H, std::initializer_list<const void*> ptrs) {
    if (H % 8 || H > 8 * 256 * kVecPer) return false;
    for (const void* q : ptrs)
        if ((uintptr_t)q & 15) return false;
    return true;
}

}  // namespace

extern "C" int rk_embed_ln_rows(const int64_t* ids, const int8_t* emb_q, const uint16_t* emb_s, const void* ln_w,
                                void* x, void* h, int dt, int T, int H, float eps, rk_stream_t stream) {
    if (!ids || !emb_q || !emb_s || !ln_w || !x || !h) return RK_ERR_NULL;
    if (!act_dt(dt)) return RK_ERR_DTYPE;
    if (T <= 0 || H <= 0 || H > kRowThreads * kMaxPer) return RK_ERR_SHAPE;
    const hipStream_t st = (hipStream_t)stream;
    if (vec_rows(H, {ln_w, x, h}) && H % 8 == 0 && !((uintptr_t)emb_q & 7)) {
        if (dt == RK_BF16)
            hipLaunchKernelGGL(embed_ln_rows_vec_kernel<true>, dim3(T), dim3(256), 0, st, ids, emb_q, emb_s,
                               (const u4_t*)ln_w, (u4_t*)x, (u4_t*)h, H, eps);
        else
            hipLaunchKernelGGL(embed_ln_rows_vec_kernel<false>, dim3(T), dim3(256), 0, st, ids, emb_q, emb_s,
                               (const u4_t*)ln_w, (u4_t*)x, (u4_t*)h, H, eps);
    } else {
        hipLaunchKernelGGL(embed_ln_rows_kernel, dim3(T), dim3(kRowThreads), 0, st, ids, emb_q, emb_s, ln_w, x, h, dt,
                           H, eps);
    }
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_add_ln_rows(void* x, const void* a, const void* b, const void* ln_w, void* h, int dt, int T, int H,
                              float eps, rk_stream_t stream) {
    if (!x || !a || !ln_w || !h) return RK_ERR_NULL;
    if (!act_dt(dt)) return RK_ERR_DTYPE;
    if (T <= 0 || H <= 0 || H > kRowThreads * kMaxPer) return RK_ERR_SHAPE;
    const hipStream_t st = (hipStream_t)stream;
    if (vec_rows(H, {x, a, ln_w, h}) && (!b || !((uintptr_t)b & 15))) {
        if (dt == RK_BF16)
            hipLaunchKernelGGL(add_ln_rows_vec_kernel<true>, dim3(T), dim3(256), 0, st, (u4_t*)x, (const u4_t*)a,
                               (const u4_t*)b, (const u4_t*)ln_w, (u4_t*)h, H, eps);
        else
            hipLaunchKernelGGL(add_ln_rows_vec_kernel<false>, dim3(T), dim3(256), 0, st, (u4_t*)x, (const u4_t*)a,
                               (const u4_t*)b, (const u4_t*)ln_w, (u4_t*)h, H, eps);
    } else {
        hipLaunchKernelGGL(add_ln_rows_kernel, dim3(T), dim3(kRowThreads), 0, st, x, a, b, ln_w, h, dt, H, eps);
    }
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_post_rows(const void* y, int ldy, int p0, const void* cos_t, const void* sin_t, void* kc, void* vc,
                            void* q_out, void* act, int dt, int T, int NH, int NKV, int HD, int S, int inter, int rope,
                            rk_stream_t stream) {
    if (!y || !kc || !vc || !q_out || !act || (rope && (!cos_t || !sin_t))) return RK_ERR_NULL;
    if (!act_dt(dt)) return RK_ERR_DTYPE;
    if (T <= 0 || NH <= 0 || NKV <= 0 || HD <= 0 || HD % 2 || inter <= 0 || p0 < 0 || p0 + T > S ||
        ldy < (NH + 2 * NKV) * HD + 2 * inter)
        return RK_ERR_SHAPE;
    const hipStream_t st = (hipStream_t)stream;
    const bool vec = HD % 8 == 0 && inter % 8 == 0 && ldy % 8 == 0 && !((uintptr_t)y & 15) && !((uintptr_t)vc & 15) &&
                     !((uintptr_t)act & 15) && !((uintptr_t)kc & 3) && !((uintptr_t)q_out & 3);
    if (vec) {
        const auto* y16 = static_cast<const uint16_t*>(y);
        const dim3 pgrid(T, post_qk_parts(NH, NKV, HD) + 1 + post_act_parts(inter));
        const auto* c16 = static_cast<const uint16_t*>(cos_t);
        const auto* s16 = static_cast<const uint16_t*>(sin_t);
        if (dt == RK_BF16)
            hipLaunchKernelGGL(post_rows_vec_kernel<true>, pgrid, dim3(kPostPart), 0, st, y16, ldy, p0, c16, s16,
                               (uint16_t*)kc, (uint16_t*)vc, (uint16_t*)q_out, (uint16_t*)act, NH, NKV, HD, S, inter,
                               rope);
        else
            hipLaunchKernelGGL(post_rows_vec_kernel<false>, pgrid, dim3(kPostPart), 0, st, y16, ldy, p0, c16, s16,
                               (uint16_t*)kc, (uint16_t*)vc, (uint16_t*)q_out, (uint16_t*)act, NH, NKV, HD, S, inter,
                               rope);
    } else {
        const dim3 grid(T, NH + 2 * NKV + (inter + 255) / 256);
        hipLaunchKernelGGL(post_rows_kernel, grid, dim3(64), 0, st, y, ldy, p0, cos_t, sin_t, kc, vc, q_out, act, dt,
                           NH, NKV, HD, S, inter, rope);
    }
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_prefill_attn(const void* q, const void* kc, const void* vc, void* o, int dt, int T, int p0, int NH,
                               int NKV, int HD, int S, float scale, rk_stream_t stream) {
    if (!q || !kc || !vc || !o) return RK_ERR_NULL;
    if (dt != RK_F16) return RK_ERR_DTYPE;
    if (HD != kHD || NKV <= 0 || NH % NKV || T <= 0 || p0 < 0 || p0 + T > S) return RK_ERR_SHAPE;
    const int rep = NH / NKV;  // query heads per KV head: 1, 2, 4 or 8 (the staging splits a key block evenly)
    if (rep != 1 && rep != 2 && rep != 4 && rep != 8) return RK_ERR_SHAPE;
    if (((uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc) & 15) return RK_ERR_ALIGN;
    const hipStream_t st = (hipStream_t)stream;
    // HPB query heads per block (a share of the KV head's rep), KS key groups per block (16 waves at most). With 4
    // heads per KV head each block takes 2 of them, so a 512-token prompt runs 256 blocks (one per CU) instead of
    // 128, each staging its K / V for two heads (one head per block: the staging then dominates)
#define RK_ATTN(HPB, K)                                                                                             \
    hipLaunchKernelGGL((prefill_attn_kernel<HPB, K>), dim3(NKV * (rep / (HPB)), (T + kQT - 1) / kQT),                \
                       dim3(64 * (HPB) * (K)), attn_lds_bytes(HPB, K), st, (const uint16_t*)q, (const uint16_t*)kc,   \
                       (const uint16_t*)vc, (uint16_t*)o, T, p0, NH, NKV, S, scale)
    // the launch time is the longest query tile's key loop (p0 + T keys): past 384 keys four key groups per block
    // (two waves per SIMD) beat two (T = 512: 13.9 against 14.5 us; at T = 16 .. 256 two are faster)
    const bool long_keys = p0 + T > 384;
    switch (rep) {
        case 1: RK_ATTN(1, kAttnKS); break;
        case 2: RK_ATTN(2, kAttnKS); break;
        case 4:
            if (long_keys)
                RK_ATTN(2, 4);
            else
                RK_ATTN(2, kAttnKS);
            break;
        case 8: RK_ATTN(8, 2); break;
        default: return RK_ERR_SHAPE;
    }
#undef RK_ATTN
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
