// Decode-step glue for gfx950 (reference engine/fused.py): everything between the GEMVs.
//
// All kernels read `pos` (int64) from device memory, so one captured graph serves every sequence length, and
// write only their outputs (no allocation, no host sync). Activations are fp16 or bf16 (`dt`), math is fp32 and
// each stored value is rounded once, at the same points as the reference's fused step.
#include "common.h"

namespace {

constexpr int kLnThreads = 256;
constexpr int kLnMaxPerThread = 32;  // H <= 8192

// sum over the block (every thread gets the total); `red` holds one float per wave
RK_DEV float block_sum(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();  // red may still be read by a previous call
    if (lane == 0) red[wave] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// Cohere LayerNorm of the block's register copy xv (element i = tid + k*blockDim), written to h:
// d = x - mean, h = d * rsqrt(mean(d^2) + eps) * w (reference engine/rumik_int4.py:38-43, engine/fused.py:23-26)
RK_DEV void layernorm_store(const float (&xv)[kLnMaxPerThread], const void* __restrict__ w, void* __restrict__ h,
                            int dt, int H, float eps, float* red) {
    const int per = (H + blockDim.x - 1) / blockDim.x;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kLnMaxPerThread; ++k)
        if (k < per && threadIdx.x + k * blockDim.x < H) s += xv[k];
    const float mean = block_sum(s, red) / (float)H;
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < kLnMaxPerThread; ++k)
        if (k < per && threadIdx.x + k * blockDim.x < H) {
            const float d = xv[k] - mean;
            ss += d * d;
        }
    const float rstd = 1.0f / sqrtf(block_sum(ss, red) / (float)H + eps);
#pragma unroll
    for (int k = 0; k < kLnMaxPerThread; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        if (k < per && i < H) store_act(h, dt, (size_t)i, (xv[k] - mean) * rstd * load_act(w, dt, (size_t)i));
    }
}

RK_DEV float round_act(float v, int dt) {
    if (dt == RK_F16) return (float)(_Float16)v;
    if (dt == RK_BF16) return bf16_bits_to_f32(f32_to_bf16_bits(v));
    return v;
}

// x = dt(emb_q[tok] * emb_s[tok]); h = LN(x) * w        (reference engine/fused.py:16-27)
__global__ __launch_bounds__(kLnThreads) void embed_ln_kernel(const int64_t* __restrict__ tok,
                                                              const int8_t* __restrict__ eq,
                                                              const uint16_t* __restrict__ es,
                                                              const void* __restrict__ w, void* __restrict__ x,
                                                              void* __restrict__ h, int dt, int H, float eps) {
    __shared__ float red[16];
    const int64_t t = tok[0];
    const float sc = f16_bits_to_f32(es[t]);
    const int8_t* row = eq + (size_t)t * H;
    float xv[kLnMaxPerThread];
#pragma unroll
    for (int k = 0; k < kLnMaxPerThread; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        xv[k] = 0.f;
        if (i < H) {
            xv[k] = round_act((float)row[i] * sc, dt);
            store_act(x, dt, (size_t)i, xv[k]);
        }
    }
    layernorm_store(xv, w, h, dt, H, eps, red);
}

// x = dt(x + a + b) (fp32 sum, one rounding); h = LN(x) * w    (reference engine/fused.py:30-41)
__global__ __launch_bounds__(kLnThreads) void add_ln_kernel(void* __restrict__ x, const void* __restrict__ a,
                                                            const void* __restrict__ b, const void* __restrict__ w,
                                                            void* __restrict__ h, int dt, int H, float eps) {
    __shared__ float red[16];
    float xv[kLnMaxPerThread];
#pragma unroll
    for (int k = 0; k < kLnMaxPerThread; ++k) {
        const int i = threadIdx.x + k * blockDim.x;
        xv[k] = 0.f;
        if (i < H) {
            float v = load_act(x, dt, (size_t)i) + load_act(a, dt, (size_t)i);
            if (b) v += load_act(b, dt, (size_t)i);
            xv[k] = round_act(v, dt);
            store_act(x, dt, (size_t)i, xv[k]);
        }
    }
    layernorm_store(xv, w, h, dt, H, eps, red);
}

// One launch for everything after the fused projection (reference engine/fused.py:44-84). Block b:
//   b < NH + NKV        RoPE one q or k head (interleaved pairs) -> q_out or the k cache slot pos
//   b < NH + 2 NKV      copy one v head into the v cache slot pos
//   otherwise           act = silu(gate) * up for 256 MLP channels
__global__ __launch_bounds__(64) void post_kernel(const void* __restrict__ y, const int64_t* __restrict__ posp,
                                                  const void* __restrict__ cos_t, const void* __restrict__ sin_t,
                                                  void* __restrict__ kc, void* __restrict__ vc, void* __restrict__ qo,
                                                  void* __restrict__ act, int dt, int NH, int NKV, int HD, int S,
                                                  int inter, int rope) {
    const int b = blockIdx.x, tid = threadIdx.x;
    const int64_t pos = posp[0];
    if (b < NH + 2 * NKV && (pos < 0 || pos >= S)) return;  // no cache slot for this position: write nothing
    if (b < NH + NKV) {
        for (int j = tid; j < HD / 2; j += 64) {
            const float xe = load_act(y, dt, (size_t)b * HD + 2 * j);
            const float xo = load_act(y, dt, (size_t)b * HD + 2 * j + 1);
            float oe = xe, oo = xo;
            if (rope) {
                const float c = load_act(cos_t, dt, (size_t)pos * HD + 2 * j);
                const float s = load_act(sin_t, dt, (size_t)pos * HD + 2 * j);
                oe = xe * c - xo * s;
                oo = xo * c + xe * s;
            }
            if (b < NH) {
                store_act(qo, dt, (size_t)b * HD + 2 * j, oe);
                store_act(qo, dt, (size_t)b * HD + 2 * j + 1, oo);
            } else {
                const size_t base = ((size_t)(b - NH) * S + pos) * HD;
                store_act(kc, dt, base + 2 * j, oe);
                store_act(kc, dt, base + 2 * j + 1, oo);
            }
        }
    } else if (b < NH + 2 * NKV) {
        const int vh = b - NH - NKV;
        const size_t src = (size_t)(NH + NKV) * HD + (size_t)vh * HD;
        const size_t dst = ((size_t)vh * S + pos) * HD;
        for (int d = tid; d < HD; d += 64) store_act(vc, dt, dst + d, load_act(y, dt, src + d));
    } else {
        const size_t off = (size_t)(NH + 2 * NKV) * HD;
        const int i0 = (b - NH - 2 * NKV) * 256;
        for (int i = i0 + tid; i < min(i0 + 256, inter); i += 64) {
            const float g = load_act(y, dt, off + i);
            const float u = load_act(y, dt, off + inter + i);
            store_act(act, dt, (size_t)i, g / (1.0f + __expf(-g)) * u);
        }
    }
}

// act[i] = silu(gate[i]) * up[i] (the MLP job of post on its own)
__global__ __launch_bounds__(256) void silu_mul_kernel(const void* __restrict__ gu, void* __restrict__ act, int dt,
                                                       int inter) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= inter) return;
    const float g = load_act(gu, dt, (size_t)i);
    const float u = load_act(gu, dt, (size_t)inter + i);
    store_act(act, dt, (size_t)i, g / (1.0f + __expf(-g)) * u);
}

// slots per split for n filled slots: ceil(n / nsplit) rounded up to a multiple of 8
RK_DEV int split_chunk(int n, int nsplit) { return ((n + nsplit - 1) / nsplit + 7) & ~7; }

constexpr int kAttnWaves = 4;
// Flash-decoding partials (reference engine/fused.py:120-169). Block (g, sp): KV head g, slots
// [sp*ch, min((sp+1)*ch, pos+1)), all REP query heads of g. Wave w takes every kAttnWaves-th slot; lane l holds
// dims (2l, 2l+1) of q, k, v and of the running acc (HD = 128). Per slot: REP dot products (fp16: v_dot2_f32_f16,
// exact products; bf16: fp32 products of the widened values, so no bf16 value is narrowed to fp16 range), a
// transposed lane reduction, an online-softmax update per head. The waves' partials are merged in LDS and
// written as (m, l, acc) per head and split; an empty split writes m = -inf, l = 0.
template <int REP>
__global__ __launch_bounds__(64 * kAttnWaves) void attn_split_kernel(const void* __restrict__ q,
                                                                      const void* __restrict__ kc,
                                                                      const void* __restrict__ vc,
                                                                      const int64_t* __restrict__ posp,
                                                                      float* __restrict__ po, float* __restrict__ pm,
                                                                      float* __restrict__ pl, int dt, int NH, int S,
                                                                      int nsplit, float scale) {
    __shared__ float s_m[kAttnWaves][REP], s_l[kAttnWaves][REP];
    __shared__ float2 s_acc[kAttnWaves][REP][64];
    const int g = blockIdx.x, sp = blockIdx.y;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int n = (int)min<int64_t>(posp[0] + 1, (int64_t)S);
    const int ch = split_chunk(n, nsplit);
    const int start = sp * ch, end = min(start + ch, n);
    const int HD = 128;

    // q pairs of the REP heads of this KV head (fp16 pairs for v_dot2; fp32 pairs for bf16 activations)
    h2_t qv[REP];
    float2 qf[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const size_t base = (size_t)(g * REP + r) * HD + 2 * lane;
        qf[r] = make_float2(load_act(q, dt, base), load_act(q, dt, base + 1));
        h2_t p;
        p.x = (_Float16)qf[r].x;
        p.y = (_Float16)qf[r].y;
        qv[r] = p;
    }
    float m[REP], l[REP];
    float2 acc[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        m[r] = -INFINITY;
        l[r] = 0.f;
        acc[r] = make_float2(0.f, 0.f);
    }
    const size_t kv_base = (size_t)g * S * HD + 2 * lane;
    for (int t = start + wave; t < end; t += kAttnWaves) {
        const size_t o = kv_base + (size_t)t * HD;
        const float k0 = load_act(kc, dt, o), k1 = load_act(kc, dt, o + 1);
        const float v0 = load_act(vc, dt, o), v1 = load_act(vc, dt, o + 1);
        float sc[REP];
        if (dt == RK_BF16) {
#pragma unroll
            for (int r = 0; r < REP; ++r) sc[r] = __builtin_fmaf(qf[r].x, k0, qf[r].y * k1);
        } else {
            h2_t kp;
            kp.x = (_Float16)k0;
            kp.y = (_Float16)k1;
#pragma unroll
            for (int r = 0; r < REP; ++r) sc[r] = dot2(qv[r], kp, 0.f);
        }
        wave_reduce_rows<REP>(sc);
        // totals: row r sits in lane writer_lane<REP>(r); broadcast each to the whole wave
        float sr[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) sr[r] = __shfl(sc[0], writer_lane<REP>(r)) * scale;
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            const float mn = fmaxf(m[r], sr[r]);
            const float alpha = __expf(m[r] - mn);  // m = -inf at the first slot: alpha = 0
            const float p = __expf(sr[r] - mn);
            l[r] = l[r] * alpha + p;
            acc[r].x = acc[r].x * alpha + p * v0;
            acc[r].y = acc[r].y * alpha + p * v1;
            m[r] = mn;
        }
    }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        if (lane == 0) {
            s_m[wave][r] = m[r];
            s_l[wave][r] = l[r];
        }
        s_acc[wave][r][lane] = acc[r];
    }
    __syncthreads();
    // wave w merges the kAttnWaves partials of heads r = w, w + kAttnWaves, ...
    for (int r = wave; r < REP; r += kAttnWaves) {
        float M = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < kAttnWaves; ++w2) M = fmaxf(M, s_m[w2][r]);
        float L = 0.f, ax = 0.f, ay = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kAttnWaves; ++w2) {
            const float wt = s_m[w2][r] == -INFINITY ? 0.f : __expf(s_m[w2][r] - M);
            L += wt * s_l[w2][r];
            ax += wt * s_acc[w2][r][lane].x;
            ay += wt * s_acc[w2][r][lane].y;
        }
        const size_t pi = (size_t)(g * REP + r) * nsplit + sp;
        po[pi * HD + 2 * lane] = ax;
        po[pi * HD + 2 * lane + 1] = ay;
        if (lane == 0) {
            pm[pi] = M;
            pl[pi] = L;
        }
    }
}

// out[h] = sum_i w_i acc_i / sum_i w_i l_i, w_i = exp(m_i - max m) over non-empty splits (fused.py:172-187)
__global__ __launch_bounds__(128) void attn_combine_kernel(const float* __restrict__ po, const float* __restrict__ pm,
                                                           const float* __restrict__ pl, void* __restrict__ out,
                                                           int dt, int HD, int nsplit) {
    const int h = blockIdx.x;
    float M = -INFINITY;
    for (int i = 0; i < nsplit; ++i) M = fmaxf(M, pm[(size_t)h * nsplit + i]);
    for (int d = threadIdx.x; d < HD; d += blockDim.x) {
        float num = 0.f, den = 0.f;
        for (int i = 0; i < nsplit; ++i) {
            const size_t pi = (size_t)h * nsplit + i;
            const float mi = pm[pi];
            const float wt = mi == -INFINITY ? 0.f : __expf(mi - M);
            num += wt * po[pi * HD + d];
            den += wt * pl[pi];
        }
        store_act(out, dt, (size_t)h * HD + d, num / den);
    }
}

__global__ void pos_advance_kernel(int64_t* pos) {
    if (threadIdx.x == 0) pos[0] += 1;
}

bool act_dt_ok(int dt) { return dt == RK_F16 || dt == RK_BF16; }

}  // namespace

extern "C" {

int rk_silu_mul(const void* gate_up, void* act, int act_dtype, int inter, rk_stream_t stream) {
    if (!gate_up || !act) return RK_ERR_NULL;
    if (inter <= 0) return RK_ERR_SHAPE;
    if (act_dtype != RK_F16 && act_dtype != RK_BF16 && act_dtype != RK_F32) return RK_ERR_DTYPE;
    hipLaunchKernelGGL(silu_mul_kernel, dim3((inter + 255) / 256), dim3(256), 0, (hipStream_t)stream, gate_up, act,
                       act_dtype, inter);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

int rk_embed_ln(const int64_t* tok, const int8_t* emb_q, const uint16_t* emb_s, const void* ln_w, void* x, void* h,
                int act_dtype, int H, float eps, rk_stream_t stream) {
    if (!tok || !emb_q || !emb_s || !ln_w || !x || !h) return RK_ERR_NULL;
    if (H <= 0 || H > kLnThreads * kLnMaxPerThread) return RK_ERR_SHAPE;
    if (!act_dt_ok(act_dtype)) return RK_ERR_DTYPE;
    hipLaunchKernelGGL(embed_ln_kernel, dim3(1), dim3(kLnThreads), 0, (hipStream_t)stream, tok, emb_q, emb_s, ln_w, x,
                       h, act_dtype, H, eps);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

int rk_add_ln(void* x, const void* a, const void* b, const void* ln_w, void* h, int act_dtype, int H, float eps,
              rk_stream_t stream) {
    if (!x || !a || !ln_w || !h) return RK_ERR_NULL;
    if (H <= 0 || H > kLnThreads * kLnMaxPerThread) return RK_ERR_SHAPE;
    if (!act_dt_ok(act_dtype)) return RK_ERR_DTYPE;
    hipLaunchKernelGGL(add_ln_kernel, dim3(1), dim3(kLnThreads), 0, (hipStream_t)stream, x, a, b, ln_w, h, act_dtype,
                       H, eps);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

int rk_post(const void* y, const int64_t* pos, const void* cos_t, const void* sin_t, void* k_cache, void* v_cache,
            void* q_out, void* act, int act_dtype, int NH, int NKV, int HD, int S, int inter, int rope,
            rk_stream_t stream) {
    if (!y || !pos || !k_cache || !v_cache || !q_out || !act || (rope && (!cos_t || !sin_t))) return RK_ERR_NULL;
    if (NH <= 0 || NKV <= 0 || HD <= 0 || HD % 2 || S <= 0 || inter <= 0) return RK_ERR_SHAPE;
    if (!act_dt_ok(act_dtype)) return RK_ERR_DTYPE;
    const int blocks = NH + 2 * NKV + (inter + 255) / 256;
    hipLaunchKernelGGL(post_kernel, dim3(blocks), dim3(64), 0, (hipStream_t)stream, y, pos, cos_t, sin_t, k_cache,
                       v_cache, q_out, act, act_dtype, NH, NKV, HD, S, inter, rope);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

int rk_attn_split(const void* q, const void* k_cache, const void* v_cache, const int64_t* pos, float* po, float* pm,
                  float* pl, int act_dtype, int NH, int NKV, int HD, int S, int nsplit, float scale,
                  rk_stream_t stream) {
    if (!q || !k_cache || !v_cache || !pos || !po || !pm || !pl) return RK_ERR_NULL;
    if (HD != 128 || NKV <= 0 || NH % NKV || S <= 0 || nsplit <= 0) return RK_ERR_SHAPE;
    if (!act_dt_ok(act_dtype)) return RK_ERR_DTYPE;
    const int rep = NH / NKV;
    dim3 grid(NKV, nsplit);
    hipStream_t s = (hipStream_t)stream;
    switch (rep) {
        case 1: hipLaunchKernelGGL(attn_split_kernel<1>, grid, dim3(64 * kAttnWaves), 0, s, q, k_cache, v_cache, pos, po, pm, pl, act_dtype, NH, S, nsplit, scale); break;
        case 2: hipLaunchKernelGGL(attn_split_kernel<2>, grid, dim3(64 * kAttnWaves), 0, s, q, k_cache, v_cache, pos, po, pm, pl, act_dtype, NH, S, nsplit, scale); break;
        case 4: hipLaunchKernelGGL(attn_split_kernel<4>, grid, dim3(64 * kAttnWaves), 0, s, q, k_cache, v_cache, pos, po, pm, pl, act_dtype, NH, S, nsplit, scale); break;
        case 8: hipLaunchKernelGGL(attn_split_kernel<8>, grid, dim3(64 * kAttnWaves), 0, s, q, k_cache, v_cache, pos, po, pm, pl, act_dtype, NH, S, nsplit, scale); break;
        default: return RK_ERR_SHAPE;
    }
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

int rk_attn_combine(const float* po, const float* pm, const float* pl, const int64_t* pos, void* out, int act_dtype,
                    int NH, int HD, int nsplit, rk_stream_t stream) {
    if (!po || !pm || !pl || !out) return RK_ERR_NULL;
    if (NH <= 0 || HD <= 0 || nsplit <= 0) return RK_ERR_SHAPE;
    if (!act_dt_ok(act_dtype)) return RK_ERR_DTYPE;
    (void)pos;  // empty splits carry m = -inf and drop out of the merge, so the split lengths are not needed here
    hipLaunchKernelGGL(attn_combine_kernel, dim3(NH), dim3(128), 0, (hipStream_t)stream, po, pm, pl, out, act_dtype,
                       HD, nsplit);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

int rk_pos_advance(int64_t* pos, rk_stream_t stream) {
    if (!pos) return RK_ERR_NULL;
    hipLaunchKernelGGL(pos_advance_kernel, dim3(1), dim3(64), 0, (hipStream_t)stream, pos);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

}  // extern "C"
