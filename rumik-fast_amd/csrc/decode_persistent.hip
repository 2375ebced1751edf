// One batch-1 decode step of the Rumik decoder in ONE kernel launch (gfx950, MI355X).
//
// Why: a step is ~36 x 3 dependent GEMVs plus glue. As separate kernels each pays a launch gap and a cold
// memory-latency ramp (measured ~3-10 us per node in a hipGraph), which alone exceeds the ~330 us a 3000 tok/s
// step may take. Here a grid of one block per CU stays resident for the whole step; each block owns fixed slices
// of every weight matrix and streams them, and the dependent phases of a layer are separated by device-side grid
// barriers instead of kernel boundaries.
//
// Per layer (the reference's step, engine/rumik_fused.py:97-121, with its parallel block x += attn(h) + mlp(h)):
//   A  every block: h = LayerNorm(x) (redundantly, 2048 values) staged in LDS as MFMA fragments;
//      its tiles of w_in (16 rows each, v_mfma_f32_16x16x32_f16, exact int4 dequant) with the epilogue fused:
//      RoPE on q / k rows (pairs are adjacent rows), K/V written at slot pos, act = silu(gate) * up (gate and up
//      rows are interleaved by 8 in the weight layout, so a tile holds both)                    [grid barrier]
//   B  block b: one flash-decoding split (KV head b / NSP, split b % NSP) for the REP query heads of that KV head;
//      the last block to finish a KV head merges its NSP partials into the attention output; and rows
//      [8b, 8b+8) of w_down . act (its weight loads are issued before the attention work)      [grid barrier]
//   C  block b: rows [8b, 8b+8) of w_o . attn; x[rows] = x + o + d (each rounded once, as the reference's
//      add_ln)                                                                                 [grid barrier]
// After the last layer: final LayerNorm and the int8 audio head (rows split over blocks); pos += 1.
//
// Cross-block data: everything one block writes for another within the step (q, K/V at pos, act, attention
// partials and output, x) is stored with agent-scope atomic stores and read with agent-scope atomic loads, which
// bypass the per-XCD (non-coherent) L2. A barrier is then only: wait for the block's stores to complete, publish an
// epoch in the block's own flag word, and poll all flags — no L2 write-back / invalidate (measured ~9 us each).
// Every wait is bounded by wall-clock time: on timeout the kernel sets an abort bit in `status` and every later
// barrier returns at once, so the grid always drains.
#include "dequant.h"

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kH = 2048;             // hidden size (compile-time: tiles and LDS staging are sized for it)
constexpr int kHD = 128;             // head dim
constexpr int kNG = kH / 128;        // groups of a 2048-long row
constexpr int kMaxRep = 8;
constexpr uint64_t kBarrierTicks = 20000000ull;  // 200 ms at the 100 MHz wall clock
constexpr unsigned kAbort = 1u, kTimeout = 2u, kBadPos = 4u;
constexpr int kFlagStride = 32;  // one 128-byte line per block flag: polls spread over memory channels

typedef rk_decode_params Params;

RK_DEV float h16(uint16_t b) { return f16_bits_to_f32(b); }
RK_DEV uint16_t f16b(float v) { return f32_to_f16_bits(v); }
RK_DEV float rnd16(float v) { return (float)(_Float16)v; }

// ---------------------------------------------------------------------------------------------- coherent access
RK_DEV void st_coh(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RK_DEV void st_coh_f(float* p, float v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RK_DEV uint32_t ld_coh(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV float ld_coh_f(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV uint32_t pack_h2(float a, float b) {
    h2_t v;
    v.x = (_Float16)a;
    v.y = (_Float16)b;
    return as_u32(v);
}

// ---------------------------------------------------------------------------------------------- grid barrier
RK_DEV void grid_sync(const Params& p, unsigned epoch) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's coherent stores have completed
    __syncthreads();
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        if (lane == 0)
            __hip_atomic_store(p.flags + blockIdx.x * kFlagStride, epoch, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const uint64_t t0 = wall_clock64();
        while (true) {
            bool ok = true;
            for (int b = lane; b < (int)gridDim.x; b += 64)
                ok = ok && (int)(__hip_atomic_load(p.flags + b * kFlagStride, __ATOMIC_RELAXED,
                                                   __HIP_MEMORY_SCOPE_AGENT) - epoch) >= 0;
            if (__all(ok)) break;
            if (__hip_atomic_load(p.status, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & kAbort) break;
            if (wall_clock64() - t0 > kBarrierTicks) {
                if (lane == 0) atomicOr(p.status, kAbort | kTimeout);
                break;
            }
            __builtin_amdgcn_s_sleep(1);
        }
    }
    __syncthreads();
}

// block-wide sum (every thread receives it); red: >= kWaves floats of LDS
RK_DEV float block_sum(float v, float* red) {
    v = wave_sum(v);
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float t = 0.f;
#pragma unroll
    for (int i = 0; i < kWaves; ++i) t += red[i];
    return t;
}

// ---------------------------------------------------------------------------------------------- LDS layout
struct Lds {
    uint4 hfrag[kH / 8];        // MFMA A fragments of h (phase A)
    float hsum[kNG];
    uint4 vecp[11008 / 8 + 8];  // permuted pairs of act (phase B) / ob (phase C) / natural pairs (head), per 8 cols
    float vsum[11008 / 32 + 8];
    float red[16];
    float drow[kWaves];         // this block's down rows (phase B -> C)
    float xrow[kWaves];         // this block's rows of the residual stream (kept across layers)
    float s_m[kWaves][kMaxRep], s_l[kWaves][kMaxRep];
    union {
        float2 s_acc[kWaves][kMaxRep][64];  // the waves' partial attention outputs
        struct {                            // then, in the combining block:
            float cw[kMaxRep][256];         //   per-split weights exp(m_i - M)
            float2 part[4][64];             //   per-quarter partial sums of one head
        };
    };
    float cden[kMaxRep];
    int flag;
};

// LayerNorm of 2048 values held as 8-value blocks by threads 0..255 (v[8] each): h = round(LN(x) * w).
RK_DEV void layernorm8(float (&v)[8], bool active, const uint16_t* w, float eps, float* red) {
    float s = 0.f;
    if (active)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += v[e];
    const float mean = block_sum(s, red) * (1.0f / kH);
    float ss = 0.f;
    if (active)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float d = v[e] - mean;
            ss += d * d;
        }
    const float rstd = 1.0f / sqrtf(block_sum(ss, red) * (1.0f / kH) + eps);
    if (active) {
        const u4_t wv = reinterpret_cast<const u4_t*>(w)[threadIdx.x];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t wb = (uint16_t)(wv[e >> 1] >> (16 * (e & 1)));
            v[e] = rnd16((v[e] - mean) * rstd * h16(wb));
        }
    }
}

// the residual stream written by the other blocks: 8 values per thread 0..255, coherent loads
RK_DEV void load_x8(const Params& p, float (&v)[8]) {
    const uint32_t* xs = reinterpret_cast<const uint32_t*>(p.x) + threadIdx.x * 4;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const h2_t h = as_h2(ld_coh(xs + e));
        v[2 * e] = (float)h.x;
        v[2 * e + 1] = (float)h.y;
    }
}

// h (8 values per thread 0..255) -> MFMA A fragments + group sums in LDS
RK_DEV void stage_h_frag(const float (&v)[8], bool active, Lds& S) {
    const int i = threadIdx.x;
    float sum = 0.f;
    if (active) {
        u4_t d;
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = pack_h2(v[2 * e], v[2 * e + 1]);
        uint32_t hp[4];
        pair_permute(d, hp);
        const int g = i >> 4, r = i & 15, s = r >> 2, t = r & 3;
        S.hfrag[g * 16 + t * 4 + s] = make_uint4(hp[0], hp[1], hp[2], hp[3]);
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += v[e];
    }
    if (i < 256) {  // 16-thread groups = one 128-column group, inside one DPP row
        sum += dpp<0x128>(sum);
        sum += dpp<0x124>(sum);
        sum += dpp<0x122>(sum);
        sum += dpp<0x121>(sum);
        if ((i & 15) == 0) S.hsum[i >> 4] = sum;
    }
}

// an fp16 vector of n (multiple of 32) values written by other blocks -> permuted pairs per 8 columns + fp32
// sums per 32 columns, in LDS (for the VALU row dots of phases B / C)
RK_DEV void stage_vec_pairs(const uint16_t* src, int n, Lds& S) {
    const int nb = n >> 3;
    const uint32_t* s32 = reinterpret_cast<const uint32_t*>(src);
    for (int base = 0; base < nb; base += kThreads) {
        const int i = base + threadIdx.x;
        float sum = 0.f;
        if (i < nb) {
            u4_t d;
#pragma unroll
            for (int e = 0; e < 4; ++e) d[e] = ld_coh(s32 + 4 * i + e);
            uint32_t hp[4];
            pair_permute(d, hp);
            S.vecp[i] = make_uint4(hp[0], hp[1], hp[2], hp[3]);
            const h2_t one = {(_Float16)1.0f, (_Float16)1.0f};
#pragma unroll
            for (int e = 0; e < 4; ++e) sum = dot2(as_h2(d[e]), one, sum);
        }
        sum += dpp<0xB1>(sum);  // 4 consecutive 8-blocks = one 32-column chunk
        sum += dpp<0x4E>(sum);
        if (i < nb && (i & 3) == 0) S.vsum[i >> 2] = sum;
    }
}

// One int4 row of length K (K % 32 == 0) by one wave: the codes / scales are loaded first (RowPrefetch), the dot
// runs once the activation vector is staged by stage_vec_pairs.
template <int NJ>
struct RowPrefetch {
    u4_t w[NJ];
    uint16_t s[NJ], m[NJ];
};

template <int NJ>
RK_DEV void row_prefetch(RowPrefetch<NJ>& rp, const uint8_t* q, const uint16_t* sc, const uint16_t* mn, int row,
                         int K) {
    const int lane = threadIdx.x & 63, nch = K >> 5, ng = K >> 7;
    const u4_t* qr = reinterpret_cast<const u4_t*>(q + (size_t)row * (K >> 1));
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = lane + 64 * j;
        if (c < nch) {
            rp.w[j] = __builtin_nontemporal_load(qr + c);
            rp.s[j] = sc[(size_t)row * ng + (c >> 2)];
            rp.m[j] = mn[(size_t)row * ng + (c >> 2)];
        } else {
            rp.w[j] = u4_t{0u, 0u, 0u, 0u};
            rp.s[j] = 0;
            rp.m[j] = 0;
        }
    }
}

template <int NJ>
RK_DEV float row_dot(const RowPrefetch<NJ>& rp, int K, const Lds& S, const Int4Masks& km) {
    const int lane = threadIdx.x & 63, nch = K >> 5;
    float acc = 0.f;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
        const int c = lane + 64 * j;
        if (c < nch) {
            uint32_t xp[16];
#pragma unroll
            for (int k = 0; k < 4; ++k) {
                const uint4 v = S.vecp[c * 4 + k];
                xp[4 * k] = v.x; xp[4 * k + 1] = v.y; xp[4 * k + 2] = v.z; xp[4 * k + 3] = v.w;
            }
            const float d = chunk_dot_int4(rp.w[j], xp, km);
            acc = __builtin_fmaf(d, h16(rp.s[j]), __builtin_fmaf(h16(rp.m[j]), S.vsum[c], acc));
        }
    }
    return wave_sum(acc);
}

RK_DEV int split_chunk(int n, int nsp) { return ((n + nsp - 1) / nsp + 7) & ~7; }

// ---------------------------------------------------------------------------------------------- phase A
// one 16-row tile of w_in: codes / scales of all 16 groups, loaded before anything else
struct TileLoad {
    u4_t w[kNG];
    u4_t s8[kNG / 8], m8[kNG / 8];
};

RK_DEV void tile_load(TileLoad& tl, const uint8_t* wq, const uint16_t* ws, const uint16_t* wm, int row, int s) {
    const uint8_t* qr = wq + (size_t)row * (kH / 2) + 16 * s;
#pragma unroll
    for (int g = 0; g < kNG; ++g) tl.w[g] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(qr + 64 * g));
#pragma unroll
    for (int b = 0; b < kNG / 8; ++b) {
        tl.s8[b] = reinterpret_cast<const u4_t*>(ws + (size_t)row * kNG)[b];
        tl.m8[b] = reinterpret_cast<const u4_t*>(wm + (size_t)row * kNG)[b];
    }
}

RK_DEV void tile_compute(const Params& p, int l, int tile, const TileLoad& tl, int64_t pos, bool rope,
                         const Lds& S, const Int4Masks& km) {
    const int lane = threadIdx.x & 63, j = lane & 15, s = lane >> 4;
    const int row = tile * 16 + j;
    const int NH = p.NH, NKV = p.NKV;
    float acc = 0.f;
#pragma unroll
    for (int g = 0; g < kNG; ++g) {
        f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const h8_t A = __builtin_bit_cast(h8_t, S.hfrag[g * 16 + t * 4 + s]);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, dequant_frag(tl.w[g][t], km), d, 0, 0, 0);
        }
        const uint16_t sb = (uint16_t)(tl.s8[g >> 3][(g & 7) >> 1] >> (16 * (g & 1)));
        const uint16_t mb = (uint16_t)(tl.m8[g >> 3][(g & 7) >> 1] >> (16 * (g & 1)));
        acc = __builtin_fmaf(d[0], h16(sb), __builtin_fmaf(h16(mb), S.hsum[g], acc));
        __builtin_amdgcn_sched_barrier(0);  // keep one group's fragments live at a time
    }
    // ---- epilogue: the projection output is rounded to fp16 first (the reference's buf_in)
    const float y = rnd16(acc);
    const float partner = dpp<0xB1>(y);  // lane j ^ 1: the other element of a RoPE pair
    const float upv = dpp<0x128>(y);     // lane (j + 8) % 16: the up row of gate row j (j < 8)
    const int qk_rows = (NH + NKV) * kHD, v_end = (NH + 2 * NKV) * kHD;
    float out = y;
    if (row < qk_rows && rope) {
        const int dd = row % kHD;
        const float c = h16(p.cos_t[(size_t)pos * kHD + (dd & ~1)]);
        const float sn = h16(p.sin_t[(size_t)pos * kHD + (dd & ~1)]);
        out = (dd & 1) ? (y * c + partner * sn) : (y * c - partner * sn);
    } else if (row >= v_end) {
        out = y / (1.0f + __expf(-y)) * upv;  // lanes j < 8: act of channel 8 * (tile index) + j
    }
    out = rnd16(out);
    const float out1 = dpp<0xB1>(out);  // the odd neighbour: even lanes store (out, out1) as one dword
    if (lane < 16 && (j & 1) == 0) {
        const uint32_t pr = pack_h2(out, out1);
        if (row < NH * kHD) {
            st_coh(reinterpret_cast<uint32_t*>(p.qbuf) + row / 2, pr);
        } else if (row < v_end) {
            const bool is_k = row < qk_rows;
            const int r2 = is_k ? row - NH * kHD : row - qk_rows;
            const int kvh = r2 / kHD, dd = r2 % kHD;
            uint16_t* cache = is_k ? p.kc : p.vc;
            st_coh(reinterpret_cast<uint32_t*>(cache + (((size_t)l * NKV + kvh) * p.S + pos) * kHD + dd), pr);
        } else if (j < 8) {
            const int ch = ((row - v_end) >> 4) * 8 + j;
            st_coh(reinterpret_cast<uint32_t*>(p.act) + ch / 2, pr);
        }
    }
}

RK_DEV void phase_a(const Params& p, int l, float (&xv)[8], bool from_global, int64_t pos, Lds& S) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int j = lane & 15, s = lane >> 4;
    const bool active = tid < kH / 8;
    const int n_in = (p.NH + 2 * p.NKV) * kHD + 2 * p.inter;
    const int ntiles = n_in / 16;
    const int t0 = (int)((long long)blockIdx.x * ntiles / gridDim.x);
    const int t1 = (int)((long long)(blockIdx.x + 1) * ntiles / gridDim.x);
    const uint8_t* wq = p.win_q + (size_t)l * n_in * (kH / 2);
    const uint16_t* ws = p.win_s + (size_t)l * n_in * kNG;
    const uint16_t* wm = p.win_m + (size_t)l * n_in * kNG;

    // weights first: this wave's tile streams in while x is gathered and normalized
    TileLoad tl;
    const int tile = t0 + wave;
    if (tile < t1) tile_load(tl, wq, ws, wm, tile * 16 + j, s);

    float v[8];
    if (from_global && active) load_x8(p, xv);
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = xv[e];
    layernorm8(v, active, p.ln_w + (size_t)l * kH, p.eps, S.red);
    stage_h_frag(v, active, S);
    __syncthreads();

    const Int4Masks km = int4_masks();
    const bool rope = (p.sliding >> l) & 1ull;
    if (tile < t1) tile_compute(p, l, tile, tl, pos, rope, S, km);
    for (int t2 = tile + kWaves; t2 < t1; t2 += kWaves) {  // blocks with more tiles than waves
        tile_load(tl, wq, ws, wm, t2 * 16 + j, s);
        tile_compute(p, l, t2, tl, pos, rope, S, km);
    }
}

// ---------------------------------------------------------------------------------------------- phase B
template <int REP>
RK_DEV void attention_split(const Params& p, int l, int64_t pos, Lds& S) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nsp = p.nsp, g = blockIdx.x / nsp, sp = blockIdx.x % nsp;
    const int n = (int)min<int64_t>(pos + 1, (int64_t)p.S);
    const int ch = split_chunk(n, nsp);
    const int start = sp * ch, end = min(start + ch, n);
    h2_t qv[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r)
        qv[r] = as_h2(ld_coh(reinterpret_cast<const uint32_t*>(p.qbuf + (size_t)(g * REP + r) * kHD) + lane));
    float m[REP], lsum[REP];
    float2 acc[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        m[r] = -INFINITY;
        lsum[r] = 0.f;
        acc[r] = make_float2(0.f, 0.f);
    }
    const size_t base = (((size_t)l * p.NKV + g) * p.S) * kHD;
    const uint32_t* kr = reinterpret_cast<const uint32_t*>(p.kc + base);
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(p.vc + base);
    constexpr int kB = 8;  // slots per wave whose K / V loads are in flight together
    for (int tb = start + wave; tb < end; tb += kB * kWaves) {
        uint32_t kw[kB], vw[kB];
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            const int t = tb + u * kWaves;
            const size_t o = (size_t)min(t, end - 1) * (kHD / 2) + lane;
            // slot pos was written in this step by another block: read it coherently; older slots: plain loads
            kw[u] = t == pos ? ld_coh(kr + o) : kr[o];
            vw[u] = t == pos ? ld_coh(vr + o) : vr[o];
        }
#pragma unroll
        for (int u = 0; u < kB; ++u) {
            const int t = tb + u * kWaves;
            if (t >= end) break;
            const h2_t kp = as_h2(kw[u]), vp = as_h2(vw[u]);
            float sc[REP];
#pragma unroll
            for (int r = 0; r < REP; ++r) sc[r] = dot2(qv[r], kp, 0.f);
            wave_reduce_rows<REP>(sc);
            float sr[REP];
#pragma unroll
            for (int r = 0; r < REP; ++r) sr[r] = __shfl(sc[0], writer_lane<REP>(r)) * p.scale;
            const float v0 = (float)vp.x, v1 = (float)vp.y;
#pragma unroll
            for (int r = 0; r < REP; ++r) {
                const float mn = fmaxf(m[r], sr[r]);
                const float alpha = __expf(m[r] - mn);
                const float e = __expf(sr[r] - mn);
                lsum[r] = lsum[r] * alpha + e;
                acc[r].x = acc[r].x * alpha + e * v0;
                acc[r].y = acc[r].y * alpha + e * v1;
                m[r] = mn;
            }
        }
    }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        if (lane == 0) {
            S.s_m[wave][r] = m[r];
            S.s_l[wave][r] = lsum[r];
        }
        S.s_acc[wave][r][lane] = acc[r];
    }
    __syncthreads();
    for (int r = wave; r < REP; r += kWaves) {
        float M = -INFINITY;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; ++w2) M = fmaxf(M, S.s_m[w2][r]);
        float Lt = 0.f, ax = 0.f, ay = 0.f;
#pragma unroll
        for (int w2 = 0; w2 < kWaves; ++w2) {
            const float wt = S.s_m[w2][r] == -INFINITY ? 0.f : __expf(S.s_m[w2][r] - M);
            Lt += wt * S.s_l[w2][r];
            ax += wt * S.s_acc[w2][r][lane].x;
            ay += wt * S.s_acc[w2][r][lane].y;
        }
        const size_t pi = (size_t)(g * REP + r) * nsp + sp;
        st_coh_f(p.po + pi * kHD + 2 * lane, ax);
        st_coh_f(p.po + pi * kHD + 2 * lane + 1, ay);
        if (lane == 0) {
            st_coh_f(p.pm + pi, M);
            st_coh_f(p.pl + pi, Lt);
        }
    }
    // ---- the last block of this KV head merges the nsp partials of its REP heads
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid == 0) {
        const unsigned old = __hip_atomic_fetch_add(p.grp_ctr + g, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        S.flag = old == (unsigned)(nsp - 1);
        if (S.flag) __hip_atomic_store(p.grp_ctr + g, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!S.flag) return;
    // split weights w_i = exp(m_i - M) per head, and the denominators, into LDS
    for (int r = wave; r < REP; r += kWaves) {
        const int hh = g * REP + r;
        float mi[4], mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = lane + 64 * k;
            mi[k] = i < nsp ? ld_coh_f(p.pm + (size_t)hh * nsp + i) : -INFINITY;
            mx = fmaxf(mx, mi[k]);
        }
        mx = wave_max(mx);
        float den = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int i = lane + 64 * k;
            const float wt = (i < nsp && mi[k] != -INFINITY) ? __expf(mi[k] - mx) : 0.f;
            if (i < nsp) S.cw[r][i] = wt;
            den += i < nsp ? wt * ld_coh_f(p.pl + (size_t)hh * nsp + i) : 0.f;
        }
        den = wave_sum(den);
        if (lane == 0) S.cden[r] = den;
    }
    __syncthreads();
    // num[h][d] = sum_i w_i po_i[d]: thread = (dim pair, split quarter) for each head; every load of a thread
    // is independent, so all of them are in flight at once
    constexpr int kQ = 4;                       // split quarters
    for (int r = 0; r < REP; ++r) {
        const int hh = g * REP + r;
        for (int e = tid; e < kQ * (kHD / 2); e += kThreads) {
            const int qtr = e / (kHD / 2), d2 = 2 * (e % (kHD / 2));
            const int i0 = qtr * ((nsp + kQ - 1) / kQ), i1 = min(nsp, i0 + (nsp + kQ - 1) / kQ);
            const float* pr = p.po + (size_t)hh * nsp * kHD + d2;
            float n0 = 0.f, n1 = 0.f;
#pragma unroll 16
            for (int i = i0; i < i1; ++i) {
                const float wt = S.cw[r][i];
                n0 += wt * ld_coh_f(pr + (size_t)i * kHD);
                n1 += wt * ld_coh_f(pr + (size_t)i * kHD + 1);
            }
            S.part[qtr][d2 / 2] = make_float2(n0, n1);
        }
        __syncthreads();
        if (tid < kHD / 2) {
            float2 t = S.part[0][tid];
#pragma unroll
            for (int q = 1; q < kQ; ++q) {
                t.x += S.part[q][tid].x;
                t.y += S.part[q][tid].y;
            }
            const float inv = 1.0f / S.cden[r];
            st_coh(reinterpret_cast<uint32_t*>(p.ob) + ((size_t)hh * kHD) / 2 + tid, pack_h2(t.x * inv, t.y * inv));
        }
        __syncthreads();
    }
}

template <int REP>
RK_DEV void phase_b(const Params& p, int l, int64_t pos, Lds& S) {
    const int wave = threadIdx.x >> 6;
    const int rpb = (kH + gridDim.x - 1) / gridDim.x;
    const int inter = p.inter;
    // the down row's weights go out first: independent of everything this phase waits on
    constexpr int NJ = 6;  // ceil(11008 / 32 / 64)
    RowPrefetch<NJ> rp;
    const int row = blockIdx.x * rpb + wave;  // at most one down row per wave (rpb <= kWaves is checked at launch)
    const bool mine = wave < rpb && row < kH;
    if (mine)
        row_prefetch<NJ>(rp, p.wd_q + (size_t)l * kH * (inter / 2), p.wd_s + (size_t)l * kH * (inter / 128),
                         p.wd_m + (size_t)l * kH * (inter / 128), row, inter);

    attention_split<REP>(p, l, pos, S);
    __syncthreads();

    stage_vec_pairs(p.act, inter, S);
    __syncthreads();
    const Int4Masks km = int4_masks();
    if (mine) {
        const float d = row_dot<NJ>(rp, inter, S, km);
        if ((threadIdx.x & 63) == 0) S.drow[wave] = d;
    }
}

// ---------------------------------------------------------------------------------------------- phase C
RK_DEV void phase_c(const Params& p, int l, Lds& S) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rpb = (kH + gridDim.x - 1) / gridDim.x;
    const int K = p.NH * kHD;
    RowPrefetch<1> rp;
    const int row = blockIdx.x * rpb + wave;
    const bool mine = wave < rpb && row < kH;
    if (mine)
        row_prefetch<1>(rp, p.wo_q + (size_t)l * kH * (K / 2), p.wo_s + (size_t)l * kH * (K / 128),
                        p.wo_m + (size_t)l * kH * (K / 128), row, K);
    stage_vec_pairs(p.ob, K, S);
    __syncthreads();
    const Int4Masks km = int4_masks();
    if (mine) {
        const float o = row_dot<1>(rp, K, S, km);
        if (lane == 0) S.xrow[wave] = rnd16(S.xrow[wave] + rnd16(o) + rnd16(S.drow[wave]));
    }
    __syncthreads();
    if (tid < rpb / 2)  // rows 2t, 2t+1 of this block as one dword
        st_coh(reinterpret_cast<uint32_t*>(p.x) + (blockIdx.x * rpb) / 2 + tid,
               pack_h2(S.xrow[2 * tid], S.xrow[2 * tid + 1]));
}

// ---------------------------------------------------------------------------------------------- head
RK_DEV void head_phase(const Params& p, const float (&hv)[8], bool active, Lds& S) {
    if (active) S.vecp[threadIdx.x] = make_uint4(pack_h2(hv[0], hv[1]), pack_h2(hv[2], hv[3]), pack_h2(hv[4], hv[5]),
                                                 pack_h2(hv[6], hv[7]));
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int per = (p.n_audio + gridDim.x - 1) / gridDim.x;
    const int r0 = blockIdx.x * per, r1 = min(p.n_audio, r0 + per);
    for (int r = r0 + wave; r < r1; r += kWaves) {
        const u4_t* qr = reinterpret_cast<const u4_t*>(p.head_q + (size_t)r * kH);
        u4_t w[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) w[j] = __builtin_nontemporal_load(qr + lane + 64 * j);
        float acc = 0.f;
#pragma unroll
        for (int j = 0; j < 2; ++j) {  // 128 chunks of 16 columns
            const int c = lane + 64 * j;
            uint32_t xp[8];
            const uint4 a = S.vecp[2 * c], b = S.vecp[2 * c + 1];
            xp[0] = a.x; xp[1] = a.y; xp[2] = a.z; xp[3] = a.w;
            xp[4] = b.x; xp[5] = b.y; xp[6] = b.z; xp[7] = b.w;
            acc += chunk_dot_int8<true>(w[j], xp);
        }
        acc = wave_sum(acc);
        if (lane == 0) p.logits[r] = acc * h16(p.head_s[r]);
    }
}

template <int REP>
__global__ __launch_bounds__(kThreads) void decode_step_kernel(Params p) {
    extern __shared__ __align__(16) uint8_t smem_raw[];
    Lds& S = *reinterpret_cast<Lds*>(smem_raw);
    const int tid = threadIdx.x;
    const int64_t pos = p.pos[0];
    const int64_t tok = p.tok[0];
    if (pos < 0 || pos >= p.S) {  // no cache slot for this position: every block leaves before any barrier
        if (blockIdx.x == 0 && tid == 0) atomicOr(p.status, kBadPos);
        return;
    }
    unsigned epoch = __hip_atomic_load(p.flags + blockIdx.x * kFlagStride, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    const int rpb = (kH + gridDim.x - 1) / gridDim.x;

    // embedding: x = round(emb_q[tok] * emb_s[tok]); every block keeps the whole vector for its LayerNorm and
    // its own rows in LDS
    const bool active = tid < kH / 8;
    float xv[8];
    {
        const float es = h16(p.emb_s[tok]);
        const int8_t* er = p.emb_q + (size_t)tok * kH;
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = active ? rnd16((float)er[tid * 8 + e] * es) : 0.f;
        if (tid < rpb) S.xrow[tid] = rnd16((float)er[blockIdx.x * rpb + tid] * es);
    }

    for (int l = 0; l < p.L; ++l) {
        phase_a(p, l, xv, l > 0, pos, S);
        grid_sync(p, ++epoch);
        if (l == 0 && blockIdx.x == 0 && tid == 0) p.pos[0] = pos + 1;  // every block has read pos by now
        phase_b<REP>(p, l, pos, S);
        grid_sync(p, ++epoch);
        phase_c(p, l, S);
        grid_sync(p, ++epoch);
    }

    // final LayerNorm + audio head
    if (active) load_x8(p, xv);
    layernorm8(xv, active, p.norm_w, p.eps, S.red);
    head_phase(p, xv, active, S);
}

}  // namespace

extern "C" int rk_decode_step_persistent(const rk_decode_params* params, int nblocks, rk_stream_t stream) {
    if (!params) return RK_ERR_NULL;
    const Params& p = *params;
    if (p.L <= 0 || p.L > 64 || p.NKV <= 0 || p.NH % p.NKV || p.NH * kHD != kH || p.S <= 0) return RK_ERR_SHAPE;
    const int rep = p.NH / p.NKV;
    if (!(rep == 1 || rep == 2 || rep == 4 || rep == 8)) return RK_ERR_SHAPE;
    if (p.inter <= 0 || p.inter % 128 || p.inter > 11008 || (p.inter + 2047) / 2048 > 6) return RK_ERR_SHAPE;
    if (nblocks <= 0 || nblocks % p.NKV || nblocks / p.NKV != p.nsp || p.nsp > 256) return RK_ERR_BLOCK;
    if ((kH + nblocks - 1) / nblocks > kWaves) return RK_ERR_BLOCK;  // each wave owns one row of down / O
    if (!p.tok || !p.pos || !p.emb_q || !p.emb_s || !p.win_q || !p.wo_q || !p.wd_q || !p.kc || !p.vc ||
        !p.head_q || !p.logits || !p.x || !p.flags || !p.status || !p.grp_ctr)
        return RK_ERR_NULL;
    hipStream_t st = (hipStream_t)stream;
    switch (rep) {
        case 1: hipLaunchKernelGGL(decode_step_kernel<1>, dim3(nblocks), dim3(kThreads), sizeof(Lds), st, p); break;
        case 2: hipLaunchKernelGGL(decode_step_kernel<2>, dim3(nblocks), dim3(kThreads), sizeof(Lds), st, p); break;
        case 4: hipLaunchKernelGGL(decode_step_kernel<4>, dim3(nblocks), dim3(kThreads), sizeof(Lds), st, p); break;
        default: hipLaunchKernelGGL(decode_step_kernel<8>, dim3(nblocks), dim3(kThreads), sizeof(Lds), st, p); break;
    }
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_decode_params_size(void) { return (int)sizeof(Params); }
