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
// epoch in the block's own arrival word; block 0 gathers the arrivals and publishes a release word the others poll
// — no L2 write-back / invalidate (measured ~9 us each). The weights of each phase are issued before the barrier
// in front of it, so they stream in while the block waits.
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
RK_DEV uint64_t ld_coh64(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV void st_coh64(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RK_DEV uint64_t pack_f2(float a, float b) {
    return (uint64_t)__builtin_bit_cast(uint32_t, a) | ((uint64_t)__builtin_bit_cast(uint32_t, b) << 32);
}
RK_DEV uint32_t pack_h2(float a, float b) {
    h2_t v;
    v.x = (_Float16)a;
    v.y = (_Float16)b;
    return as_u32(v);
}

// ---------------------------------------------------------------------------------------------- grid barrier
// flags[b] holds the last barrier epoch block b arrived at; the release word after them (own 128-byte line) holds
// the last epoch every block has reached. Block 0's first wave gathers the arrivals and publishes the release; the
// other blocks poll only the release word (one line polled by all, measured faster than all-poll-all).
RK_DEV int release_index(int nblocks) { return (nblocks + 31) & ~31; }

RK_DEV bool wait_epoch(const uint32_t* w, unsigned epoch, const Params& p, uint64_t t0) {
    while ((int)(ld_coh(w) - epoch) < 0) {
        if (ld_coh(p.status) & kAbort) return false;
        if (wall_clock64() - t0 > kBarrierTicks) {
            atomicOr(p.status, kAbort | kTimeout);
            return false;
        }
    }
    return true;
}

// Arrival: every wave's coherent stores have completed (vmcnt counts loads too, so this comes before the next
// phase's weight loads are issued), then the block publishes the epoch.
RK_DEV void grid_arrive(const Params& p, unsigned epoch) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) st_coh(p.flags + blockIdx.x, epoch);
}

// Wait for the release of `epoch`, polled by wave 0 only: vector memory results return in issue order, so a wave
// with weight loads in flight could not see the release before they land. Wave 0 issues its own share of the next
// phase's loads after this returns.
RK_DEV void grid_wait(const Params& p, unsigned epoch) {
    if (threadIdx.x < 64) {
        const int lane = threadIdx.x;
        const uint64_t t0 = wall_clock64();
        uint32_t* release = p.flags + release_index(gridDim.x);
        if (blockIdx.x == 0) {
            bool done = false;
            while (!done) {  // every iteration has all of the lane's arrival words in flight at once
                bool ok = true;
                for (int b = lane; b < (int)gridDim.x; b += 64) ok &= (int)(ld_coh(p.flags + b) - epoch) >= 0;
                done = __all(ok);
                if (!done && (ld_coh(p.status) & kAbort)) break;
                if (!done && wall_clock64() - t0 > kBarrierTicks) {
                    if (lane == 0) atomicOr(p.status, kAbort | kTimeout);
                    break;
                }
            }
            if (lane == 0 && done) st_coh(release, epoch);
        } else if (lane == 0) {
            wait_epoch(release, epoch, p, t0);
        }
    }
    __syncthreads();
}

// ---------------------------------------------------------------------------------------------- LDS layout
struct Lds {
    uint4 hfrag[kH / 8];        // MFMA A fragments of h (phase A)
    float hsum[kNG];
    uint4 vecp[11008 / 8 + 8];  // permuted pairs of act (phase B) / ob (phase C) / natural pairs (head), per 8 cols
    float vsum[11008 / 32 + 8];
    float drow[kWaves];         // this block's down rows (phase B -> C)
    float xrow[kWaves];         // this block's rows of the residual stream (kept across layers)
    float s_m[kWaves][kMaxRep], s_l[kWaves][kMaxRep];
    float2 s_acc[kWaves][kMaxRep][64];  // the waves' partial attention outputs; then the combine's partial sums
    float c_m[kWaves], c_l[kWaves];     // the combine's per-wave running max / denominator
    int flag;
};

// x as held by wave 0 for its LayerNorm: lane holds the 8-column blocks i = lane + 64k, k < 4
struct XWave {
    float v[4][8];
};

RK_DEV void x_from_embedding(const Params& p, int64_t tok, XWave& xw) {
    const int lane = threadIdx.x & 63;
    const float es = h16(p.emb_s[tok]);
    const uint2* er = reinterpret_cast<const uint2*>(p.emb_q + (size_t)tok * kH);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint2 b = er[lane + 64 * k];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int8_t c = (int8_t)(((e < 4 ? b.x : b.y) >> (8 * (e & 3))) & 0xFF);
            xw.v[k][e] = rnd16((float)c * es);
        }
    }
}

// the residual stream written by all blocks (coherent loads)
RK_DEV void x_load(const Params& p, XWave& xw) {
    const int lane = threadIdx.x & 63;
    const uint64_t* xs = reinterpret_cast<const uint64_t*>(p.x);
    uint64_t d[4][2];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int h = 0; h < 2; ++h) d[k][h] = ld_coh64(xs + 2 * (lane + 64 * k) + h);
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t b = (uint16_t)(d[k][e >> 2] >> (16 * (e & 3)));
            xw.v[k][e] = h16(b);
        }
}

// h = round(LN(x) * w) over the 2048 values of the wave (biased variance, the reference's LayerNorm)
RK_DEV void layernorm_wave(XWave& xw, const uint16_t* w, float eps) {
    const int lane = threadIdx.x & 63;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) s += xw.v[k][e];
    const float mean = wave_sum(s) * (1.0f / kH);
    float ss = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float d = xw.v[k][e] - mean;
            ss += d * d;
        }
    const float rstd = 1.0f / sqrtf(wave_sum(ss) * (1.0f / kH) + eps);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const u4_t wv = reinterpret_cast<const u4_t*>(w)[lane + 64 * k];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const uint16_t wb = (uint16_t)(wv[e >> 1] >> (16 * (e & 1)));
            xw.v[k][e] = rnd16((xw.v[k][e] - mean) * rstd * h16(wb));
        }
    }
}

// h -> MFMA A fragments + per-group sums in LDS (wave 0)
RK_DEV void stage_h_frag(const XWave& xw, Lds& S) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int i = lane + 64 * k;
        u4_t d;
#pragma unroll
        for (int e = 0; e < 4; ++e) d[e] = pack_h2(xw.v[k][2 * e], xw.v[k][2 * e + 1]);
        uint32_t hp[4];
        pair_permute(d, hp);
        const int g = i >> 4, r = i & 15, s = r >> 2, t = r & 3;
        S.hfrag[g * 16 + t * 4 + s] = make_uint4(hp[0], hp[1], hp[2], hp[3]);
        float sum = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sum += xw.v[k][e];
        // 16 lanes = one 128-column group, inside one DPP row
        sum += dpp<0x128>(sum);
        sum += dpp<0x124>(sum);
        sum += dpp<0x122>(sum);
        sum += dpp<0x121>(sum);
        if ((lane & 15) == 0) S.hsum[i >> 4] = sum;
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

// this wave's first w_in tile of layer l (the caller issues it before the barrier that precedes phase A)
struct TileRange {
    int t0, t1;
};

RK_DEV TileRange tile_range(const Params& p) {
    const int n_in = (p.NH + 2 * p.NKV) * kHD + 2 * p.inter;
    const int ntiles = n_in / 16;
    return {(int)((long long)blockIdx.x * ntiles / gridDim.x), (int)((long long)(blockIdx.x + 1) * ntiles / gridDim.x)};
}

// wave w's first tile: waves 1..7 take the block's first seven tiles, wave 0 (which polls the barriers and issues
// its loads last) an eighth if there is one
RK_DEV int first_tile(const TileRange& tr) { return tr.t0 + ((threadIdx.x >> 6) + kWaves - 1) % kWaves; }

RK_DEV void tile_issue(const Params& p, int l, TileLoad& tl) {
    const int lane = threadIdx.x & 63;
    const TileRange tr = tile_range(p);
    const int tile = first_tile(tr);
    const size_t n_in = (size_t)(p.NH + 2 * p.NKV) * kHD + 2 * p.inter;
    if (tile < tr.t1)
        tile_load(tl, p.win_q + (size_t)l * n_in * (kH / 2), p.win_s + (size_t)l * n_in * kNG,
                  p.win_m + (size_t)l * n_in * kNG, tile * 16 + (lane & 15), lane >> 4);
}

RK_DEV void phase_a(const Params& p, int l, TileLoad& tl, int64_t tok, int64_t pos, Lds& S) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int j = lane & 15, s = lane >> 4;
    const size_t n_in = (size_t)(p.NH + 2 * p.NKV) * kHD + 2 * p.inter;
    const TileRange tr = tile_range(p);
    const int tile = first_tile(tr);

    if (tid < 64) {  // wave 0: gather x, LayerNorm, stage h (the other waves' tiles are landing meanwhile)
        XWave xw;
        if (l == 0)
            x_from_embedding(p, tok, xw);
        else
            x_load(p, xw);
        layernorm_wave(xw, p.ln_w + (size_t)l * kH, p.eps);
        stage_h_frag(xw, S);
    }
    __syncthreads();

    const Int4Masks km = int4_masks();
    const bool rope = (p.sliding >> l) & 1ull;
    if (tile < tr.t1) tile_compute(p, l, tile, tl, pos, rope, S, km);
    for (int t2 = tile + kWaves; t2 < tr.t1; t2 += kWaves) {  // blocks with more tiles than waves
        tile_load(tl, p.win_q + (size_t)l * n_in * (kH / 2), p.win_s + (size_t)l * n_in * kNG,
                  p.win_m + (size_t)l * n_in * kNG, t2 * 16 + j, s);
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
        st_coh64(reinterpret_cast<uint64_t*>(p.po + pi * kHD) + lane, pack_f2(ax, ay));
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
    // wave w merges splits part, part + kParts, ... of head r (kParts waves per head, one dim pair per lane); every
    // load of a batch is independent of the others, so a batch costs one memory round trip
    constexpr int kParts = kWaves / REP;
    const int na = min(nsp, (n + ch - 1) / ch);  // splits holding at least one slot
    const int r = wave / kParts, part = wave % kParts;
    const size_t hb = (size_t)(g * REP + r) * nsp;
    const uint64_t* po2 = reinterpret_cast<const uint64_t*>(p.po + hb * kHD) + lane;
    float M = -INFINITY, den = 0.f, nx = 0.f, ny = 0.f;
    constexpr int kCB = 8;
    for (int i0 = part; i0 < na; i0 += kCB * kParts) {
        float mi[kCB], li[kCB];
        uint64_t oi[kCB];
#pragma unroll
        for (int u = 0; u < kCB; ++u) {
            const int i = min(i0 + u * kParts, na - 1);
            mi[u] = ld_coh_f(p.pm + hb + i);
            li[u] = ld_coh_f(p.pl + hb + i);
            oi[u] = ld_coh64(po2 + (size_t)i * (kHD / 2));
        }
        float bm = M;
#pragma unroll
        for (int u = 0; u < kCB; ++u)
            if (i0 + u * kParts < na) bm = fmaxf(bm, mi[u]);
        if (bm == -INFINITY) continue;  // only empty splits so far
        const float a = __expf(M - bm);
        den *= a;
        nx *= a;
        ny *= a;
#pragma unroll
        for (int u = 0; u < kCB; ++u) {
            if (i0 + u * kParts < na && mi[u] != -INFINITY) {
                const float wt = __expf(mi[u] - bm);
                den += wt * li[u];
                nx += wt * __builtin_bit_cast(float, (uint32_t)oi[u]);
                ny += wt * __builtin_bit_cast(float, (uint32_t)(oi[u] >> 32));
            }
        }
        M = bm;
    }
    S.s_acc[wave][0][lane] = make_float2(nx, ny);
    if (lane == 0) {
        S.c_m[wave] = M;
        S.c_l[wave] = den;
    }
    __syncthreads();
    if (tid < REP * 64) {  // thread = (head r2, dim pair d2): merge the kParts waves of the head
        const int r2 = tid >> 6, d2 = tid & 63;
        float Mx = -INFINITY;
#pragma unroll
        for (int k = 0; k < kParts; ++k) Mx = fmaxf(Mx, S.c_m[r2 * kParts + k]);
        float dd = 0.f, ox = 0.f, oy = 0.f;
#pragma unroll
        for (int k = 0; k < kParts; ++k) {
            const int w2 = r2 * kParts + k;
            const float wt = S.c_m[w2] == -INFINITY ? 0.f : __expf(S.c_m[w2] - Mx);
            dd += wt * S.c_l[w2];
            ox += wt * S.s_acc[w2][0][d2].x;
            oy += wt * S.s_acc[w2][0][d2].y;
        }
        const float inv = 1.0f / dd;
        st_coh(reinterpret_cast<uint32_t*>(p.ob) + ((size_t)(g * REP + r2) * kHD) / 2 + d2, pack_h2(ox * inv, oy * inv));
    }
}

constexpr int kDownNJ = 6;  // ceil(11008 / 32 / 64): chunks per lane of one down row

// at most one row of w_down / w_o per wave (rpb <= kWaves is checked at launch)
RK_DEV int own_row(int& row) {
    const int rpb = (kH + gridDim.x - 1) / gridDim.x, wave = threadIdx.x >> 6;
    row = blockIdx.x * rpb + wave;
    return wave < rpb && row < kH;
}

RK_DEV void down_issue(const Params& p, int l, RowPrefetch<kDownNJ>& rp) {
    int row;
    const int inter = p.inter;
    if (own_row(row))
        row_prefetch<kDownNJ>(rp, p.wd_q + (size_t)l * kH * (inter / 2), p.wd_s + (size_t)l * kH * (inter / 128),
                              p.wd_m + (size_t)l * kH * (inter / 128), row, inter);
}

template <int REP>
RK_DEV void phase_b(const Params& p, int l, int64_t pos, const RowPrefetch<kDownNJ>& rp, Lds& S) {
    attention_split<REP>(p, l, pos, S);
    __syncthreads();
    stage_vec_pairs(p.act, p.inter, S);
    __syncthreads();
    const Int4Masks km = int4_masks();
    int row;
    if (own_row(row)) {
        const float d = row_dot<kDownNJ>(rp, p.inter, S, km);
        if ((threadIdx.x & 63) == 0) S.drow[threadIdx.x >> 6] = d;
    }
}

// ---------------------------------------------------------------------------------------------- phase C
RK_DEV void o_issue(const Params& p, int l, RowPrefetch<1>& rp) {
    int row;
    const int K = p.NH * kHD;
    if (own_row(row))
        row_prefetch<1>(rp, p.wo_q + (size_t)l * kH * (K / 2), p.wo_s + (size_t)l * kH * (K / 128),
                        p.wo_m + (size_t)l * kH * (K / 128), row, K);
}

RK_DEV void phase_c(const Params& p, const RowPrefetch<1>& rp, Lds& S) {
    const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63;
    const int rpb = (kH + gridDim.x - 1) / gridDim.x;
    const int K = p.NH * kHD;
    stage_vec_pairs(p.ob, K, S);
    __syncthreads();
    const Int4Masks km = int4_masks();
    int row;
    if (own_row(row)) {
        const float o = row_dot<1>(rp, K, S, km);
        if (lane == 0) S.xrow[wave] = rnd16(S.xrow[wave] + rnd16(o) + rnd16(S.drow[wave]));
    }
    __syncthreads();
    if (tid < rpb / 2)  // rows 2t, 2t+1 of this block as one dword
        st_coh(reinterpret_cast<uint32_t*>(p.x) + (blockIdx.x * rpb) / 2 + tid,
               pack_h2(S.xrow[2 * tid], S.xrow[2 * tid + 1]));
}

// ---------------------------------------------------------------------------------------------- head
// int8 audio head: block b owns rows [b * per, (b + 1) * per), wave w rows r0 + w + 8k. The first batch of a
// wave's rows is issued before the last barrier.
constexpr int kHeadB = 8;  // rows per wave per batch

struct HeadLoad {
    u4_t w[kHeadB][2];
};

RK_DEV void head_rows(const Params& p, int& r0, int& r1) {
    const int per = (p.n_audio + gridDim.x - 1) / gridDim.x;
    r0 = min(p.n_audio, (int)blockIdx.x * per);
    r1 = min(p.n_audio, r0 + per);
}

RK_DEV void head_load(const Params& p, int first, int r1, HeadLoad& hl) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < kHeadB; ++k) {
        const int r = first + kWaves * k;
        if (r < r1) {
            const u4_t* qr = reinterpret_cast<const u4_t*>(p.head_q + (size_t)r * kH);
#pragma unroll
            for (int j = 0; j < 2; ++j) hl.w[k][j] = __builtin_nontemporal_load(qr + lane + 64 * j);
        }
    }
}

RK_DEV void head_phase(const Params& p, HeadLoad& hl, Lds& S) {
    if (threadIdx.x < 64) {  // wave 0: final LayerNorm, natural pairs of h in LDS
        XWave xw;
        x_load(p, xw);
        layernorm_wave(xw, p.norm_w, p.eps);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float* v = xw.v[k];
            S.vecp[threadIdx.x + 64 * k] = make_uint4(pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), pack_h2(v[4], v[5]),
                                                      pack_h2(v[6], v[7]));
        }
    }
    __syncthreads();
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    int r0, r1;
    head_rows(p, r0, r1);
    for (int first = r0 + wave; first < r1; first += kWaves * kHeadB) {
        if (first != r0 + wave) head_load(p, first, r1, hl);
#pragma unroll
        for (int k = 0; k < kHeadB; ++k) {
            const int r = first + kWaves * k;
            if (r >= r1) break;
            float acc = 0.f;
#pragma unroll
            for (int j = 0; j < 2; ++j) {  // 128 chunks of 16 columns
                const int c = lane + 64 * j;
                uint32_t xp[8];
                const uint4 a = S.vecp[2 * c], b = S.vecp[2 * c + 1];
                xp[0] = a.x; xp[1] = a.y; xp[2] = a.z; xp[3] = a.w;
                xp[4] = b.x; xp[5] = b.y; xp[6] = b.z; xp[7] = b.w;
                acc += chunk_dot_int8<true>(hl.w[k][j], xp);
            }
            acc = wave_sum(acc);
            if (lane == 0) p.logits[r] = acc * h16(p.head_s[r]);
        }
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
    unsigned epoch = ld_coh(p.flags + blockIdx.x);
    const int rpb = (kH + gridDim.x - 1) / gridDim.x;
    const bool poller = tid < 64;

    // Each phase's weights are issued between the block's arrival at the barrier in front of the phase and the
    // wait for its release, so they stream in while the grid synchronizes: layer 0's w_in tiles right away.
    TileLoad tl;
    tile_issue(p, 0, tl);
    // this block's rows of the residual stream, x = round(emb_q[tok] * emb_s[tok]), kept in LDS across layers
    if (tid < rpb) S.xrow[tid] = rnd16((float)p.emb_q[(size_t)tok * kH + blockIdx.x * rpb + tid] * h16(p.emb_s[tok]));

    for (int l = 0; l < p.L; ++l) {
        phase_a(p, l, tl, tok, pos, S);
        RowPrefetch<kDownNJ> rd;
        grid_arrive(p, ++epoch);
        if (!poller) down_issue(p, l, rd);
        grid_wait(p, epoch);
        if (poller) down_issue(p, l, rd);
        if (l == 0 && blockIdx.x == 0 && tid == 0) p.pos[0] = pos + 1;  // every block has read pos by now

        phase_b<REP>(p, l, pos, rd, S);
        RowPrefetch<1> ro;
        grid_arrive(p, ++epoch);
        if (!poller) o_issue(p, l, ro);
        grid_wait(p, epoch);
        if (poller) o_issue(p, l, ro);

        phase_c(p, ro, S);
        if (l + 1 == p.L) break;
        grid_arrive(p, ++epoch);
        if (!poller) tile_issue(p, l + 1, tl);
        grid_wait(p, epoch);
        if (poller) tile_issue(p, l + 1, tl);
    }

    // final LayerNorm + audio head
    HeadLoad hl;
    int r0, r1;
    head_rows(p, r0, r1);
    grid_arrive(p, ++epoch);
    if (!poller) head_load(p, r0 + (tid >> 6), r1, hl);
    grid_wait(p, epoch);
    if (poller) head_load(p, r0, r1, hl);
    head_phase(p, hl, S);
}

// can `nblocks` blocks of the kernel be resident on the current device at the same time?
bool co_resident(int rep, int nblocks) {
    constexpr int kMaxDev = 64;
    static int cached[kMaxDev][4];  // resident blocks per device and rep (0: not yet asked)
    const int ri = rep == 1 ? 0 : rep == 2 ? 1 : rep == 4 ? 2 : 3;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (dev >= 0 && dev < kMaxDev && cached[dev][ri] > 0) return nblocks <= cached[dev][ri];
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
    const void* fn = rep == 1   ? (const void*)decode_step_kernel<1>
                     : rep == 2 ? (const void*)decode_step_kernel<2>
                     : rep == 4 ? (const void*)decode_step_kernel<4>
                                : (const void*)decode_step_kernel<8>;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, sizeof(Lds)) != hipSuccess) return false;
    if (dev >= 0 && dev < kMaxDev) cached[dev][ri] = per_cu * cus;
    return nblocks <= per_cu * cus;
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
    if (!co_resident(rep, nblocks)) return RK_ERR_BLOCK;  // the grid barriers need every block resident at once
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
