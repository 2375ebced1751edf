// One batch-1 decode step of the Rumik decoder in ONE kernel launch (gfx950, MI355X).
//
// Why one launch: a step is ~36 x 3 dependent GEMVs plus glue. As separate kernels each pays a launch gap and a
// cold memory-latency ramp (measured 2-10 us per hipGraph node), far more than the ~330 us a 3000 tok/s step may
// take. Here a grid of one block per CU stays resident for the whole step and streams its fixed share of every
// weight matrix.
//
// Synchronization is dataflow, not grid barriers: every value one block hands to another is stored as a tagged
// 32-bit word (fp16 value | tag << 16; the tag names the step and the layer) with an agent-scope atomic store, and
// the consumer polls the words themselves with agent-scope atomic loads (coherent across the XCDs' L2s). One
// cross-block edge then costs one store-to-load hop (measured 0.75 us idle, ~1.5 us while HBM streams) instead of
// a barrier's two plus a data load. Every poll loads all its words and the status word as one batch: one round
// trip per poll iteration.
//
// Roles inside a block: wave 0 only polls, gathers and stages exchanged data in LDS. It never has weight loads in
// flight: vector-memory results return in issue order, so a poll behind a weight burst would wait for the burst.
// Waves 1..7 ("streamers") stream weights, issued a phase or more ahead of use, and compute. A wave has at most 63
// vector-memory instructions outstanding, so the issue points keep each streamer's in-flight loads below that.
//
// Per layer l (the reference's step, engine/rumik_fused.py:97-121, with its parallel block x += attn(h) + mlp(h)):
//   wave 0: x of layer l-1 (tagged, all 2048) -> LayerNorm -> h as MFMA fragments in LDS
//   streamers: the block's w_in tiles (16 rows each), K-split: streamer w computes 2-3 of the 16 column groups of
//     every tile (v_mfma_f32_16x16x32_f16, exact int4 dequant), so each wave reads its h fragments once; the
//     partial sums meet in LDS; epilogue: RoPE on q / k rows, q / k / v published tagged (K/V also into the cache
//     at pos), act = silu(gate) * up kept in LDS for the block's own MLP channels
//   streamers: the w_down columns of those channels (16-column slices) times act -> a partial down output for all
//     2048 rows, published tagged (each x-row owner sums the partials of all blocks for its rows)
//   wave 0: q of its KV head (+ k, v at pos) -> LDS;  streamers: one flash-decoding split over the cached slots,
//     partial (m, l, o / l) published tagged
//   block b = (head h = b / 16, row group r = b % 16): the streamers poll head h's split partials, wave 0 merges
//     them -> h's attention output in LDS; streamers: w_o[128r .. 128r + 128, h's 128 columns] . attn -> o partials
//     of those rows, published tagged (no separate combiner and no all-to-all of the attention output)
//   wave 0: its 8 rows of the down partials of all blocks and of the o partials of all heads, one poll batch;
//     x rows = x + o + d (each rounded once, as add_ln), published
// After the last layer: final LayerNorm and the int8 audio head (rows split over blocks); pos += 1.
//
// Every wait is bounded by wall-clock time (200 ms): on expiry the kernel sets an abort bit in `status`, every
// later wait returns at once and the grid drains with garbage results.
#include "dequant.h"

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kStreamers = kWaves - 1;
constexpr int kSLanes = 64 * kStreamers;  // 448 streamer lanes
constexpr int kH = 2048;                   // hidden size (compile-time: tiles and staging are sized for it)
constexpr int kHD = 128;                   // head dim
constexpr int kNG = kH / 128;              // column groups of a w_in row
constexpr int kMaxRep = 8;
constexpr int kMaxTiles = 7;               // w_in tiles per block
constexpr int kGPW = 2;                    // column groups per wave (8 waves x 2 = 16)
constexpr int kTileSplit = 3;              // next-layer tiles [0, 3) are issued after the tile compute, the rest later
constexpr int kMaxSlices = 3;              // w_down 16-column slices per block
constexpr int kRP = (kH / 2 + kSLanes - 1) / kSLanes;  // down row pairs per streamer lane (3)
constexpr int kKVPre = 5;                  // cached slots per streamer whose K / V are loaded ahead (7 x 5 >= 2048 / 64)
constexpr int kHeadRows = 7;               // head rows per streamer loaded ahead (the rest load when used)
constexpr int kWork = 16;                  // int16 entries per block in the work table
constexpr int kPreRows = 1;                // ~0.5 us wait before the down / o partial poll
constexpr int kPace = 28;                  // s_sleep(1) units between the streamers' next-layer load groups
// x is polled by every block: it is published in kXRep copies 8 KB apart and block b polls copy b % kXRep, so no
// 8 KB stretch of memory serves more than 16 pollers
constexpr int kXRep = 16;
constexpr int kRepQwords = kH / 2;         // qwords per copy (2048 tagged fp16 words)
constexpr uint64_t kWaitTicks = 20000000ull;  // 200 ms at the 100 MHz wall clock
constexpr unsigned kAbort = 1u, kTimeout = 2u, kBadPos = 4u;

typedef rk_decode_params Params;

RK_DEV float h16(uint16_t b) { return f16_bits_to_f32(b); }
RK_DEV uint16_t f16b(float v) { return f32_to_f16_bits(v); }
RK_DEV float rnd16(float v) { return (float)(_Float16)v; }

RK_DEV uint32_t pack_h2(float a, float b) {
    h2_t v;
    v.x = (_Float16)a;
    v.y = (_Float16)b;
    return as_u32(v);
}

// ---------------------------------------------------------------------------------------------- coherent access
RK_DEV void st_coh(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RK_DEV uint32_t ld_coh(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV uint64_t ld_coh64(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV void st_coh64(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// ---------------------------------------------------------------------------------------------- tagged words
RK_DEV uint32_t tag_of(uint32_t step, int l) { return 1u + (step * 64u + (uint32_t)l) % 65535u; }
RK_DEV uint32_t tword(float v, uint32_t tag) { return (uint32_t)f16b(v) | (tag << 16); }
RK_DEV uint64_t tpair(float a, float b, uint32_t tag) {
    return (uint64_t)tword(a, tag) | ((uint64_t)tword(b, tag) << 32);
}
RK_DEV bool pair_ok(uint64_t q, uint32_t tag) {
    return (uint32_t)((q >> 16) & 0xFFFFu) == tag && (uint32_t)(q >> 48) == tag;
}
// the two fp16 values of a tagged pair as one packed fp16x2 dword
RK_DEV uint32_t pair_val(uint64_t q) { return (uint32_t)(q & 0xFFFFu) | ((uint32_t)(q >> 16) & 0xFFFF0000u); }

// true while a wait may go on; on expiry raise the abort bit. `status` is the status word loaded in the same batch
// as the poll it belongs to (one round trip per poll iteration).
RK_DEV bool wait_more(const Params& p, uint64_t t0, uint32_t status) {
    if (status & kAbort) return false;
    if (wall_clock64() - t0 > kWaitTicks) {
        if ((threadIdx.x & 63) == 0) atomicOr(p.status, kAbort | kTimeout);
        return false;
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

// Every poller first waits `pre` x ~0.5 us (s_sleep 20): measured on 256 blocks, all-to-all exchanges complete
// fastest when the first poll comes ~0.5 us after the data is written and polls then follow back to back; polls
// sent long before the data exists only load the coherent path that every other exchange shares.
// Streamers spread the next layer's loads over the window in which wave 0 gathers the rows, publishes x and polls
// it back (they have nothing else to do until the next LayerNorm): a CU's memory requests are served in order, so
// a poll issued behind the whole burst waited for all of it. Measured (36 layers, ctx 256 / 2048 us per token):
// one burst 688 / 772, kPace 24 684 / 758, 32 680 / 758, 40 728 / 794 (longer than wave 0's window); with the
// down prefetch in three pieces (half a pace apart) and no pre-wait before the x poll: kPace 24 684 / 755, 28
// 666 / 743, 32 672 / 748, 36 694 / 765.
RK_DEV void pace_wait(int n) {
    for (int i = 0; i < n; ++i) __builtin_amdgcn_s_sleep(1);
}

RK_DEV void pre_wait(int pre) {
    for (int i = 0; i < pre; ++i) __builtin_amdgcn_s_sleep(20);
}

// Poll N tagged fp16 pairs per lane (qword addresses from addr(k); nullptr = not needed) until every tag matches;
// val[k] receives the packed pair. Every iteration loads all N words and the status word unconditionally, so they
// are one batch with a single wait: reloading a word already validated is harmless, because its next value is
// written only after every consumer has finished this poll (the exchanges' dataflow order), and its first
// validated value is the one kept. Wave-uniform control flow; false after an abort or a timeout.
template <int N, class Addr>
RK_DEV bool poll_pairs(const Params& p, uint32_t tag, Addr addr, uint32_t (&val)[N], int pre = 1) {
    static_assert(N <= 32, "pending mask");
    pre_wait(pre);
    // a valid, lane-varying address for the unneeded slots (a uniform one is turned into scalar moves and waits)
    const uint64_t* dummy = reinterpret_cast<const uint64_t*>(p.tx) + (threadIdx.x & 63);
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (addr(k)) pending |= 1u << k;
    const uint64_t t0 = wall_clock64();
    while (true) {
        uint64_t q[N];
#pragma unroll
        for (int k = 0; k < N; ++k) {
            const uint64_t* a = addr(k);
            q[k] = ld_coh64(a ? a : dummy);
        }
        const uint32_t st = ld_coh(p.status);
#pragma unroll
        for (int k = 0; k < N; ++k)
            if ((pending & (1u << k)) && pair_ok(q[k], tag)) {
                val[k] = pair_val(q[k]);
                pending &= ~(1u << k);
            }
        if (__all(pending == 0)) return true;
        if (!wait_more(p, t0, st)) return false;
    }
}

// ---------------------------------------------------------------------------------------------- LDS layout
struct Lds {
    uint4 hfrag[kH / 8];                      // MFMA A fragments of h
    float hsum[kNG];                          // per-group sums of h
    float tpart[kWaves][kMaxTiles][16];       // K-split partial dots of the block's tiles
    float ty[kMaxTiles][16];                  // the tiles' projection outputs (rounded)
    float act[kMaxSlices * 16];               // act of the block's MLP channels
    uint32_t qs[kMaxRep][64];                 // q pairs of the block's KV head
    uint32_t knew[64], vnew[64];              // k, v at pos of that KV head
    float s_m[kStreamers][kMaxRep], s_l[kStreamers][kMaxRep];
    float2 s_acc[kStreamers][kMaxRep][64];    // per-streamer attention partials
    uint4 vecp[kH / 8];                       // h as natural pairs (the int8 head's input)
    uint32_t attn[kHD / 2];                   // head (block / 16)'s attention output, natural fp16 pairs
    float asum;                               //   and the sum of its 128 values
    float2 cpa[kStreamers][64];               // the combine's per-streamer parts: sum of w_i o_i per dim pair,
    float cpm[kStreamers], cpl[kStreamers];   //   the streamer's max m and sum of w_i
    float orow[8], drow[8], xrow[8];          // this block's rows of o, down and the residual stream
    float rcos[kHD / 2], rsin[kHD / 2];       // RoPE cos / sin of pair i at pos
    uint4 xraw[kH / 8];                       // x (fp16, 8 per entry) for the block-wide LayerNorm
    uint4 lnw[kH / 8];                        // its weights
    float ln_mean, ln_rstd;
    int16_t work[kWork];
};

// ---------------------------------------------------------------------------------------------- block work
struct Work {
    int nt;     // w_in tiles
    int sb, se; // down slices [sb, se)
};

RK_DEV Work work_of(const Lds& S) {
    Work w;
    w.nt = 0;
#pragma unroll
    for (int t = 0; t < kMaxTiles; ++t) w.nt += S.work[t] >= 0;
    w.sb = S.work[8];
    w.se = S.work[9];
    return w;
}

// wave w's two column groups of every tile: streamers (w = 1..7) groups 2(w - 1), 2(w - 1) + 1, wave 0 groups 14,
// 15 (it computes them while it would otherwise wait for the streamers)
RK_DEV int wave_id() { return threadIdx.x >> 6; }
RK_DEV int group0(int w) { return 2 * ((w + kWaves - 1) % kWaves); }

// ---------------------------------------------------------------------------------------------- x / h (wave 0)
// lane holds the 8-column blocks i = lane + 64k, k < 4
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

RK_DEV bool x_poll(const Params& p, uint32_t tag, XWave& xw) {
    const int lane = threadIdx.x & 63;
    // the opaque zero keeps the addresses from being hoisted out of the layer loop (they would pin ~30 VGPRs)
    const uint64_t* tx =
        reinterpret_cast<const uint64_t*>(p.tx) + (blockIdx.x % kXRep) * kRepQwords + opaque_vgpr(0u);
    uint32_t v[16];
    // no pre-wait: x is polled after the row gather and the x publication, when most rows are out already
    const bool ok = poll_pairs<16>(
        p, tag, [&](int k) -> const uint64_t* { return tx + 4 * (lane + 64 * (k >> 2)) + (k & 3); }, v, 0);
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const h2_t h = as_h2(v[4 * k + e]);
            xw.v[k][2 * e] = (float)h.x;
            xw.v[k][2 * e + 1] = (float)h.y;
        }
    return ok;
}

// LayerNorm (the reference's, engine/rumik_int4.py:38-43: biased variance, no bias), split over the block:
// wave 0 holds x after its poll, computes mean and rstd and stages x and the weights in LDS (ln_stats); then
// threads 0..255 normalize one 8-column block each and stage it (ln_apply_frag for the MFMA fragments of h,
// ln_apply_pairs for the head's natural pairs).
// the LayerNorm weights of one row, 4 x 16 bytes per lane; loaded before the x poll so that their round trip
// overlaps it
struct LnW {
    u4_t v[4];
};
RK_DEV void ln_w_issue(const uint16_t* w, LnW& wv) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int k = 0; k < 4; ++k) wv.v[k] = reinterpret_cast<const u4_t*>(w)[lane + 64 * k];
}

RK_DEV void ln_stats(const XWave& xw, const LnW& lw, float eps, Lds& S) {
    const int lane = threadIdx.x & 63;
    const u4_t* wv = lw.v;
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
        const float* v = xw.v[k];
        S.xraw[lane + 64 * k] =
            make_uint4(pack_h2(v[0], v[1]), pack_h2(v[2], v[3]), pack_h2(v[4], v[5]), pack_h2(v[6], v[7]));
        S.lnw[lane + 64 * k] = make_uint4(wv[k][0], wv[k][1], wv[k][2], wv[k][3]);
    }
    if (lane == 0) {
        S.ln_mean = mean;
        S.ln_rstd = rstd;
    }
}

// thread i < 256: h of 8-column block i = round((x - mean) * rstd * w)
RK_DEV void ln_block(const Lds& S, int i, float (&h)[8]) {
    const uint4 xv = S.xraw[i], wv = S.lnw[i];
    const uint32_t xs[4] = {xv.x, xv.y, xv.z, xv.w}, ws[4] = {wv.x, wv.y, wv.z, wv.w};
    const float mean = S.ln_mean, rstd = S.ln_rstd;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const h2_t xh = as_h2(xs[e]), wh = as_h2(ws[e]);
        h[2 * e] = rnd16(((float)xh.x - mean) * rstd * (float)wh.x);
        h[2 * e + 1] = rnd16(((float)xh.y - mean) * rstd * (float)wh.y);
    }
}

// h -> MFMA A fragments (pairs permuted as the dequant orders the codes) + per-group sums; threads 0..255
RK_DEV void ln_apply_frag(Lds& S) {
    const int i = (int)opaque_vgpr(threadIdx.x);  // recomputed per call: a hoisted LDS address would be spilled
    if (i >= kH / 8) return;
    float h[8];
    ln_block(S, i, h);
    u4_t d;
#pragma unroll
    for (int e = 0; e < 4; ++e) d[e] = pack_h2(h[2 * e], h[2 * e + 1]);
    uint32_t hp[4];
    pair_permute(d, hp);
    const int g = i >> 4, r = i & 15, sq = r >> 2, t = r & 3;
    S.hfrag[g * 16 + t * 4 + sq] = make_uint4(hp[0], hp[1], hp[2], hp[3]);
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) sum += h[e];
    sum += dpp<0x128>(sum);  // 16 threads = one 128-column group, inside one DPP row
    sum += dpp<0x124>(sum);
    sum += dpp<0x122>(sum);
    sum += dpp<0x121>(sum);
    if ((i & 15) == 0) S.hsum[g] = sum;
}

// h -> natural fp16 pairs per 8 columns (the int8 head's input); threads 0..255
RK_DEV void ln_apply_pairs(Lds& S) {
    const int i = threadIdx.x;
    if (i >= kH / 8) return;
    float h[8];
    ln_block(S, i, h);
    S.vecp[i] = make_uint4(pack_h2(h[0], h[1]), pack_h2(h[2], h[3]), pack_h2(h[4], h[5]), pack_h2(h[6], h[7]));
}

// ---------------------------------------------------------------------------------------------- w_in tiles
struct TileRegs {
    u4_t w[kGPW][kMaxTiles];
    uint32_t sm[kGPW][kMaxTiles];  // scale | min << 16 of (group, tile) for row lane % 16
};

RK_DEV size_t n_tiles(const Params& p) { return ((size_t)(p.NH + 2 * p.NKV) * kHD + 2 * p.inter) / 16; }

// Streamer prefetches are branch-free with a fixed instruction count (addresses clamped to valid data that is then
// ignored): the compiler can then wait for exactly the loads a computation needs. With data-dependent branches
// around loads it cannot count the loads issued after a prefetch and waits for all of them, so e.g. the attention
// would wait for the down-projection burst issued just before it.
//
// win_t: per (layer, tile, group) 1 KiB of codes in lane order. win_sm: per (layer, tile, wave, row) the two
// scale | min << 16 words of the wave's groups, one 8-byte load per tile.
RK_DEV void tile_issue(const Params& p, int l, const Lds& S, const Work& wk, TileRegs& tr, int tb, int te) {
    const int lane = threadIdx.x & 63, w = wave_id();
    const int g0 = group0(w);
    const size_t base = (size_t)l * n_tiles(p);
    const int t_fallback = wk.nt > 0 ? S.work[0] : 0;
#pragma unroll
    for (int t = 0; t < kMaxTiles; ++t) {
        if (t < tb || t >= te) continue;  // compile-time after inlining
        const size_t T = base + (t < wk.nt ? S.work[t] : t_fallback);
#pragma unroll
        for (int k = 0; k < kGPW; ++k)
            tr.w[k][t] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p.win_t) + (T * kNG + g0 + k) * 64 + lane);
        const u2_t sm = *(reinterpret_cast<const u2_t*>(p.win_sm) + (T * kWaves + w) * 16 + (lane & 15));
        tr.sm[0][t] = sm.x;
        tr.sm[1][t] = sm.y;
    }
}

// the wave's groups of every tile -> S.tpart[w][t][row]. Per group the four 32-column chunks are the outer
// loop and the tiles the inner one, so up to 7 independent MFMA accumulations are in flight.
template <int TB, int TE>
RK_DEV void tile_compute(const TileRegs& tr, const Work& wk, Lds& S) {
    const int lane = threadIdx.x & 63, w = wave_id(), s = lane >> 4;
    const int g0 = group0(w), ng = kGPW;
    const Int4Masks km = int4_masks();
    float acc[kMaxTiles];
#pragma unroll
    for (int t = TB; t < TE; ++t) acc[t] = 0.f;
#pragma unroll
    for (int k = 0; k < kGPW; ++k) {
        if (k < ng) {
            const int g = g0 + k;
            f4_t d[kMaxTiles];
#pragma unroll
            for (int t = TB; t < TE; ++t) d[t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int t4 = 0; t4 < 4; ++t4) {
                const h8_t A = __builtin_bit_cast(h8_t, S.hfrag[g * 16 + t4 * 4 + s]);
#pragma unroll
                for (int t = TB; t < TE; ++t)  // tiles beyond the block's count hold zero codes
                    d[t] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, dequant_frag(tr.w[k][t][t4], km), d[t], 0, 0, 0);
                __builtin_amdgcn_sched_barrier(0);  // one chunk's fragments live at a time
            }
            const float hs = S.hsum[g];
#pragma unroll
            for (int t = TB; t < TE; ++t) {
                const uint32_t sm = tr.sm[k][t];
                acc[t] = __builtin_fmaf(d[t][0], h16((uint16_t)sm), __builtin_fmaf(h16((uint16_t)(sm >> 16)), hs, acc[t]));
            }
        }
    }
    if (lane < 16)
#pragma unroll
        for (int t = TB; t < TE; ++t)
            if (t < wk.nt) S.tpart[w][t][lane] = acc[t];
}

// thread (t - tb, j): tile t's row j output, its epilogue and its publication, for tiles [tb, te)
RK_DEV void tile_epilogue(const Params& p, int l, int64_t pos, uint32_t tag, const Work& wk, Lds& S, int tb,
                          int te) {
    const int tid = threadIdx.x;
    const int t = tb + (tid >> 4), j = tid & 15;
    const bool mine = t < te && t < wk.nt;
    if (mine) {
        float y = 0.f;
#pragma unroll
        for (int w = 0; w < kWaves; ++w) y += S.tpart[w][t][j];
        S.ty[t][j] = rnd16(y);  // the projection output in fp16 (the reference's buf_in)
    }
    __syncthreads();
    if (!mine) return;
    const int NH = p.NH, NKV = p.NKV;
    const int T = S.work[t];
    const int row = T * 16 + j;
    const int qk_rows = (NH + NKV) * kHD, v_end = (NH + 2 * NKV) * kHD;
    const float y = S.ty[t][j];
    if (row < qk_rows) {
        float out = y;
        if ((p.sliding >> l) & 1ull) {  // interleaved RoPE: pairs (2i, 2i + 1)
            const int dd = row % kHD;
            const float c = S.rcos[dd >> 1], sn = S.rsin[dd >> 1];
            const float partner = S.ty[t][j ^ 1];
            out = (dd & 1) ? (y * c + partner * sn) : (y * c - partner * sn);
        }
        out = rnd16(out);
        if (row < NH * kHD) {
            st_coh(p.tq + row, tword(out, tag));
        } else {
            const int r2 = row - NH * kHD;
            st_coh(p.tkv + r2, tword(out, tag));
            p.kc[(((size_t)l * NKV + r2 / kHD) * p.S + pos) * kHD + r2 % kHD] = f16b(out);
        }
    } else if (row < v_end) {
        const int r2 = row - qk_rows;
        st_coh(p.tkv + NKV * kHD + r2, tword(y, tag));
        p.vc[(((size_t)l * NKV + r2 / kHD) * p.S + pos) * kHD + r2 % kHD] = f16b(y);
    } else if (j < 8) {  // gate row j, up row j + 8 of MLP channel 8 * (tile - qkv tiles) + j
        const float up = S.ty[t][j + 8];
        const int ch = (T - v_end / 16) * 8 + j;
        if (ch >= wk.sb * 16 && ch < wk.se * 16) S.act[ch - wk.sb * 16] = rnd16(y / (1.0f + __expf(-y)) * up);
    }
}

// ---------------------------------------------------------------------------------------------- w_down slices
// streamer lane sl takes the row pairs rp = sl + 448k (rows 2rp, 2rp + 1): per slice one 16-byte load of codes
// (wd_t: per (layer, slice), 2048 rows x 8 bytes), per 128-column group one 8-byte load of scale | min << 16
struct DownRegs {
    u4_t c[kRP][kMaxSlices];
    u2_t sm[kRP][2];  // the block's slices span at most two groups
};

// row-pair sets [KB, KE) of the lane (the whole set at once, or in pieces to pace the issue)
template <int KB = 0, int KE = kRP>
RK_DEV void down_issue(const Params& p, int l, const Work& wk, DownRegs& dr) {
    const int sl = threadIdx.x - 64;
    const int nsl = p.inter / 16, ngd = p.inter / 128;
    const int gb = wk.sb / 8;
#pragma unroll
    for (int k = KB; k < KE; ++k) {
        const int rp = min(sl + kSLanes * k, kH / 2 - 1);
#pragma unroll
        for (int i = 0; i < kMaxSlices; ++i)
            dr.c[k][i] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p.wd_t) +
                                                    ((size_t)l * nsl + min(wk.sb + i, nsl - 1)) * (kH / 2) + rp);
#pragma unroll
        for (int q = 0; q < 2; ++q)
            dr.sm[k][q] = *reinterpret_cast<const u2_t*>(p.wd_sm + ((size_t)l * ngd + min(gb + q, ngd - 1)) * kH + 2 * rp);
    }
}

// partial down output of this block's channels for all 2048 rows, published tagged. tdp is laid out
// [consumer block][producer block][8 rows]: a consumer's rows from all producers form one contiguous 8 KB run, so
// its polls touch 64 cache lines instead of one line per producer.
RK_DEV void down_compute(const Params& p, uint32_t tag, const Work& wk, const DownRegs& dr, const Lds& S) {
    const int sl = threadIdx.x - 64;
    const Int4Masks km = int4_masks();
    const int gb = wk.sb / 8;
    uint32_t xp[kMaxSlices][8];
    float asum[kMaxSlices];
#pragma unroll
    for (int i = 0; i < kMaxSlices; ++i) {
        asum[i] = 0.f;
        const float* a = S.act + 16 * i;
#pragma unroll
        for (int e = 0; e < 2; ++e)  // dword e holds codes 8e..8e+7: pairs (a0, a4), (a1, a5), ...
#pragma unroll
            for (int k = 0; k < 4; ++k) xp[i][4 * e + k] = pack_h2(a[8 * e + k], a[8 * e + k + 4]);
#pragma unroll
        for (int c = 0; c < 16; ++c) asum[i] += a[c];
    }
    uint64_t* out = reinterpret_cast<uint64_t*>(p.tdp) + (size_t)blockIdx.x * 4;  // + (consumer * nb) * 4 + pair
#pragma unroll
    for (int k = 0; k < kRP; ++k) {
        const int rp = min(sl + kSLanes * k, kH / 2 - 1);  // the clamped lanes rewrite the last pair's own value
        {
            float d[2] = {0.f, 0.f};
#pragma unroll
            for (int i = 0; i < kMaxSlices; ++i) {
                if (wk.sb + i < wk.se) {
                    const int q = (wk.sb + i) / 8 - gb;
#pragma unroll
                    for (int h = 0; h < 2; ++h) {  // row 2rp + h: dwords 2h, 2h + 1
                        float dot = 0.f;
#pragma unroll
                        for (int e = 0; e < 2; ++e) {
                            h2_t pr[4];
                            dequant_pairs(dr.c[k][i][2 * h + e], km, pr);
#pragma unroll
                            for (int kk = 0; kk < 4; ++kk) dot = dot2(pr[kk], as_h2(xp[i][4 * e + kk]), dot);
                        }
                        const uint32_t sm = q == 0 ? dr.sm[k][0][h] : dr.sm[k][1][h];
                        d[h] = __builtin_fmaf(dot, h16((uint16_t)sm),
                                              __builtin_fmaf(h16((uint16_t)(sm >> 16)), asum[i], d[h]));
                    }
                }
            }
            st_coh64(out + (size_t)(rp >> 2) * gridDim.x * 4 + (rp & 3), tpair(d[0], d[1], tag));
        }
    }
}

// ---------------------------------------------------------------------------------------------- attention
// slots per attention split: n / nsp rounded up to 8, at least kMinChunk (short contexts use fewer, fuller splits,
// so the combine waits on fewer blocks)
constexpr int kMinChunk = 16;
RK_DEV int split_chunk(int n, int nsp) { return max(kMinChunk, ((n + nsp - 1) / nsp + 7) & ~7); }

struct Split {
    bool att;           // this block runs a split
    int g, sp, start, end, n, ch;
};

RK_DEV Split split_of(const Params& p, int64_t pos) {
    Split s;
    s.att = (int)blockIdx.x < p.NKV * p.nsp;
    s.g = s.att ? blockIdx.x / p.nsp : 0;
    s.sp = s.att ? blockIdx.x % p.nsp : 0;
    s.n = (int)min<int64_t>(pos + 1, (int64_t)p.S);
    s.ch = split_chunk(s.n, p.nsp);
    s.start = s.sp * s.ch;
    s.end = s.att ? min(s.start + s.ch, s.n) : s.start;
    return s;
}

struct KVRegs {
    uint32_t k[kKVPre], v[kKVPre];
};

// cached slots start + sw + 7u (u < kKVPre) of this block's split; slot pos is read from the tagged copy. Every
// lane loads kKVPre slots (clamped into the cache), used or not.
RK_DEV void kv_issue(const Params& p, int l, int64_t pos, KVRegs& kv) {
    const int lane = threadIdx.x & 63, sw = (threadIdx.x >> 6) - 1;
    const Split s = split_of(p, pos);
    const size_t base = (((size_t)l * p.NKV + s.g) * p.S) * kHD;
    const uint32_t* kr = reinterpret_cast<const uint32_t*>(p.kc + base);
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(p.vc + base);
#pragma unroll
    for (int u = 0; u < kKVPre; ++u) {
        const int t = min(s.start + sw + kStreamers * u, p.S - 1);
        kv.k[u] = kr[(size_t)t * (kHD / 2) + lane];
        kv.v[u] = vr[(size_t)t * (kHD / 2) + lane];
    }
}

// wave 0: q of the block's KV head (REP heads) and, when the split holds pos, k / v at pos -> LDS
RK_DEV bool q_poll(const Params& p, int rep, int64_t pos, uint32_t tag, Lds& S) {
    const int lane = threadIdx.x & 63;
    const Split s = split_of(p, pos);
    if (!s.att) return true;
    const bool has_pos = s.start <= pos && pos < s.end;
    const uint32_t z = opaque_vgpr(0u);  // not hoistable: see x_poll
    const uint64_t* tq = reinterpret_cast<const uint64_t*>(p.tq) + z;
    const uint64_t* tkv = reinterpret_cast<const uint64_t*>(p.tkv) + z;
    uint32_t v[kMaxRep + 2];
    const bool ok = poll_pairs<kMaxRep + 2>(
        p, tag,
        [&](int k) -> const uint64_t* {
            if (k < kMaxRep) return k < rep ? tq + (size_t)(s.g * rep + k) * (kHD / 2) + lane : nullptr;
            if (!has_pos) return nullptr;
            return tkv + (size_t)((k - kMaxRep) * p.NKV + s.g) * (kHD / 2) + lane;
        },
        v, 0);  // no pre-wait: the poll starts after the second tile pass, well after q was written
#pragma unroll
    for (int k = 0; k < kMaxRep; ++k)
        if (k < rep) S.qs[k][lane] = v[k];
    if (has_pos) {
        S.knew[lane] = v[kMaxRep];
        S.vnew[lane] = v[kMaxRep + 1];
    }
    return ok;
}

// streamers: online softmax over the split's slots for the REP heads, merged over the streamers in LDS, then the
// normalized partial (o / l, m, l) of each head published tagged
template <int REP>
RK_DEV void attention(const Params& p, int l, int64_t pos, uint32_t tag, const KVRegs& kv, Lds& S) {
    const int tid = threadIdx.x, lane = tid & 63, sw = (tid >> 6) - 1;
    const Split s = split_of(p, pos);
    if (sw >= 0) {
        h2_t qv[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) qv[r] = as_h2(S.qs[r][lane]);
        float m[REP], lsum[REP];
        float2 acc[REP];
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            m[r] = -INFINITY;
            lsum[r] = 0.f;
            acc[r] = make_float2(0.f, 0.f);
        }
        const size_t base = (((size_t)l * p.NKV + s.g) * p.S) * kHD;
        const uint32_t* kr = reinterpret_cast<const uint32_t*>(p.kc + base);
        const uint32_t* vr = reinterpret_cast<const uint32_t*>(p.vc + base);
        for (int u = 0; s.start + sw + kStreamers * u < s.end; ++u) {
            const int t = s.start + sw + kStreamers * u;
            uint32_t kw, vw;
            if (t == pos) {
                kw = S.knew[lane];
                vw = S.vnew[lane];
            } else if (u < kKVPre) {
                kw = kv.k[0];
                vw = kv.v[0];
#pragma unroll
                for (int uu = 1; uu < kKVPre; ++uu)
                    if (u == uu) {
                        kw = kv.k[uu];
                        vw = kv.v[uu];
                    }
            } else {  // beyond the prefetched slots (long contexts with few splits)
                kw = kr[(size_t)t * (kHD / 2) + lane];
                vw = vr[(size_t)t * (kHD / 2) + lane];
            }
            const h2_t kp = as_h2(kw), vp = as_h2(vw);
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
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            if (lane == 0) {
                S.s_m[sw][r] = m[r];
                S.s_l[sw][r] = lsum[r];
            }
            S.s_acc[sw][r][lane] = acc[r];
        }
    }
    __syncthreads();
    if (!s.att) return;
    for (int e = tid - 64; e >= 0 && e < REP * 64; e += kSLanes) {  // streamer thread = (head r, dim pair d2)
        const int r = e >> 6, d2 = e & 63;
        float M = -INFINITY;
#pragma unroll
        for (int w = 0; w < kStreamers; ++w) M = fmaxf(M, S.s_m[w][r]);
        float Lt = 0.f, ax = 0.f, ay = 0.f;
#pragma unroll
        for (int w = 0; w < kStreamers; ++w) {
            const float wt = S.s_m[w][r] == -INFINITY ? 0.f : __expf(S.s_m[w][r] - M);
            Lt += wt * S.s_l[w][r];
            ax += wt * S.s_acc[w][r][d2].x;
            ay += wt * S.s_acc[w][r][d2].y;
        }
        const size_t pi = (size_t)(s.g * REP + r) * p.nsp + s.sp;
        const float inv = Lt > 0.f ? 1.0f / Lt : 0.f;
        st_coh64(reinterpret_cast<uint64_t*>(p.tpo + pi * kHD) + d2, tpair(ax * inv, ay * inv, tag));
        if (d2 == 0) {
            st_coh64(reinterpret_cast<uint64_t*>(p.tml) + 2 * pi,
                     (uint64_t)__builtin_bit_cast(uint32_t, M) | ((uint64_t)tag << 32));
            st_coh64(reinterpret_cast<uint64_t*>(p.tml) + 2 * pi + 1,
                     (uint64_t)__builtin_bit_cast(uint32_t, Lt) | ((uint64_t)tag << 32));
        }
    }
}

// Head h's combine: out = sum_i w_i o_i / sum_i w_i, w_i = exp(m_i - max m) * l_i over the splits holding at least
// one slot (at most 64). The streamers of each of the head's 16 blocks share the polling: streamer sw polls splits
// [kCombPer * sw, kCombPer * (sw + 1)) in one batch per iteration and leaves (M = its max m, L = sum of its w_i taken
// against M, sum of w_i o_i) in LDS; after a block barrier wave 0 merges the 7 parts (comb_merge). The sums run in split order within a wave and in
// wave order across waves, so the result does not depend on arrival order.
RK_DEV int comb_splits(const Params& p, int64_t pos) {
    const int n = (int)min<int64_t>(pos + 1, (int64_t)p.S);
    const int ch = split_chunk(n, p.nsp);
    return min(p.nsp, (n + ch - 1) / ch);
}

constexpr int kCombPer = 10;  // splits per streamer (7 x 10 >= 64)

RK_DEV bool comb_part(const Params& p, int h, int64_t pos, uint32_t tag, Lds& S) {
    const int lane = threadIdx.x & 63, sw = (threadIdx.x >> 6) - 1;
    const int nsp = p.nsp, i0 = kCombPer * sw;
    const int cnt = min(max(comb_splits(p, pos) - i0, 0), kCombPer);
    float M = -INFINITY, L = 0.f, ax = 0.f, ay = 0.f;
    bool ok = true;
    if (cnt > 0) {
        const size_t hb = (size_t)h * nsp;
        const uint32_t z = opaque_vgpr(0u);  // not hoistable: see x_poll
        const uint64_t* po = reinterpret_cast<const uint64_t*>(p.tpo + hb * kHD) + lane + z;
        // lane j < kCombPer brings split i0 + j's (m, l); the other lanes repeat one of those loads
        const int jl = lane % kCombPer;
        const uint64_t* tml = reinterpret_cast<const uint64_t*>(p.tml) + 2 * (hb + min(i0 + jl, nsp - 1)) + z;
        const uint64_t t0 = wall_clock64();
        uint32_t pending = (1u << cnt) - 1;
        bool ml_done = jl >= cnt;
        float mi = -INFINITY, li = 0.f;
        uint32_t val[kCombPer];
        while (true) {
            // one batch per iteration (see poll_pairs): the splits' pairs, the (m, l) words and the status
            uint64_t q[kCombPer];
#pragma unroll
            for (int k = 0; k < kCombPer; ++k) q[k] = ld_coh64(po + (size_t)min(i0 + k, nsp - 1) * (kHD / 2));
            const uint64_t qm = ld_coh64(tml), ql = ld_coh64(tml + 1);
            const uint32_t st = ld_coh(p.status);
#pragma unroll
            for (int k = 0; k < kCombPer; ++k)
                if ((pending & (1u << k)) && __all(pair_ok(q[k], tag))) {
                    val[k] = pair_val(q[k]);
                    pending &= ~(1u << k);
                }
            if (!ml_done && (uint32_t)(qm >> 32) == tag && (uint32_t)(ql >> 32) == tag) {
                mi = __builtin_bit_cast(float, (uint32_t)qm);
                li = __builtin_bit_cast(float, (uint32_t)ql);
                ml_done = true;
            }
            if (pending == 0 && __all(ml_done)) break;
            if (!wait_more(p, t0, st)) {
                ok = false;
                break;
            }
        }
        if (ok) {
            // lanes 0..kCombPer-1 hold the splits' (m, l): the max, then each split's weight, broadcast by readlane
            M = -INFINITY;
#pragma unroll
            for (int k = 0; k < kCombPer; ++k)
                if (k < cnt) M = fmaxf(M, __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, mi), k)));
            const float wl = (jl < cnt && mi != -INFINITY) ? __expf(mi - M) * li : 0.f;
#pragma unroll
            for (int k = 0; k < kCombPer; ++k) {
                const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k));
                const h2_t o = as_h2(k < cnt ? val[k] : 0u);
                ax = __builtin_fmaf(wk, (float)o.x, ax);
                ay = __builtin_fmaf(wk, (float)o.y, ay);
                L += wk;
            }
        }
    }
    S.cpa[sw][lane] = make_float2(ax, ay);
    if (lane == 0) {
        S.cpm[sw] = M;
        S.cpl[sw] = L;
    }
    return ok;
}

// wave 0, after the barrier that follows the streamers' comb_part: merge the parts into head h's attention output,
// rounded to fp16 (the reference keeps it in the activation dtype), staged as natural pairs with the sum of its 128
// values (for the min term of the o projection)
RK_DEV void comb_merge(Lds& S) {
    const int lane = threadIdx.x & 63;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kStreamers; ++w) M = fmaxf(M, S.cpm[w]);
    float den = 0.f, ox = 0.f, oy = 0.f;
#pragma unroll
    for (int w = 0; w < kStreamers; ++w) {
        const float f = S.cpm[w] == -INFINITY ? 0.f : __expf(S.cpm[w] - M);
        const float2 a = S.cpa[w][lane];
        den = __builtin_fmaf(f, S.cpl[w], den);
        ox = __builtin_fmaf(f, a.x, ox);
        oy = __builtin_fmaf(f, a.y, oy);
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    const float a0 = rnd16(ox * inv), a1 = rnd16(oy * inv);
    S.attn[lane] = pack_h2(a0, a1);
    const float sum = wave_sum(a0 + a1);
    if (lane == 0) S.asum = sum;
}

// ---------------------------------------------------------------------------------------------- w_o partials
// Block b = (head h = b / 16, row group r = b % 16) computes the o projection of head h's attention output for
// rows [128r, 128r + 128): 512 items (row i / 4, 32-column chunk i % 4 of the head's 128 columns), one 16-byte load
// each. Streamer lane s takes item s, streamer 0's lanes also item 448 + lane. The head's 128 columns are one
// quantization group, so each row has one scale | min word (wo_sm[layer][row][head]).
constexpr int kOItems = 512;

struct ORegs {
    u4_t w[2];
    uint32_t sm[2];
};

static_assert(kH / kHD == 16 && kH / 128 == 16, "16 heads x 16 row groups of 128 = the 256 blocks");
RK_DEV int o_head() { return blockIdx.x >> 4; }
RK_DEV int o_rgroup() { return blockIdx.x & 15; }

RK_DEV void o_issue(const Params& p, int l, ORegs& o) {
    const int ls = threadIdx.x - 64;
    const int h = o_head(), r = o_rgroup();
    const u4_t* base = reinterpret_cast<const u4_t*>(p.wo_q) + ((size_t)(l * p.NH + h) * 16 + r) * kOItems;
#pragma unroll
    for (int k = 0; k < 2; ++k) {  // lanes without a second item load their first one again (unused)
        const int i = k == 1 && ls < kOItems - kSLanes ? ls + kSLanes : ls;
        o.w[k] = __builtin_nontemporal_load(base + i);
        o.sm[k] = p.wo_sm[((size_t)l * kH + 128 * r + (i >> 2)) * p.NH + h];
    }
}

// the items' dots, summed per row over the 4 lanes of its chunks; lanes i % 8 == 0 publish rows (i/4, i/4 + 1) as
// one tagged pair to top[consumer block][head][8 rows]
RK_DEV void o_part(const Params& p, uint32_t tag, const ORegs& o, const Lds& S) {
    const int ls = threadIdx.x - 64, lane = threadIdx.x & 63;
    const int h = o_head(), r = o_rgroup();
    const Int4Masks km = int4_masks();
    uint64_t* top = reinterpret_cast<uint64_t*>(p.top);
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        if (k == 1 && ls >= kOItems - kSLanes) break;  // wave-uniform: only streamer 0 has a second item
        const int i = ls + k * kSLanes, c = i & 3;
        uint32_t xp[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // natural pairs of 8 columns -> the dequant's pair order
            const u4_t d = {S.attn[16 * c + 4 * q], S.attn[16 * c + 4 * q + 1], S.attn[16 * c + 4 * q + 2],
                            S.attn[16 * c + 4 * q + 3]};
            uint32_t hp[4];
            pair_permute(d, hp);
#pragma unroll
            for (int e = 0; e < 4; ++e) xp[4 * q + e] = hp[e];
        }
        float v = chunk_dot_int4(o.w[k], xp, km);
        v += dpp<0xB1>(v);  // the row's 4 chunks sit in lanes 4j .. 4j + 3
        v += dpp<0x4E>(v);
        v = __builtin_fmaf(v, h16((uint16_t)o.sm[k]), h16((uint16_t)(o.sm[k] >> 16)) * S.asum);
        const float nxt = __shfl_down(v, 4);  // the next row's total (lane + 4)
        if ((lane & 7) == 0) {
            const int row = 128 * r + (i >> 2);  // even
            st_coh64(top + ((size_t)(row >> 3) * p.NH + h) * 4 + ((row & 7) >> 1), tpair(v, nxt, tag));
        }
    }
}

// wave 0: this block's 8 rows of the down partials of all blocks and of the o partials of all heads, one poll
// batch; each summed over its producers (-> S.drow, S.orow)
RK_DEV bool gather_rows(const Params& p, uint32_t tag, Lds& S, int pre) {
    const int lane = threadIdx.x & 63;
    const int nb = gridDim.x;  // at most 256 down producers, 4 qwords (8 rows) each: 16 qwords per lane
    const uint32_t z = opaque_vgpr(0u);  // not hoistable: see x_poll
    // down: qword q = 64k + lane of this block's run: producer q / 4, rows 2(q % 4), 2(q % 4) + 1;
    // o: lane = head * 4 + pair (16 heads)
    const uint64_t* run = reinterpret_cast<const uint64_t*>(p.tdp + z) + (size_t)blockIdx.x * nb * 4;
    const uint64_t* orun = reinterpret_cast<const uint64_t*>(p.top + z) + (size_t)blockIdx.x * p.NH * 4;
    uint32_t v[17];
    const bool ok = poll_pairs<17>(
        p, tag,
        [&](int k) -> const uint64_t* {
            if (k == 16) return lane < 4 * p.NH ? orun + lane : nullptr;
            return 64 * k + lane < 4 * nb ? run + 64 * k + lane : nullptr;
        },
        v, pre);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int k = 0; k < 16; ++k) {
        if (64 * k + lane < 4 * nb) {
            const h2_t h = as_h2(v[k]);
            d0 += (float)h.x;
            d1 += (float)h.y;
        }
    }
    float o0 = 0.f, o1 = 0.f;
    if (lane < 4 * p.NH) {
        const h2_t h = as_h2(v[16]);
        o0 = (float)h.x;
        o1 = (float)h.y;
    }
    // sum over the lanes that share lane % 4
#pragma unroll
    for (int m = 4; m < 64; m *= 2) {
        d0 += __shfl_xor(d0, m);
        d1 += __shfl_xor(d1, m);
        o0 += __shfl_xor(o0, m);
        o1 += __shfl_xor(o1, m);
    }
    if (lane < 4) {
        S.drow[2 * lane] = d0;
        S.drow[2 * lane + 1] = d1;
        S.orow[2 * lane] = o0;
        S.orow[2 * lane + 1] = o1;
    }
    return ok;
}

// ---------------------------------------------------------------------------------------------- head
// The head rows are loaded into the tile registers (free after the last layer's tiles): streamer sw's row k
// (r0 + sw + 7k, k < kHeadRows) half j goes to flat entry 2k + j of TileRegs::w.
static_assert(2 * kHeadRows <= kGPW * kMaxTiles, "head rows fit the tile registers");

RK_DEV u4_t& head_slot(TileRegs& tr, int e) { return tr.w[e / kMaxTiles][e % kMaxTiles]; }
RK_DEV const u4_t& head_slot(const TileRegs& tr, int e) { return tr.w[e / kMaxTiles][e % kMaxTiles]; }

RK_DEV void head_rows(const Params& p, int& r0, int& r1) {
    const int per = (p.n_audio + gridDim.x - 1) / gridDim.x;
    r0 = min(p.n_audio, (int)blockIdx.x * per);
    r1 = min(p.n_audio, r0 + per);
}

RK_DEV void head_issue(const Params& p, TileRegs& tr) {
    const int lane = threadIdx.x & 63, sw = (threadIdx.x >> 6) - 1;
    int r0, r1;
    head_rows(p, r0, r1);
#pragma unroll
    for (int k = 0; k < kHeadRows; ++k) {
        const int r = min(r0 + sw + kStreamers * k, p.n_audio - 1);
        const u4_t* qr = reinterpret_cast<const u4_t*>(p.head_q + (size_t)r * kH);
#pragma unroll
        for (int j = 0; j < 2; ++j) head_slot(tr, 2 * k + j) = __builtin_nontemporal_load(qr + lane + 64 * j);
    }
}

RK_DEV void head_compute(const Params& p, const TileRegs& tr, const Lds& S) {
    const int lane = threadIdx.x & 63, sw = (threadIdx.x >> 6) - 1;
    int r0, r1;
    head_rows(p, r0, r1);
    for (int k = 0; r0 + sw + kStreamers * k < r1; ++k) {
        const int r = r0 + sw + kStreamers * k;
        u4_t w[2];
        if (k < kHeadRows) {
            w[0] = head_slot(tr, 0);
            w[1] = head_slot(tr, 1);
#pragma unroll
            for (int kk = 1; kk < kHeadRows; ++kk)
                if (k == kk) {
                    w[0] = head_slot(tr, 2 * kk);
                    w[1] = head_slot(tr, 2 * kk + 1);
                }
        } else {
            const u4_t* qr = reinterpret_cast<const u4_t*>(p.head_q + (size_t)r * kH);
            w[0] = qr[lane];
            w[1] = qr[lane + 64];
        }
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

// ---------------------------------------------------------------------------------------------- the step
// Wave 0 and the streamers run separate code (so each role's registers are allocated for its own peak, not the
// sum) and meet at the same sequence of block barriers per layer:
//   B0 x + LN statistics staged | B1 h staged | B2 partials of tiles [0, 3) | B3 (epilogue) | B4 q / k / v of
//   those tiles published | B5 partials of tiles [3, 7), q staged | B6 (epilogue) | B7 act staged |
//   B8 (attention) | BC combine parts of head b / 16 staged | BO its attention output staged | B9 the streamers'
//   next-layer loads issued; wave 0 reaches B9 only after its row gather, the x publication, the next layer's x
//   poll and LayerNorm statistics (so it passes B9 and B0 back to back; nothing in LDS needs B9 earlier).
//   Head: H0 LN statistics staged | H1 h staged.
// The work table lists a block's q / k / v tiles first (at most kTileSplit), so they are computed and published in
// the first pass and the q / k / v hop overlaps the second pass. This is required, not only faster: a q / k / v tile
// in the second pass would be published after B5, which waits for wave 0's q poll, which may wait for that very
// tile in another block -- a circular wait that ends in the timeout. Measured first-pass sizes (ctx 256 / 2048, us
// per token): 1 726 / 799, 2 697 / 767, 3 664 / 740, 4 692 / 769, 5 712 / 802.
// Streamer issue order (each wait covers only older loads, see tile_issue): tiles(l + 1) [0, 3) after the first
// epilogue; after the o partials of layer l, paced (pace_wait): tiles(l + 1) [3, 7), K/V(l + 1), down(l + 1),
// O(l + 1) -- the order layer l + 1 consumes them. The loop's back edge and its preheader leave the same sequence
// outstanding. At most ~57 vector-memory instructions are in
// flight per streamer (the hardware counter holds 63).

template <int REP>
RK_DEV void poller_main(const Params& p, uint32_t step, int64_t pos, int64_t tok, const Work& wk, Lds& S) {
    const int lane = threadIdx.x & 63;
    TileRegs tr;  // wave 0's two column groups of the block's tiles, issued a layer ahead (before the x poll)
    tile_issue(p, 0, S, wk, tr, 0, kMaxTiles);
    for (int l = 0; l < p.L; ++l) {
        const uint32_t tag = tag_of(step, l);
        XWave xw;
        LnW lw;
        ln_w_issue(p.ln_w + (size_t)l * kH, lw);
        if (l == 0) {
            x_from_embedding(p, tok, xw);
        } else {
            x_poll(p, tag_of(step, l - 1), xw);
            if (l == 1 && blockIdx.x == 0 && lane == 0) p.pos[0] = pos + 1;  // every block has read pos
        }
        ln_stats(xw, lw, p.eps, S);
        if (l > 0) __syncthreads();                           // B9 of layer l - 1 (after the row gather, the x
                                                              // publication and this layer's x poll)
        __syncthreads();                                      // B0
        ln_apply_frag(S);
        __syncthreads();                                      // B1
        tile_compute<0, kTileSplit>(tr, wk, S);
        __syncthreads();                                      // B2
        tile_epilogue(p, l, pos, tag, wk, S, 0, kTileSplit);  // B3 inside
        __syncthreads();                                      // B4
        tile_compute<kTileSplit, kMaxTiles>(tr, wk, S);
        q_poll(p, REP, pos, tag, S);
        __syncthreads();                                      // B5
        tile_epilogue(p, l, pos, tag, wk, S, kTileSplit, kMaxTiles);  // B6 inside
        __syncthreads();                                      // B7
        __syncthreads();                                      // B8
        __syncthreads();                                      // BC
        comb_merge(S);
        __syncthreads();                                      // BO
        gather_rows(p, tag, S, kPreRows);
        if (lane < 8) S.xrow[lane] = rnd16(S.xrow[lane] + rnd16(S.orow[lane]) + rnd16(S.drow[lane]));
        static_assert(4 * kXRep <= 64, "one store per lane");
        if (lane < 4 * kXRep)  // lane = copy * 4 + pair
            st_coh64(reinterpret_cast<uint64_t*>(p.tx) + (lane >> 2) * kRepQwords + 4 * blockIdx.x + (lane & 3),
                     tpair(S.xrow[2 * (lane & 3)], S.xrow[2 * (lane & 3) + 1], tag));
        tile_issue(p, l + 1 < p.L ? l + 1 : l, S, wk, tr, 0, kMaxTiles);
    }
    // final LayerNorm, h as natural pairs for the int8 head
    XWave xw;
    LnW lw;
    ln_w_issue(p.norm_w, lw);
    x_poll(p, tag_of(step, p.L - 1), xw);
    if (p.L == 1 && blockIdx.x == 0 && lane == 0) p.pos[0] = pos + 1;
    ln_stats(xw, lw, p.eps, S);
    __syncthreads();                                          // B9 of the last layer
    __syncthreads();                                          // H0
    ln_apply_pairs(S);
    __syncthreads();                                          // H1
    if (p.hn && blockIdx.x == 0)  // the final hidden state (the sampler's stop predictor reads it)
        for (int i = lane; i < kH / 8; i += 64) reinterpret_cast<uint4*>(p.hn)[i] = S.vecp[i];
}

template <int REP>
RK_DEV void streamer_main(const Params& p, int64_t pos, uint32_t step, const Work& wk, Lds& S) {
    TileRegs tr;
    DownRegs dr;
    KVRegs kv;
    ORegs orr;
    // the same outstanding sequence the loop leaves behind at its back edge, in the order the layer consumes it:
    // tiles [0, 3), tiles [3, 7), K/V, down, O
    tile_issue(p, 0, S, wk, tr, 0, kTileSplit);
    tile_issue(p, 0, S, wk, tr, kTileSplit, kMaxTiles);
    kv_issue(p, 0, pos, kv);
    down_issue(p, 0, wk, dr);
    o_issue(p, 0, orr);
    for (int l = 0; l < p.L; ++l) {
        const uint32_t tag = tag_of(step, l);
        const int ln = l + 1 < p.L ? l + 1 : l;  // the last layer re-issues its own (cache-resident) weights
        __syncthreads();                                      // B0
        ln_apply_frag(S);
        __syncthreads();                                      // B1
        tile_compute<0, kTileSplit>(tr, wk, S);
        __syncthreads();                                      // B2
        tile_epilogue(p, l, pos, tag, wk, S, 0, kTileSplit);  // B3 inside
        __syncthreads();                                      // B4
        tile_issue(p, ln, S, wk, tr, 0, kTileSplit);          // next layer's tiles, first part
        tile_compute<kTileSplit, kMaxTiles>(tr, wk, S);
        __syncthreads();                                      // B5
        tile_epilogue(p, l, pos, tag, wk, S, kTileSplit, kMaxTiles);  // B6 inside
        __syncthreads();                                      // B7
        attention<REP>(p, l, pos, tag, kv, S);                // B8 inside
        down_compute(p, tag, wk, dr, S);
        comb_part(p, o_head(), pos, tag, S);
        __syncthreads();                                      // BC
        __syncthreads();                                      // BO
        o_part(p, tag, orr, S);
        // the next layer's loads in the order they are consumed, paced (wave 0 meanwhile gathers rows, publishes x,
        // polls it back and computes the next LayerNorm statistics; it meets the streamers at B9)
#pragma unroll
        for (int t = kTileSplit; t < kMaxTiles; ++t) {
            tile_issue(p, ln, S, wk, tr, t, t + 1);           // second part, one tile at a time
            pace_wait(kPace);
        }
        kv_issue(p, ln, pos, kv);
        pace_wait(kPace);
        static_assert(kRP == 3, "three down pieces");
        down_issue<0, 1>(p, ln, wk, dr);
        pace_wait(kPace / 2);
        down_issue<1, 2>(p, ln, wk, dr);
        pace_wait(kPace / 2);
        down_issue<2, 3>(p, ln, wk, dr);
        pace_wait(kPace / 2);
        o_issue(p, ln, orr);
        __syncthreads();                                      // B9
    }
    head_issue(p, tr);
    __syncthreads();                                          // H0
    ln_apply_pairs(S);
    __syncthreads();                                          // H1
    head_compute(p, tr, S);
}

template <int REP>
__global__ __launch_bounds__(kThreads) void decode_step_kernel(Params p) {
    extern __shared__ __align__(16) uint8_t smem_raw[];
    Lds& S = *reinterpret_cast<Lds*>(smem_raw);
    const int tid = threadIdx.x;
    const int64_t pos = p.pos[0];
    const int64_t tok = p.tok[0];
    if (pos < 0 || pos >= p.S) {  // no cache slot for this position: every block leaves at once
        if (blockIdx.x == 0 && tid == 0) atomicOr(p.status, kBadPos);
        return;
    }
    const uint32_t step = p.ctr[blockIdx.x];
    if (tid < kWork) S.work[tid] = p.work[(size_t)blockIdx.x * kWork + tid];
    if (tid < kHD / 2) {  // the table holds each angle twice (pair elements 2i, 2i + 1)
        S.rcos[tid] = h16(p.cos_t[(size_t)pos * kHD + 2 * tid]);
        S.rsin[tid] = h16(p.sin_t[(size_t)pos * kHD + 2 * tid]);
    }
    if (tid < 8) S.xrow[tid] = rnd16((float)p.emb_q[(size_t)tok * kH + 8 * blockIdx.x + tid] * h16(p.emb_s[tok]));
    __syncthreads();
    const Work wk = work_of(S);
    if (tid < 64)
        poller_main<REP>(p, step, pos, tok, wk, S);
    else
        streamer_main<REP>(p, pos, step, wk, S);
    if (tid == 0) p.ctr[blockIdx.x] = step + 1;
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
    if (p.inter <= 0 || p.inter % 128 || p.inter > 11008) return RK_ERR_SHAPE;
    if (nblocks <= 0 || nblocks * 8 != kH) return RK_ERR_BLOCK;  // block b owns rows [8b, 8b + 8)
    if (p.nsp <= 0 || p.nsp > 64 || p.NKV * p.nsp > nblocks || p.inter / 16 > kMaxSlices * nblocks ||
        (p.S + p.nsp - 1) / p.nsp > kStreamers * kKVPre)  // every cached slot of a split is prefetched
        return RK_ERR_BLOCK;
    if (!p.tok || !p.pos || !p.emb_q || !p.emb_s || !p.win_t || !p.win_sm || !p.wo_q || !p.wo_sm ||
        !p.wd_t || !p.wd_sm || !p.ln_w || !p.norm_w || !p.cos_t || !p.sin_t || !p.kc || !p.vc || !p.head_q ||
        !p.head_s || !p.logits || !p.work || !p.tx || !p.tq || !p.tkv || !p.top || !p.tdp || !p.tpo || !p.tml ||
        !p.ctr || !p.status)
        return RK_ERR_NULL;
    if (!co_resident(rep, nblocks)) return RK_ERR_BLOCK;  // the waits need every block resident at once
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

extern "C" int rk_decode_get_limits(rk_decode_limits* out) {
    if (!out) return RK_ERR_NULL;
    out->max_tiles = kMaxTiles;
    out->first_pass = kTileSplit;
    out->max_slices = kMaxSlices;
    out->work_stride = kWork;
    out->slice_begin_col = 8;
    out->slice_end_col = 9;
    out->x_copies = kXRep;
    out->max_splits = 64;
    out->max_slots_per_split = kStreamers * kKVPre;
    return RK_OK;
}
