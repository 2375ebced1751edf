// One batch-1 decode step of the Rumik decoder in ONE kernel launch (gfx950, MI355X).
//
// Why one launch: a step is ~36 x 3 dependent GEMVs plus glue. As separate kernels each pays a launch gap and a
// cold memory-latency ramp (measured 2-10 us per hipGraph node), far more than the ~330 us a 3000 tok/s step may
// take. Here a grid of one block per CU stays resident for the whole step and streams its fixed share of every
// weight matrix.
//
// Synchronization between blocks is dataflow, not grid barriers: every value one block hands to another is a
// tagged 32-bit word (fp16 value | tag << 16; the tag names the step and the layer) written with an agent-scope
// atomic store, and the consumer polls the words themselves with agent-scope atomic loads (coherent across the
// XCDs' L2s). Every poll loads all its words and the status word as one batch: one round trip per poll iteration.
//
// Inside a block the waves have fixed roles and meet through LDS flags and arrival counters, never a block
// barrier inside the layer loop, so a wave waits only for the data it consumes:
//   row waves (W0..W3 and W12..W15): each polls 256 columns of x, the eight combine their LayerNorm statistics
//     through LDS, and each stages its own two column groups of h and computes those groups of the block's first
//     w_in tile (its q / k / v tile when it has one) on the matrix cores; the last of the eight finishes that tile
//     (RoPE, K / V into the cache, q / k / v published). At the end of the layer each gathers its share of the
//     block's 8 rows of the down (and, W0, o) partials; the last arriver publishes the x rows.
//   attention waves W0..W3 (raised issue priority): q poll -> split attention -> merge (one head each) and publish
//     the split partials -> combine poll of head b / 16 -> each wave merges the four parts -> the o projection
//     slice of that head for row group b % 16 -> o partials published.
//   tile waves W4..W11: the block's other w_in tiles (pass 2, K-split: wave m computes column groups 2m, 2m + 1
//     of every tile), released once the q / k / v tile is out; the last arriver forms act = silu(gate) * up. They
//     also load tile 0's codes and copy them to LDS for the row waves.
//   down waves W12..W15: the w_down columns of the block's channels for all 2048 rows, published as partials.
// A wave that polls never has its own weight loads in flight ahead of the poll (vector-memory results return in
// issue order, and on gfx9 a wait for a load also waits for every earlier store). Weight loads are issued where
// they cannot delay the critical path: the tile waves prefetch the next layer's tiles paced, two tiles at a time
// (a chip-wide burst would queue ahead of every poll for microseconds), and the row waves issue theirs after the
// q / k / v tile is published (a load or store issued into a full memory queue stalls its wave). The dataflow
// itself orders the reuse of every LDS buffer across layers (e.g. h of layer l + 1 is written only after x of
// layer l + 1 exists, which needs this block's down partials of layer l, which need act of layer l, which its
// tile waves form after their last read of h).
//
// Every wait is bounded by wall-clock time (200 ms): on expiry the kernel sets an abort bit in `status`, every
// later wait returns at once and the grid drains with garbage results. A residual sum that leaves the fp16 range
// (or is NaN) sets a sticky status bit and the step runs on: the caller decides what to do with the token.
#include "dequant.h"

namespace {

constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
constexpr int kAW = 4;                     // attention waves W0..W3 (also row waves 0..3)
constexpr int kALanes = 64 * kAW;          // 256
constexpr int kM0 = 4;                     // first tile wave
constexpr int kMW = 8;                     // tile waves W4..W11
constexpr int kD0 = 12;                    // first down wave
constexpr int kDW = 4;                     // down waves W12..W15
constexpr int kDLanes = 64 * kDW;          // 256
constexpr int kH = 2048;                   // hidden size (compile-time: tiles and staging are sized for it)
constexpr int kRW = kAW + kDW;             // row waves (attention + down waves): x poll, LayerNorm, row gather
constexpr int kRCols = kH / kRW;           // 256 columns of x per row wave, 4 per lane
constexpr int kHD = 128;                   // head dim
constexpr int kNG = kH / 128;              // column groups of a w_in row
constexpr int kMaxRep = 8;
constexpr int kMaxTiles = 7;               // w_in tiles per block
constexpr int kGPW = 2;                    // column groups per MLP wave (8 x 2 = 16)
constexpr int kFirstPass = 1;              // q / k / v tiles per block (published before the gate / up pass)
constexpr int kMaxSlices = 3;              // w_down 16-column slices per block
constexpr int kCombPer = 16;               // splits per attention wave in the combine (4 x 16 = 64)
constexpr int kRP = kH / 2 / kDLanes;      // down row pairs per down lane (4)
constexpr int kSlotsPerWave = 8;           // cached slots per attention wave (4 x 8 = 32 per split)
constexpr int kOItems = 512;               // o items per (head, row group); 2 per attention lane
constexpr int kHeadRows = 7;               // head rows per MLP wave loaded ahead (the rest load when used)
constexpr int kWork = 16;                  // int16 entries per block in the work table
constexpr int kSliceBegin = 8, kSliceEnd = 9;
// x is polled by every block: it is published in kXRep copies 8 KB apart and block b polls copy b % kXRep, so no
// 8 KB stretch of memory serves more than 16 pollers
constexpr int kXRep = 16;
constexpr int kRepQwords = kH / 2;         // qwords per copy (2048 tagged fp16 words)
constexpr uint64_t kWaitTicks = 20000000ull;  // 200 ms at the 100 MHz wall clock
constexpr unsigned kAbort = 1u, kTimeout = 2u, kBadPos = 4u, kNonFinite = 8u;
constexpr int kMaxSplits = 64;

static_assert(kRP * kDLanes * 2 == kH, "down rows split evenly over the down lanes");
static_assert(kOItems == 2 * kALanes, "two o items per attention lane");
static_assert(kMW * kGPW == kNG, "MLP waves cover the 16 column groups");
static_assert(kAW * kCombPer >= kMaxSplits, "the combine's polls cover every split");

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

// The lane index through an empty asm: every use recomputes its lane addresses instead of the optimizer hoisting
// them out of the layer loop, where dozens of 64-bit addresses would stay live (and spill) across the whole step.
RK_DEV int lane_id() { return (int)opaque_vgpr(threadIdx.x & 63); }
RK_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

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

// ---------------------------------------------------------------------------------------------- phase trace
// A build option (RK_DECODE_TRACE; off in the product library, where every RK_TRACE is empty): wall-clock stamps per
// (layer, event), kept in LDS during the step and copied out at its end to the buffer rk_decode_trace_set names
// ([block][64 layers][kTrEvents] uint64, 100 MHz ticks). rumik-fast_amd/decode_trace.py builds and reads it.
enum TraceEvent {
    kTrXPolled,        // row wave 0: its part of x polled
    kTrLnDone,         // row wave 0: LayerNorm statistics combined, h formed
    kTrHStaged,        // row wave 0: its h groups staged
    kTrTile0Done,      // row wave 0: its part of tile 0 computed
    kTrQkvPublished,   // the last row wave: q / k / v tile published
    kTrQPolled,        // attention wave 0: q (and k / v at pos) polled
    kTrAttnDone,       // attention wave 0: its slots' attention computed
    kTrMerged,         // attention wave 0: its head's split partial published
    kTrCombDone,       // attention wave 0: its combine part formed (poll included)
    kTrCombMerged,     // attention wave 0: the head's attention output merged
    kTrOPublished,     // attention wave 0: its o partials published
    kTrPass2Start,     // tile wave W4: released for pass 2
    kTrActReady,       // the last tile wave: act formed
    kTrDownPublished,  // down wave W12: its down partials published
    kTrGatherPolled,   // row wave 0: its down / o partials polled
    kTrXPublished,     // the gather's last arriver: x rows published
    kTrXPolled4,       // row wave 4 (W12): its part of x polled
    kTrGatherPolled4,  // row wave 4 (W12): its down partials polled
    kTrEvents
};
#ifdef RK_DECODE_TRACE
__device__ unsigned long long* g_trace;
#define RK_TRACE(cond, ev)                                                             \
    do {                                                                               \
        if ((cond) && lane_id() == 0) S.trace[l][(ev)] = wall_clock64();               \
    } while (0)
#else
#define RK_TRACE(cond, ev) \
    do {                   \
    } while (0)
#endif

// ---------------------------------------------------------------------------------------------- LDS layout
struct Lds {
    uint4 hfrag[kH / 8];                      // MFMA A fragments of h
    float hsum[kNG];                          // per-group sums of h
    float tpart[kMW][kMaxTiles][16];          // K-split partial dots of the block's tiles
    uint4 t0w[kMW][kGPW][64];                 // tile 0's codes, per tile wave's group pair (read by the row waves)
    uint32_t t0sm[kMW][kGPW][16];             //   and its scale | min words
    float act[kMaxSlices * 16];               // act of the block's MLP channels
    alignas(16) uint32_t qst[kAW][kMaxRep + 1][64];  // per attention wave: q of its heads and k at pos, dim pairs
    float s_m[kAW][kMaxRep], s_l[kAW][kMaxRep];
    float2 s_acc[kAW][kMaxRep][64];           // per-wave attention partials
    float2 cpa[kAW][64];                      // the combine's per-wave parts: sum of w_i o_i per dim pair,
    float cpm[kAW], cpl[kAW];                 //   the wave's max m and sum of w_i
    uint32_t attn[kAW][kHD / 2];              // each attention wave's copy of head (block / 16)'s attention
                                              //   output, natural fp16 pairs (read back in the o slice's order)
    float2 lnst[kRW];                         // per row wave: sum and squared deviations of its 256 x values
    float2 gpart[kRW][4];                     // per row wave: its down-partial sums of the block's 4 row pairs
    float2 opart[4];                          // the o-partial sums of those row pairs
    uint4 vecp[kH / 8];                       // the final h as natural pairs (the int8 head's input)
    float rcos[kHD / 2], rsin[kHD / 2];       // RoPE cos / sin of pair i at pos
    float xrow[8];                            // this block's 8 rows of the residual stream
    int16_t work[kWork];
    // intra-block synchronization: flags hold the layer + 1 they announce, counters count arrivals
#ifdef RK_DECODE_TRACE
    unsigned long long trace[64][kTrEvents];
#endif
    uint32_t p1_done, act_ready;
    uint32_t cnt_ln, cnt_h, cnt_g, cnt_head, cnt_t0, cnt_p1, cnt_p2, cnt_att, cnt_comb;
    uint32_t abort;
};

// ---------------------------------------------------------------------------------------------- waits
// true while a wait may go on; on expiry raise the abort bit (globally and in this block). `status` is the status
// word loaded in the same batch as the poll it belongs to (one round trip per poll iteration).
RK_DEV bool wait_more(const Params& p, Lds& S, uint64_t t0, uint32_t status) {
    if (status & kAbort) {
        S.abort = 1u;
        return false;
    }
    if (wall_clock64() - t0 > kWaitTicks) {
        if (lane_id() == 0) atomicOr(p.status, kAbort | kTimeout);
        S.abort = 1u;
        return false;
    }
    __builtin_amdgcn_s_sleep(1);
    return true;
}

// One lane per wave arrives at an LDS counter; true (in every lane) for the wave whose arrival brings it to
// `target`. The release fence covers every lane's earlier LDS writes; the acquire makes the other waves' writes
// visible to the last arriver.
RK_DEV bool arrive_last(uint32_t* ctr, uint32_t target) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    uint32_t old = 0;
    if (lane_id() == 0) old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = __builtin_amdgcn_readfirstlane(old);
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    return old + 1 == target;
}

RK_DEV void flag_set(uint32_t* f, uint32_t v) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane_id() == 0) __hip_atomic_store(f, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// spin until the LDS flag reaches v; false after an abort or a timeout
RK_DEV bool flag_wait(const Params& p, Lds& S, const uint32_t* f, uint32_t v) {
    const uint64_t t0 = wall_clock64();
    for (int it = 0;; ++it) {
        const uint32_t cur =
            __builtin_amdgcn_readfirstlane(__hip_atomic_load(const_cast<uint32_t*>(f), __ATOMIC_RELAXED,
                                                             __HIP_MEMORY_SCOPE_WORKGROUP));
        if (cur >= v) break;
        if (__builtin_amdgcn_readfirstlane(S.abort)) return false;
        if ((it & 31) == 31 && wall_clock64() - t0 > kWaitTicks) {
            if (lane_id() == 0) atomicOr(p.status, kAbort | kTimeout);
            S.abort = 1u;
            return false;
        }
        __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    return true;
}

// one lane per wave arrives at an LDS counter (no return value needed)
RK_DEV void arrive(uint32_t* ctr) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    if (lane_id() == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

// Poll N tagged fp16 pairs per lane (qword addresses from addr(k); nullptr = not needed) until every tag matches;
// val[k] receives the packed pair. Each iteration loads the words this lane still lacks (lanes holding a validated
// word, or needing none, are masked off and fetch nothing, so a second round re-reads only what is missing) and
// the status word, as one batch with a single wait; a word's first validated value is the one kept (its next value
// is written only after every consumer has finished this poll: the exchanges' dataflow order). Wave-uniform control
// flow; false after an abort or a timeout.
template <int N, class Addr>
RK_DEV bool poll_pairs(const Params& p, Lds& S, uint32_t tag, Addr addr, uint32_t (&val)[N]) {
    static_assert(N <= 32, "pending mask");
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < N; ++k)
        if (addr(k)) pending |= 1u << k;
    const uint64_t t0 = wall_clock64();
    uint64_t q[N];
#pragma unroll
    for (int k = 0; k < N; ++k) q[k] = 0;
    while (true) {
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (pending & (1u << k)) q[k] = ld_coh64(addr(k));
        const uint32_t st = ld_coh(p.status);
#pragma unroll
        for (int k = 0; k < N; ++k)
            if ((pending & (1u << k)) && pair_ok(q[k], tag)) {
                val[k] = pair_val(q[k]);
                pending &= ~(1u << k);
            }
        if (__all(pending == 0)) return true;
        if (!wait_more(p, S, t0, st)) return false;
    }
}

// ---------------------------------------------------------------------------------------------- block work
struct Work {
    int nt;      // w_in tiles
    int nq;      // of which q / k / v tiles (the first nq entries; 0 or 1)
    int sb, se;  // down slices [sb, se)
};

RK_DEV Work work_of(const Params& p, const Lds& S) {
    Work w;
    w.nt = 0;
#pragma unroll
    for (int t = 0; t < kMaxTiles; ++t) w.nt += S.work[t] >= 0;
    const int qkv_tiles = (p.NH + 2 * p.NKV) * kHD / 16;
    w.nq = (w.nt > 0 && S.work[0] < qkv_tiles) ? 1 : 0;
    w.sb = S.work[kSliceBegin];
    w.se = S.work[kSliceEnd];
    return w;
}

// ---------------------------------------------------------------------------------------------- x / h (row waves)
// Row wave rho (attention waves W0..W3 -> 0..3, down waves W12..W15 -> 4..7) owns columns [256 rho, 256 rho + 256)
// of every 2048-vector: lane L holds columns 256 rho + 4L .. + 3 as two fp16 pairs (qwords 128 rho + 2L, + 1 of a
// tagged copy). Each row wave polls its part of x, the eight combine their LayerNorm statistics through LDS, and
// each stages its own two column groups of h.
RK_DEV int row_index() {
    const int w = wave_id();
    return w < kAW ? w : w - (kD0 - kAW);
}

struct RowVals {
    uint32_t v[2];  // (x0, x1), (x2, x3) of the lane's 4 columns
};

RK_DEV void x_from_embedding(const Params& p, int64_t tok, int rho, RowVals& xv) {
    const float es = h16(p.emb_s[tok]);
    const uint32_t c = *reinterpret_cast<const uint32_t*>(p.emb_q + (size_t)tok * kH + kRCols * rho + 4 * lane_id());
    const float c0 = (float)(int8_t)(c & 0xFF), c1 = (float)(int8_t)((c >> 8) & 0xFF);
    const float c2 = (float)(int8_t)((c >> 16) & 0xFF), c3 = (float)(int8_t)(c >> 24);
    xv.v[0] = pack_h2(c0 * es, c1 * es);
    xv.v[1] = pack_h2(c2 * es, c3 * es);
}

RK_DEV bool x_poll(const Params& p, Lds& S, uint32_t tag, int rho, RowVals& xv) {
    // the opaque lane keeps the addresses from being hoisted out of the layer loop
    const uint64_t* tx = reinterpret_cast<const uint64_t*>(p.tx) + (blockIdx.x % kXRep) * kRepQwords +
                         kRCols / 2 * rho + 2 * lane_id();
    return poll_pairs<2>(p, S, tag, [&](int k) -> const uint64_t* { return tx + k; }, xv.v);
}

// the row wave's 4 LayerNorm weights per lane, loaded before the x poll so that their round trip overlaps it
RK_DEV uint2 ln_w_issue(const uint16_t* w, int rho) {
    return *reinterpret_cast<const uint2*>(w + kRCols * rho + 4 * lane_id());
}

// LayerNorm (the reference's, engine/rumik_int4.py:38-43: biased variance, no bias) over the eight row waves'
// parts: each wave's sum and sum of squared deviations from its own mean go through LDS, and every wave combines the
// eight in the same order (Chan's pairwise update, no cancellation) -> mean, rstd. x -> h = round((x - mean) rstd w)
// in place. Returns false after an abort.
RK_DEV bool layernorm_rows(const Params& p, Lds& S, int l, int rho, const uint2& w, RowVals& xv) {
    float x[4];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const h2_t v = as_h2(xv.v[e]);
        x[2 * e] = (float)v.x;
        x[2 * e + 1] = (float)v.y;
    }
    const float sum = wave_sum(x[0] + x[1] + x[2] + x[3]);
    const float m = sum * (1.0f / kRCols);
    float d2 = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) d2 += (x[e] - m) * (x[e] - m);
    const float m2 = wave_sum(d2);
    if (lane_id() == 0) S.lnst[rho] = make_float2(sum, m2);
    arrive(&S.cnt_ln);
    const bool ok = flag_wait(p, S, &S.cnt_ln, (uint32_t)kRW * (l + 1));
    float tot = 0.f;
#pragma unroll
    for (int r = 0; r < kRW; ++r) tot += S.lnst[r].x;
    const float mean = tot * (1.0f / kH);
    float M2 = 0.f;
#pragma unroll
    for (int r = 0; r < kRW; ++r) {
        const float2 st = S.lnst[r];
        const float dm = st.x * (1.0f / kRCols) - mean;
        M2 += st.y + (float)kRCols * dm * dm;
    }
    const float rstd = 1.0f / sqrtf(M2 * (1.0f / kH) + p.eps);
    const h2_t w01 = as_h2(w.x), w23 = as_h2(w.y);
    xv.v[0] = pack_h2((x[0] - mean) * rstd * (float)w01.x, (x[1] - mean) * rstd * (float)w01.y);
    xv.v[1] = pack_h2((x[2] - mean) * rstd * (float)w23.x, (x[3] - mean) * rstd * (float)w23.y);
    return ok;
}

// h -> MFMA A fragments of groups 2 rho and 2 rho + 1 (lanes 0..31 and 32..63) + their sums. 8-column block
// r = (lane % 32) / 2 of a group is split over lanes 2r (columns 0..3) and 2r + 1 (columns 4..7): with its
// partner's pairs (DPP) each lane forms two of the block's four dequant-order pairs (x0,x4),(x1,x5) | (x2,x6),(x3,x7).
RK_DEV void stage_h_frag(const RowVals& h, int rho, Lds& S) {
    const int lane = lane_id();
    const uint32_t q0 = __builtin_bit_cast(uint32_t, dpp<0xB1>(__builtin_bit_cast(float, h.v[0])));  // partner
    const uint32_t q1 = __builtin_bit_cast(uint32_t, dpp<0xB1>(__builtin_bit_cast(float, h.v[1])));
    const bool upper = lane & 1;
    uint2 out;
    if (!upper) {
        out.x = perm(q0, h.v[0], 0x05040100u);  // (x0, x4)
        out.y = perm(q0, h.v[0], 0x07060302u);  // (x1, x5)
    } else {
        out.x = perm(h.v[1], q1, 0x05040100u);  // (x2, x6)
        out.y = perm(h.v[1], q1, 0x07060302u);  // (x3, x7)
    }
    const int g = 2 * rho + (lane >> 5), r = (lane & 31) >> 1, sq = r >> 2, t = r & 3;
    reinterpret_cast<uint2*>(&S.hfrag[g * 16 + t * 4 + sq])[upper] = out;
    float sum = 0.f;
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const h2_t v = as_h2(h.v[e]);
        sum += (float)v.x + (float)v.y;
    }
    sum += dpp<0x128>(sum);  // row_ror 8
    sum += dpp<0x124>(sum);  // row_ror 4
    sum += dpp<0x122>(sum);  // row_ror 2
    sum += dpp<0x121>(sum);  // row_ror 1
    sum = sum_xor<16>(sum);  // rows 0 + 1 (group 2 rho), rows 2 + 3 (group 2 rho + 1)
    if ((lane & 31) == 0) S.hsum[g] = sum;
}

// h -> natural fp16 pairs (the int8 head's input): 8-column block 32 rho + lane / 2, half lane % 2
RK_DEV void stage_h_pairs(const RowVals& h, int rho, Lds& S) {
    const int lane = lane_id();
    reinterpret_cast<uint2*>(&S.vecp[32 * rho + (lane >> 1)])[lane & 1] = make_uint2(h.v[0], h.v[1]);
}

// the block's rows 8b .. 8b + 7 sit in row wave b / 32, lanes 2 (b % 32) and 2 (b % 32) + 1: kept in LDS
RK_DEV void keep_xrow(const RowVals& xv, int rho, Lds& S) {
    const int lane = lane_id(), b = blockIdx.x;
    if (rho == b / 32 && (lane >> 1) == (b & 31)) {
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const h2_t v = as_h2(xv.v[e]);
            S.xrow[4 * (lane & 1) + 2 * e] = (float)v.x;
            S.xrow[4 * (lane & 1) + 2 * e + 1] = (float)v.y;
        }
    }
}

// Row wave, start of layer l: x of the previous layer (or the embedding) -> LayerNorm -> its two groups of h staged;
// arrival at cnt_h (the tile waves wait for all eight)
RK_DEV void x_phase(const Params& p, int l, uint32_t step, int64_t pos, int64_t tok, int rho, Lds& S) {
    const uint2 w = ln_w_issue(p.ln_w + (size_t)l * kH, rho);
    RowVals xv;
    if (l == 0) {
        x_from_embedding(p, tok, rho, xv);
    } else {
        x_poll(p, S, tag_of(step, l - 1), rho, xv);
        if (l == 1 && rho == 0 && blockIdx.x == 0 && lane_id() == 0) p.pos[0] = pos + 1;  // every block read pos
    }
    RK_TRACE(rho == 0, kTrXPolled);
    RK_TRACE(rho == 4, kTrXPolled4);
    keep_xrow(xv, rho, S);
    layernorm_rows(p, S, l, rho, w, xv);
    RK_TRACE(rho == 0, kTrLnDone);
    stage_h_frag(xv, rho, S);
    arrive(&S.cnt_h);
    RK_TRACE(rho == 0, kTrHStaged);
}

// Row wave after the last layer: the final LayerNorm, h as natural pairs for the int8 head (read by the tile
// waves after all eight arrive at cnt_head) and, from block 0, the exported final hidden state
RK_DEV void x_final(const Params& p, uint32_t step, int64_t pos, int rho, Lds& S) {
    const uint2 w = ln_w_issue(p.norm_w, rho);
    RowVals xv;
    x_poll(p, S, tag_of(step, p.L - 1), rho, xv);
    if (p.L == 1 && rho == 0 && blockIdx.x == 0 && lane_id() == 0) p.pos[0] = pos + 1;
    layernorm_rows(p, S, p.L, rho, w, xv);
    stage_h_pairs(xv, rho, S);
    if (p.hn && blockIdx.x == 0)
        *reinterpret_cast<uint2*>(p.hn + kRCols * rho + 4 * lane_id()) = make_uint2(xv.v[0], xv.v[1]);
    arrive(&S.cnt_head);
}

// ---------------------------------------------------------------------------------------------- w_in tiles
struct TileRegs {
    u4_t w[kGPW][kMaxTiles];
    uint32_t sm[kGPW][kMaxTiles];  // scale | min << 16 of (group, tile) for row lane % 16
};

RK_DEV size_t n_tiles(const Params& p) { return ((size_t)(p.NH + 2 * p.NKV) * kHD + 2 * p.inter) / 16; }

// tile wave m (0..7) computes column groups 2m, 2m + 1 of every tile. win_sm holds per (layer, tile, slot, row)
// the two scale | min words of a group pair; slot s serves groups 2((s + 7) % 8), so pair m is slot (m + 1) % 8.
RK_DEV int mlp_wave() { return wave_id() - kM0; }

// Prefetches are branch-free with a fixed instruction count (addresses clamped to valid data that is then ignored):
// the compiler can then wait for exactly the loads a computation needs. With data-dependent branches around loads
// it cannot count the loads issued after a prefetch and waits for all of them.
// win_t: per (layer, tile, group) 1 KiB of codes in lane order.
// Paced: at most two loads in flight per wave. The tile waves have nothing else to do meanwhile (the prefetch
// still lands well before the next layer needs it), while a chip-wide burst of every block's tiles would queue ahead
// of the critical path's polls for microseconds: a poll's loads wait behind what the CU already has in flight.
RK_DEV void tile_issue(const Params& p, int l, const Lds& S, const Work& wk, TileRegs& tr) {
    const int lane = lane_id(), m = mlp_wave();
    const size_t base = (size_t)l * n_tiles(p);
    const int t_fallback = wk.nt > 0 ? S.work[0] : 0;
    const int slot = (m + 1) % 8;
#pragma unroll
    for (int t = 0; t < kMaxTiles; ++t) {
        const size_t T = base + (t < wk.nt ? S.work[t] : t_fallback);
#pragma unroll
        for (int k = 0; k < kGPW; ++k)
            tr.w[k][t] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p.win_t) + (T * kNG + 2 * m + k) * 64 + lane);
        const u2_t sm = *(reinterpret_cast<const u2_t*>(p.win_sm) + (T * 8 + slot) * 16 + (lane & 15));
        tr.sm[0][t] = sm.x;
        tr.sm[1][t] = sm.y;
        asm volatile("s_waitcnt vmcnt(2)" ::: "memory");  // all but the last two loads have landed
    }
}

// the wave's groups of tiles [TB, TE) -> S.tpart[m][t][row], at most kTileChunk tiles at a time. Per group the four
// 32-column chunks are the outer loop and the chunk's tiles the inner one, so up to kTileChunk independent MFMA
// accumulations are in flight while only their accumulators are live.
constexpr int kTileChunk = 2;

template <int TB, int TE>
RK_DEV void tile_chunk(const TileRegs& tr, const Work& wk, Lds& S) {
    const int lane = lane_id(), m = mlp_wave(), s = lane >> 4;
    const Int4Masks km = int4_masks();
    float acc[kMaxTiles];
#pragma unroll
    for (int t = TB; t < TE; ++t) acc[t] = 0.f;
#pragma unroll
    for (int k = 0; k < kGPW; ++k) {
        const int g = 2 * m + k;
        f4_t d[kMaxTiles];
#pragma unroll
        for (int t = TB; t < TE; ++t) d[t] = f4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            const h8_t A = __builtin_bit_cast(h8_t, S.hfrag[g * 16 + t4 * 4 + s]);
#pragma unroll
            for (int t = TB; t < TE; ++t)  // tiles beyond the block's count hold copies of tile 0 (ignored)
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
    if (lane < 16)
#pragma unroll
        for (int t = TB; t < TE; ++t)
            if (t < wk.nt) S.tpart[m][t][lane] = acc[t];
}

template <int TB, int TE>
RK_DEV void tile_compute(const TileRegs& tr, const Work& wk, Lds& S) {
    if constexpr (TE - TB <= kTileChunk) {
        tile_chunk<TB, TE>(tr, wk, S);
    } else {
        tile_chunk<TB, TB + kTileChunk>(tr, wk, S);
        tile_compute<TB + kTileChunk, TE>(tr, wk, S);
    }
}

// Tile 0 (the block's q / k / v tile when it has one) is computed by the eight row waves as soon as each has staged
// its h: row wave rho takes column groups 2 rho, 2 rho + 1, the columns of x it holds, so it reads only h it wrote
// itself. Its codes come through LDS: tile wave m copies its two groups of tile 0 there once its loads have landed.
static_assert(kRW == kMW, "row wave rho computes tile wave rho's column groups of tile 0");

RK_DEV void stage_tile0(const TileRegs& tr, Lds& S) {  // tile wave m
    const int lane = lane_id(), m = mlp_wave();
#pragma unroll
    for (int k = 0; k < kGPW; ++k) {
        const u4_t w = tr.w[k][0];
        S.t0w[m][k][lane] = make_uint4(w[0], w[1], w[2], w[3]);
        if (lane < 16) S.t0sm[m][k][lane] = tr.sm[k][0];
    }
}

RK_DEV void tile0_part(const Work& wk, int rho, Lds& S) {  // row wave rho; the same sums as tile_chunk
    const int lane = lane_id(), s = lane >> 4;
    const Int4Masks km = int4_masks();
    float acc = 0.f;
#pragma unroll
    for (int k = 0; k < kGPW; ++k) {
        const int g = 2 * rho + k;
        const uint4 wq = S.t0w[rho][k][lane];
        const u4_t w = {wq.x, wq.y, wq.z, wq.w};
        f4_t d = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            const h8_t A = __builtin_bit_cast(h8_t, S.hfrag[g * 16 + t4 * 4 + s]);
            d = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, dequant_frag(w[t4], km), d, 0, 0, 0);
        }
        const uint32_t sm = S.t0sm[rho][k][lane & 15];
        acc = __builtin_fmaf(d[0], h16((uint16_t)sm), __builtin_fmaf(h16((uint16_t)(sm >> 16)), S.hsum[g], acc));
    }
    if (lane < 16 && wk.nt > 0) S.tpart[rho][0][lane] = acc;
}

// the projection output of tile t, row j (the K-split partials summed, rounded to fp16 as the reference's buf_in)
RK_DEV float tile_out(const Lds& S, int t, int j) {
    float y = 0.f;
#pragma unroll
    for (int m = 0; m < kMW; ++m) y += S.tpart[m][t][j];
    return rnd16(y);
}

// pass 1 epilogue (one wave, lanes j < 16): the block's q / k / v tile 0 -> RoPE on q / k rows, published tagged;
// k and v also into the cache at pos
RK_DEV void qkv_epilogue(const Params& p, int l, int64_t pos, uint32_t tag, const Lds& S) {
    const int lane = lane_id();
    const int j = lane & 15;
    const float y = tile_out(S, 0, j);
    const float partner = dpp<0xB1>(y);  // row j ^ 1 (quad_perm [1,0,3,2])
    if (lane >= 16) return;
    const int NH = p.NH, NKV = p.NKV;
    const int row = S.work[0] * 16 + j;
    const int qk_rows = (NH + NKV) * kHD;
    if (row < qk_rows) {
        float out = y;
        if ((p.sliding >> l) & 1ull) {  // interleaved RoPE: pairs (2i, 2i + 1)
            const int dd = row % kHD;
            const float c = S.rcos[dd >> 1], sn = S.rsin[dd >> 1];
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
    } else {
        const int r2 = row - qk_rows;
        st_coh(p.tkv + NKV * kHD + r2, tword(y, tag));
        p.vc[(((size_t)l * NKV + r2 / kHD) * p.S + pos) * kHD + r2 % kHD] = f16b(y);
    }
}

// pass 2 epilogue (one wave): lane (tile t = nq + lane / 8, channel j = lane % 8): gate row j and up row j + 8 of
// the tile -> act of MLP channel 8 (T - qkv tiles) + j (the block owns every channel of its tiles)
RK_DEV void act_epilogue(const Params& p, const Work& wk, Lds& S) {
    const int lane = lane_id();
    const int t = wk.nq + (lane >> 3), j = lane & 7;
    if (t >= wk.nt) return;
    const float g = tile_out(S, t, j), u = tile_out(S, t, j + 8);
    const int qkv_tiles = (p.NH + 2 * p.NKV) * kHD / 16;
    const int ch = (S.work[t] - qkv_tiles) * 8 + j;
    S.act[ch - wk.sb * 16] = rnd16(g / (1.0f + __expf(-g)) * u);
}

// ---------------------------------------------------------------------------------------------- w_down slices
// down lane sl takes the row pairs rp = sl + 256k (rows 2rp, 2rp + 1): per slice one 16-byte load of codes
// (wd_t: per (layer, slice), 2048 rows x 8 bytes), per 128-column group one 8-byte load of scale | min << 16
struct DownRegs {
    u4_t c[kRP][kMaxSlices];
    u2_t sm[kRP][2];  // the block's slices span at most two groups
};

RK_DEV int down_lane() { return (int)opaque_vgpr(threadIdx.x - 64 * kD0); }
RK_DEV int attn_lane() { return (int)opaque_vgpr(threadIdx.x); }  // W0..W3: 0..255

RK_DEV void down_issue(const Params& p, int l, const Work& wk, DownRegs& dr) {
    const int sl = down_lane();
    const int nsl = p.inter / 16, ngd = p.inter / 128;
    const int gb = wk.sb / 8;
#pragma unroll
    for (int k = 0; k < kRP; ++k) {
        const int rp = sl + kDLanes * k;
#pragma unroll
        for (int i = 0; i < kMaxSlices; ++i)
            dr.c[k][i] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p.wd_t) +
                                                    ((size_t)l * nsl + min(wk.sb + i, nsl - 1)) * (kH / 2) + rp);
#pragma unroll
        for (int q = 0; q < 2; ++q)
            dr.sm[k][q] = *reinterpret_cast<const u2_t*>(p.wd_sm + ((size_t)l * ngd + min(gb + q, ngd - 1)) * kH + 2 * rp);
        asm volatile("s_waitcnt vmcnt(5)" ::: "memory");  // paced like the tiles: one row-pair group in flight
    }
}

// partial down output of this block's channels for all 2048 rows, published tagged. tdp is laid out
// [consumer block][producer block][8 rows]: a consumer's rows from all producers form one contiguous 8 KB run, so
// its polls touch 64 cache lines instead of one line per producer.
RK_DEV void down_compute(const Params& p, uint32_t tag, const Work& wk, const DownRegs& dr, const Lds& S) {
    const int sl = down_lane();
    const Int4Masks km = int4_masks();
    const int gb = wk.sb / 8;
    float d[kRP][2];
#pragma unroll
    for (int k = 0; k < kRP; ++k) d[k][0] = d[k][1] = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxSlices; ++i) {
        if (wk.sb + i >= wk.se) continue;
        // the slice's 16 act values as the dequant's pairs: dword e holds codes 8e..8e+7 -> (a0, a4), (a1, a5), ...
        const float* a = S.act + 16 * i;
        uint32_t xp[8];
        float asum = 0.f;
#pragma unroll
        for (int e = 0; e < 2; ++e)
#pragma unroll
            for (int k = 0; k < 4; ++k) xp[4 * e + k] = pack_h2(a[8 * e + k], a[8 * e + k + 4]);
#pragma unroll
        for (int c = 0; c < 16; ++c) asum += a[c];
        const int q = (wk.sb + i) / 8 - gb;
#pragma unroll
        for (int k = 0; k < kRP; ++k) {
#pragma unroll
            for (int h = 0; h < 2; ++h) {  // row 2rp + h: dwords 2h, 2h + 1
                float dot = 0.f;
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    h2_t pr[4];
                    dequant_pairs(dr.c[k][i][2 * h + e], km, pr);
#pragma unroll
                    for (int kk = 0; kk < 4; ++kk) dot = dot2(pr[kk], as_h2(xp[4 * e + kk]), dot);
                }
                const uint32_t sm = q == 0 ? dr.sm[k][0][h] : dr.sm[k][1][h];
                d[k][h] = __builtin_fmaf(dot, h16((uint16_t)sm), __builtin_fmaf(h16((uint16_t)(sm >> 16)), asum, d[k][h]));
            }
        }
    }
    uint64_t* out = reinterpret_cast<uint64_t*>(p.tdp) + (size_t)blockIdx.x * 4;  // + (consumer * nb) * 4 + pair
#pragma unroll
    for (int k = 0; k < kRP; ++k) {
        const int rp = sl + kDLanes * k;
        st_coh64(out + (size_t)(rp >> 2) * gridDim.x * 4 + (rp & 3), tpair(d[k][0], d[k][1], tag));
    }
}

// ---------------------------------------------------------------------------------------------- attention
// slots per attention split: n / nsp rounded up to 8, at least kMinChunk (short contexts use fewer, fuller splits,
// so the combine waits on fewer blocks; a full split, 32 slots, measured best at ctx 256 / 1024 / 2048)
constexpr int kMinChunk = kAW * kSlotsPerWave;
RK_DEV int split_chunk(int n, int nsp) { return max(kMinChunk, ((n + nsp - 1) / nsp + 7) & ~7); }

struct Split {
    bool att;  // this block runs a split
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

// Attention wave a takes the split's slots start + a + 4u, u < kSlotsPerWave. Scores use the chunk layout: lane
// (u = lane / 8, c = lane % 8) holds dims [16c, 16c + 16) of slot u's key (32 bytes); the PV product uses the
// dim-pair layout: every lane holds dims 2 lane, 2 lane + 1 of each slot's value.
struct KVRegs {
    u4_t k[2];                   // the lane's 16 key dims of its slot
    uint32_t v[kSlotsPerWave];   // the lane's value pair of every slot
};

RK_DEV int slot_of(const Split& s, int a, int u) { return s.start + a + kAW * u; }

// every lane loads its slots (clamped into the cache), used or not; slot pos is taken from the tagged copy instead
// (the cache write of this step may not be visible yet)
RK_DEV void kv_issue(const Params& p, int l, int64_t pos, KVRegs& kv) {
    const int lane = lane_id(), a = wave_id();
    const Split s = split_of(p, pos);
    const size_t base = (((size_t)l * p.NKV + s.g) * p.S) * kHD;
    const u4_t* kr = reinterpret_cast<const u4_t*>(p.kc + base);
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(p.vc + base);
    const int tk = min(slot_of(s, a, lane >> 3), p.S - 1), c = lane & 7;
    kv.k[0] = kr[(size_t)tk * (kHD / 8) + 2 * c];
    kv.k[1] = kr[(size_t)tk * (kHD / 8) + 2 * c + 1];
#pragma unroll
    for (int u = 0; u < kSlotsPerWave; ++u) kv.v[u] = vr[(size_t)min(slot_of(s, a, u), p.S - 1) * (kHD / 2) + lane];
}

// q of the block's KV head (REP heads) and, when the split holds pos, k / v at pos, into registers
struct QRegs {
    uint32_t q[kMaxRep];
    uint32_t knew, vnew;
};

template <int REP>
RK_DEV bool q_poll(const Params& p, Lds& S, int64_t pos, uint32_t tag, QRegs& qr) {
    const int lane = lane_id();
    const Split s = split_of(p, pos);
    const bool has_pos = s.start <= pos && pos < s.end;
    const uint32_t z = opaque_vgpr(0u);  // not hoistable: see x_poll
    const uint64_t* tq = reinterpret_cast<const uint64_t*>(p.tq) + z;
    const uint64_t* tkv = reinterpret_cast<const uint64_t*>(p.tkv) + z;
    uint32_t v[REP + 2];  // one poll batch: the REP heads' q, then k and v at pos
    const bool ok = poll_pairs<REP + 2>(
        p, S, tag,
        [&](int k) -> const uint64_t* {
            if (k < REP) return tq + (size_t)(s.g * REP + k) * (kHD / 2) + lane;
            if (!has_pos) return nullptr;
            return tkv + (size_t)((k - REP) * p.NKV + s.g) * (kHD / 2) + lane;
        },
        v);
#pragma unroll
    for (int k = 0; k < REP; ++k) qr.q[k] = v[k];
    qr.knew = v[REP];
    qr.vnew = v[REP + 1];
    return ok;
}

// Wave a's share of the split for the REP heads, all its slots at once. Scores in the chunk layout: each lane dots
// its 16 key dims with the same 16 dims of up to four query heads (v_dot2, fp32 sums) and the eight chunk lanes of
// a slot reduce with three DPP steps, so every lane of slot group u holds that slot's scores. Per head the max and
// the sum of exp over the slots reduce over lane bits 3..5; the PV product takes each p through readlane. Result:
// (m, l, acc) per head in LDS (m = -inf, l = 0 for a wave without a valid slot). q (and k at pos) reach the chunk
// layout through the wave's own LDS rows (no other wave reads them).
template <int REP>
RK_DEV void attention(const Params& p, int64_t pos, const KVRegs& kv, const QRegs& qr, Lds& S) {
    const int lane = lane_id(), a = wave_id();
    const Split s = split_of(p, pos);
    const int u = lane >> 3, c = lane & 7;
    const bool valid = slot_of(s, a, u) < s.end;
    const bool is_pos = slot_of(s, a, u) == pos;
#pragma unroll
    for (int r = 0; r < REP; ++r) S.qst[a][r][lane] = qr.q[r];
    S.qst[a][kMaxRep][lane] = qr.knew;
    u4_t kk[2] = {kv.k[0], kv.k[1]};
    if (is_pos) {  // slot pos: the tagged k (dims 16c .. 16c + 15 = pairs 8c .. 8c + 7)
        kk[0] = *reinterpret_cast<const u4_t*>(&S.qst[a][kMaxRep][8 * c]);
        kk[1] = *reinterpret_cast<const u4_t*>(&S.qst[a][kMaxRep][8 * c + 4]);
    }
    float mx[REP], pe[REP], ls[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        const u4_t q0 = *reinterpret_cast<const u4_t*>(&S.qst[a][r][8 * c]);
        const u4_t q1 = *reinterpret_cast<const u4_t*>(&S.qst[a][r][8 * c + 4]);
        float d = 0.f;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            d = dot2(as_h2(q0[e]), as_h2(kk[0][e]), d);
            d = dot2(as_h2(q1[e]), as_h2(kk[1][e]), d);
        }
        d += dpp<0xB1>(d);   // xor 1
        d += dpp<0x4E>(d);   // xor 2
        d += dpp<0x141>(d);  // row_half_mirror: the other half of the 8 chunk lanes
        const float sc = valid ? d * p.scale : -INFINITY;
        float m = fmaxf(sc, dpp<0x128>(sc));  // row_ror 8 = lane ^ 8 inside a 16-lane row
        m = max_xor<16>(m);
        m = max_xor<32>(m);
        const float e = m == -INFINITY ? 0.f : __expf(sc - m);
        float l = e + dpp<0x128>(e);
        l = sum_xor<16>(l);
        l = sum_xor<32>(l);
        mx[r] = m;
        pe[r] = e;
        ls[r] = l;
    }
    // PV: acc[r] += p(u, r) * v(u) over the wave's slots; p of slot u in lane 8u
    float2 acc[REP];
#pragma unroll
    for (int r = 0; r < REP; ++r) acc[r] = make_float2(0.f, 0.f);
#pragma unroll
    for (int uu = 0; uu < kSlotsPerWave; ++uu) {
        // slots past the split's end are selected away, not multiplied by p = 0: whatever a cache slot beyond pos
        // holds (a NaN left by an overflowed step included) must not reach the result, as with the reference's
        // masked loads (other = 0)
        const int su = slot_of(s, a, uu);
        const h2_t vp = as_h2(su == pos ? qr.vnew : (su < s.end ? kv.v[uu] : 0u));
        const float v0 = (float)vp.x, v1 = (float)vp.y;
#pragma unroll
        for (int r = 0; r < REP; ++r) {
            const float pr =
                __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, pe[r]), 8 * uu));
            acc[r].x = __builtin_fmaf(pr, v0, acc[r].x);
            acc[r].y = __builtin_fmaf(pr, v1, acc[r].y);
        }
    }
#pragma unroll
    for (int r = 0; r < REP; ++r) {
        S.s_acc[a][r][lane] = acc[r];
        if (lane == 0) {
            S.s_m[a][r] = mx[r];
            S.s_l[a][r] = ls[r];
        }
    }
}

// after all four attention waves have left their partials: head r's merge over the four, published as the
// normalized split partial (o / l, m, l); wave a publishes the heads r = a, a + 4
template <int REP>
RK_DEV void attention_merge(const Params& p, int64_t pos, uint32_t tag, const Lds& S, int r) {
    const int lane = lane_id();
    const Split s = split_of(p, pos);
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAW; ++w) M = fmaxf(M, S.s_m[w][r]);
    float Lt = 0.f, ax = 0.f, ay = 0.f;
#pragma unroll
    for (int w = 0; w < kAW; ++w) {
        const float wt = S.s_m[w][r] == -INFINITY ? 0.f : __expf(S.s_m[w][r] - M);
        Lt += wt * S.s_l[w][r];
        ax += wt * S.s_acc[w][r][lane].x;
        ay += wt * S.s_acc[w][r][lane].y;
    }
    const size_t pi = (size_t)(s.g * REP + r) * p.nsp + s.sp;
    const float inv = Lt > 0.f ? 1.0f / Lt : 0.f;
    st_coh64(reinterpret_cast<uint64_t*>(p.tpo + pi * kHD) + lane, tpair(ax * inv, ay * inv, tag));
    if (lane == 0) {
        st_coh64(reinterpret_cast<uint64_t*>(p.tml) + 2 * pi,
                 (uint64_t)__builtin_bit_cast(uint32_t, M) | ((uint64_t)tag << 32));
        st_coh64(reinterpret_cast<uint64_t*>(p.tml) + 2 * pi + 1,
                 (uint64_t)__builtin_bit_cast(uint32_t, Lt) | ((uint64_t)tag << 32));
    }
}

// Head h's combine: out = sum_i w_i o_i / sum_i w_i, w_i = exp(m_i - max m) * l_i over the splits holding at least
// one slot (at most 64). Each of the head's 16 blocks combines it (its o slice needs the result): attention wave a
// polls splits [16a, 16a + 16) in one batch per iteration and leaves (M = its max m, L = sum of its w_i taken
// against M, sum of w_i o_i) in LDS; once all four have, each merges the parts itself (comb_merge). The sums run
// in split order within a wave and in wave order across waves, so the result does not depend on arrival order.
RK_DEV int comb_splits(const Params& p, int64_t pos) {
    const int n = (int)min<int64_t>(pos + 1, (int64_t)p.S);
    const int ch = split_chunk(n, p.nsp);
    return min(p.nsp, (n + ch - 1) / ch);
}

RK_DEV int o_head() { return blockIdx.x >> 4; }
RK_DEV int o_rgroup() { return blockIdx.x & 15; }

RK_DEV bool comb_part(const Params& p, Lds& S, int h, int64_t pos, uint32_t tag) {
    const int lane = lane_id(), a = wave_id();
    const int nsp = p.nsp, i0 = kCombPer * a;
    const int cnt = min(max(comb_splits(p, pos) - i0, 0), kCombPer);
    float M = -INFINITY, L = 0.f, ax = 0.f, ay = 0.f;
    bool ok = true;
    if (cnt > 0) {
        const size_t hb = (size_t)h * nsp;
        const uint32_t z = opaque_vgpr(0u);  // not hoistable: see x_poll
        const uint64_t* po = reinterpret_cast<const uint64_t*>(p.tpo + hb * kHD) + lane + z;
        // lane j brings split i0 + j % kCombPer's (m, l): every 16-lane row holds all of them
        const int jl = lane % kCombPer;
        const uint64_t* tml = reinterpret_cast<const uint64_t*>(p.tml) + 2 * (hb + min(i0 + jl, nsp - 1)) + z;
        const uint64_t t0 = wall_clock64();
        uint32_t pending = (1u << cnt) - 1;
        bool ml_done = jl >= cnt;
        float mi = -INFINITY, li = 0.f;
        uint32_t val[kCombPer];  // split i0 + k's pair of dims (2 lane, 2 lane + 1); zero for k >= cnt
#pragma unroll
        for (int k = 0; k < kCombPer; ++k) val[k] = 0u;
        uint64_t q[kCombPer], qm = 0, ql = 0;
#pragma unroll
        for (int k = 0; k < kCombPer; ++k) q[k] = 0;
        while (true) {
            // one batch per iteration (see poll_pairs): the pairs of the splits still missing (a wave-uniform set),
            // the (m, l) words a lane still lacks, and the status
#pragma unroll
            for (int k = 0; k < kCombPer; ++k)
                if (pending & (1u << k)) q[k] = ld_coh64(po + (size_t)(i0 + k) * (kHD / 2));
            if (!ml_done) {
                qm = ld_coh64(tml);
                ql = ld_coh64(tml + 1);
            }
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
            if (!wait_more(p, S, t0, st)) {
                ok = false;
                break;
            }
        }
        if (ok) {
            // the max m over the splits (a 16-lane row reduction), then each split's weight w = exp(m - M) l in its
            // lane, broadcast by readlane; the sums run in split order
            float mv = jl < cnt ? mi : -INFINITY;
            mv = fmaxf(mv, dpp<0x128>(mv));  // row_ror 8
            mv = fmaxf(mv, dpp<0x124>(mv));  // row_ror 4
            mv = fmaxf(mv, dpp<0x122>(mv));  // row_ror 2
            M = fmaxf(mv, dpp<0x121>(mv));   // row_ror 1
            const float wl = (jl < cnt && mi != -INFINITY) ? __expf(mi - M) * li : 0.f;
#pragma unroll
            for (int k = 0; k < kCombPer; ++k) {
                const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k));
                const h2_t o = as_h2(val[k]);
                ax = __builtin_fmaf(wk, (float)o.x, ax);
                ay = __builtin_fmaf(wk, (float)o.y, ay);
                L += wk;
            }
        }
    }
    S.cpa[a][lane] = make_float2(ax, ay);
    if (lane == 0) {
        S.cpm[a] = M;
        S.cpl[a] = L;
    }
    return ok;
}

// every attention wave, after all four left their combine parts: the parts merged into head h's attention output,
// rounded to fp16 (the reference keeps it in the activation dtype), into the wave's own LDS row as natural pairs
// (the o slice reads it back in its own order); returns the sum of the 128 values (the o projection's min term)
RK_DEV float comb_merge(Lds& S) {
    const int lane = lane_id(), a = wave_id();
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < kAW; ++w) M = fmaxf(M, S.cpm[w]);
    float den = 0.f, ox = 0.f, oy = 0.f;
#pragma unroll
    for (int w = 0; w < kAW; ++w) {
        const float f = S.cpm[w] == -INFINITY ? 0.f : __expf(S.cpm[w] - M);
        const float2 c = S.cpa[w][lane];
        den = __builtin_fmaf(f, S.cpl[w], den);
        ox = __builtin_fmaf(f, c.x, ox);
        oy = __builtin_fmaf(f, c.y, oy);
    }
    const float inv = den > 0.f ? 1.0f / den : 0.f;
    const float a0 = rnd16(ox * inv), a1 = rnd16(oy * inv);
    S.attn[a][lane] = pack_h2(a0, a1);
    return wave_sum(a0 + a1);
}

// ---------------------------------------------------------------------------------------------- w_o partials
// Block b = (head h = b / 16, row group r = b % 16) computes the o projection of head h's attention output for
// rows [128r, 128r + 128): 512 items (row i / 4, 32-column chunk i % 4 of the head's 128 columns), one 16-byte load
// each; attention lane ls (0..255) takes items ls and ls + 256. The head's 128 columns are one quantization group,
// so each row has one scale | min word (wo_sm[layer][row][head]).
struct ORegs {
    u4_t w[2];
    uint32_t sm[2];
};

static_assert(kH / kHD == 16 && kH / 128 == 16, "16 heads x 16 row groups of 128 = the 256 blocks");

RK_DEV void o_issue(const Params& p, int l, ORegs& o) {
    const int ls = attn_lane();
    const int h = o_head(), r = o_rgroup();
    const u4_t* base = reinterpret_cast<const u4_t*>(p.wo_q) + ((size_t)(l * p.NH + h) * 16 + r) * kOItems;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = ls + kALanes * k;
        o.w[k] = __builtin_nontemporal_load(base + i);
        o.sm[k] = p.wo_sm[((size_t)l * kH + 128 * r + (i >> 2)) * p.NH + h];
    }
}

// the items' dots, summed per row over the 4 lanes of its chunks; lanes i % 8 == 0 publish rows (i/4, i/4 + 1) as
// one tagged pair to top[consumer block][head][8 rows]
RK_DEV void o_part(const Params& p, uint32_t tag, const ORegs& o, const Lds& S, float asum) {
    const int ls = attn_lane(), lane = lane_id();
    const uint32_t* attn = S.attn[wave_id()];
    const int h = o_head(), r = o_rgroup();
    const Int4Masks km = int4_masks();
    uint64_t* top = reinterpret_cast<uint64_t*>(p.top);
    float vals[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = ls + k * kALanes, c = i & 3;
        uint32_t xp[16];
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // natural pairs of 8 columns -> the dequant's pair order
            const u4_t d = {attn[16 * c + 4 * q], attn[16 * c + 4 * q + 1], attn[16 * c + 4 * q + 2],
                            attn[16 * c + 4 * q + 3]};
            uint32_t hp[4];
            pair_permute(d, hp);
#pragma unroll
            for (int e = 0; e < 4; ++e) xp[4 * q + e] = hp[e];
        }
        float v = chunk_dot_int4(o.w[k], xp, km);
        v += dpp<0xB1>(v);  // the row's 4 chunks sit in lanes 4j .. 4j + 3
        v += dpp<0x4E>(v);
        vals[k] = __builtin_fmaf(v, h16((uint16_t)o.sm[k]), h16((uint16_t)(o.sm[k] >> 16)) * asum);
    }
    // both items before either store: after a store, gfx9 waits for its acknowledgement before any later use of a
    // load (one counter for both), which the second item's weights would otherwise pay (the empty asm keeps the
    // compiler from sinking the second item's math below the first store)
    asm volatile("" ::"v"(vals[0]), "v"(vals[1]));
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = ls + k * kALanes;
        const float nxt = dpp<0x104>(vals[k]);  // row_shl 4: the next row's total (lane + 4, same 16-lane row)
        if ((lane & 7) == 0) {
            const int row = 128 * r + (i >> 2);  // even
            st_coh64(top + ((size_t)(row >> 3) * p.NH + h) * 4 + ((row & 7) >> 1), tpair(vals[k], nxt, tag));
        }
    }
}

// Row wave rho: its 128 qwords of this block's run of down partials (qword q = 128 rho + 64k + lane: producer q / 4,
// row pair q % 4 = lane % 4) and, row wave 0, the o partials of the 16 heads (lane = head * 4 + pair), one poll
// batch; summed per row pair over the wave (lanes sharing lane % 4) into LDS. The last of the eight to arrive adds
// the eight parts in order, forms x rows = x + o + d (each rounded once, as add_ln) and publishes them in kXRep
// copies. tdp / top runs: a consumer's rows from all producers form one contiguous run (few cache lines per poll).
RK_DEV float class4_sum(float v) {  // sum over the 16 lanes that share lane % 4
    v += dpp<0x128>(v);  // row_ror 8
    v += dpp<0x124>(v);  // row_ror 4
    v = sum_xor<16>(v);
    v = sum_xor<32>(v);
    return v;
}

RK_DEV void gather_phase(const Params& p, int l, uint32_t tag, int rho, Lds& S) {
    const int lane = lane_id(), nb = gridDim.x;
    const uint64_t* run = reinterpret_cast<const uint64_t*>(p.tdp) + (size_t)blockIdx.x * nb * 4 + 128 * rho + lane;
    const uint64_t* orun = reinterpret_cast<const uint64_t*>(p.top) + (size_t)blockIdx.x * p.NH * 4 + lane;
    const bool with_o = rho == 0 && lane < 4 * p.NH;
    uint32_t v[3];
    poll_pairs<3>(p, S, tag,
                  [&](int k) -> const uint64_t* {
                      if (k == 2) return with_o ? orun : nullptr;
                      return 128 * rho + 64 * k + lane < 4 * nb ? run + 64 * k : nullptr;
                  },
                  v);
    RK_TRACE(rho == 0, kTrGatherPolled);
    RK_TRACE(rho == 4, kTrGatherPolled4);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        if (128 * rho + 64 * k + lane < 4 * nb) {
            const h2_t h = as_h2(v[k]);
            d0 += (float)h.x;
            d1 += (float)h.y;
        }
    }
    d0 = class4_sum(d0);
    d1 = class4_sum(d1);
    if (lane < 4) S.gpart[rho][lane] = make_float2(d0, d1);
    if (rho == 0) {
        float o0 = 0.f, o1 = 0.f;
        if (with_o) {
            const h2_t h = as_h2(v[2]);
            o0 = (float)h.x;
            o1 = (float)h.y;
        }
        o0 = class4_sum(o0);
        o1 = class4_sum(o1);
        if (lane < 4) S.opart[lane] = make_float2(o0, o1);
    }
    if (!arrive_last(&S.cnt_g, (uint32_t)kRW * (l + 1))) return;
    bool bad = false;
    if (lane < 4) {  // lane = row pair: rows 2 lane, 2 lane + 1
        float2 d = make_float2(0.f, 0.f);
#pragma unroll
        for (int r = 0; r < kRW; ++r) {
            d.x += S.gpart[r][lane].x;
            d.y += S.gpart[r][lane].y;
        }
        const float2 o = S.opart[lane];
        const float x0 = rnd16(S.xrow[2 * lane] + rnd16(o.x) + rnd16(d.x));
        const float x1 = rnd16(S.xrow[2 * lane + 1] + rnd16(o.y) + rnd16(d.y));
        S.xrow[2 * lane] = x0;
        S.xrow[2 * lane + 1] = x1;
        bad = !(__builtin_isfinite(x0) && __builtin_isfinite(x1));  // beyond 65504 the fp16 sum is inf
    }
    if (__ballot(bad) != 0ull && lane == 0) atomicOr(p.status, kNonFinite);
    static_assert(4 * kXRep <= 64, "one store per lane");
    if (lane < 4 * kXRep) {  // lane = copy * 4 + pair
        const int j = lane & 3;
        st_coh64(reinterpret_cast<uint64_t*>(p.tx) + (lane >> 2) * kRepQwords + 4 * blockIdx.x + j,
                 tpair(S.xrow[2 * j], S.xrow[2 * j + 1], tag));
    }
    RK_TRACE(true, kTrXPublished);
}

// ---------------------------------------------------------------------------------------------- head
// tile wave m's head rows r0 + m + 8k; the first kHeadRows are loaded ahead (after the last layer's tile pass) into
// the tile registers, free by then: row k half j in flat entry 2k + j of TileRegs::w
static_assert(2 * kHeadRows <= kGPW * kMaxTiles, "head rows fit the tile registers");

RK_DEV u4_t& head_slot(TileRegs& tr, int e) { return tr.w[e / kMaxTiles][e % kMaxTiles]; }
RK_DEV const u4_t& head_slot(const TileRegs& tr, int e) { return tr.w[e / kMaxTiles][e % kMaxTiles]; }

RK_DEV void head_rows(const Params& p, int& r0, int& r1) {
    const int per = (p.n_audio + gridDim.x - 1) / gridDim.x;
    r0 = min(p.n_audio, (int)blockIdx.x * per);
    r1 = min(p.n_audio, r0 + per);
}

RK_DEV void head_issue(const Params& p, TileRegs& tr) {
    const int lane = lane_id(), m = mlp_wave();
    int r0, r1;
    head_rows(p, r0, r1);
#pragma unroll
    for (int k = 0; k < kHeadRows; ++k) {
        const int r = min(r0 + m + kMW * k, p.n_audio - 1);
        const u4_t* qr = reinterpret_cast<const u4_t*>(p.head_q + (size_t)r * kH);
#pragma unroll
        for (int j = 0; j < 2; ++j) head_slot(tr, 2 * k + j) = __builtin_nontemporal_load(qr + lane + 64 * j);
    }
}

RK_DEV void head_compute(const Params& p, const TileRegs& tr, const Lds& S) {
    const int lane = lane_id(), m = mlp_wave();
    int r0, r1;
    head_rows(p, r0, r1);
    float res = 0.f;  // lane k: the logit of the wave's row k (at most 64 rows per wave: checked on the host)
    for (int k = 0; r0 + m + kMW * k < r1; ++k) {
        const int r = r0 + m + kMW * k;
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
        if (lane == k) res = acc * h16(p.head_s[r]);
    }
    // one store per row, all after the loop: a store inside it would make each next row's use of its (long since
    // landed) codes wait for that store's acknowledgement (gfx9 counts loads and stores together)
    const int nrows = r1 > r0 + m ? (r1 - r0 - m + kMW - 1) / kMW : 0;
    if (lane < nrows) p.logits[r0 + m + kMW * lane] = res;
}

// row wave, after its x phase: its part of tile 0 once the tile waves have staged the layer's codes; the last of
// the eight to arrive finishes the block's q / k / v tile (RoPE, K / V into the cache, q / k / v published) and
// releases the tile waves' pass 2 (which would otherwise compete with this critical step for the matrix cores)
RK_DEV void row_pass1(const Params& p, int l, int64_t pos, uint32_t tag, const Work& wk, int rho, Lds& S) {
    flag_wait(p, S, &S.cnt_t0, (uint32_t)kMW * (l + 1));
    tile0_part(wk, rho, S);
    RK_TRACE(rho == 0, kTrTile0Done);
    if (arrive_last(&S.cnt_p1, (uint32_t)kRW * (l + 1))) {
        if (wk.nq) qkv_epilogue(p, l, pos, tag, S);
        RK_TRACE(wk.nq, kTrQkvPublished);
        flag_set(&S.p1_done, (uint32_t)l + 1);
    }
    // the row waves' weight loads follow the epilogue's stores, not the other way round (a store issued into a
    // memory queue full of loads waits for room)
    flag_wait(p, S, &S.p1_done, (uint32_t)l + 1);
}

// ---------------------------------------------------------------------------------------------- the roles
// W0..W3: per layer the row work (x phase, their part of tile 0), then this layer's K / V and o weights (issued
// only now, so the x poll and the gather never wait behind weight loads), the attention path (q poll, attention,
// one head's merge each, the combine, each wave's own merge of it, the o slice) and the row gather.
template <int REP>
RK_DEV void attention_main(const Params& p, uint32_t step, int64_t pos, int64_t tok, const Work& wk, Lds& S) {
    const int a = wave_id(), rho = a;
    for (int l = 0; l < p.L; ++l) {
        const uint32_t tag = tag_of(step, l);
        x_phase(p, l, step, pos, tok, rho, S);
        row_pass1(p, l, pos, tag, wk, rho, S);
        KVRegs kv;
        ORegs orr;
        kv_issue(p, l, pos, kv);
        o_issue(p, l, orr);
        if (split_of(p, pos).att) {
            QRegs qr;
            q_poll<REP>(p, S, pos, tag, qr);
            RK_TRACE(a == 0, kTrQPolled);
            attention<REP>(p, pos, kv, qr, S);
            RK_TRACE(a == 0, kTrAttnDone);
            arrive(&S.cnt_att);
            flag_wait(p, S, &S.cnt_att, (uint32_t)kAW * (l + 1));
#pragma unroll
            for (int r = a; r < REP; r += kAW) attention_merge<REP>(p, pos, tag, S, r);
            RK_TRACE(a == 0, kTrMerged);
        }
        comb_part(p, S, o_head(), pos, tag);
        RK_TRACE(a == 0, kTrCombDone);
        arrive(&S.cnt_comb);
        flag_wait(p, S, &S.cnt_comb, (uint32_t)kAW * (l + 1));
        const float asum = comb_merge(S);
        RK_TRACE(a == 0, kTrCombMerged);
        o_part(p, tag, orr, S, asum);
        RK_TRACE(a == 0, kTrOPublished);
        gather_phase(p, l, tag, rho, S);
    }
    x_final(p, step, pos, rho, S);
}

// W4..W11: per layer, once the row waves have finished tile 0: the block's other tiles (pass 2) -> act (the last
// arriver). The next layer's tiles are issued right after, and tile 0's codes copied to LDS for the row waves once
// they land (the head rows instead, after the last layer's pass 2).
RK_DEV void tile_main(const Params& p, uint32_t step, int64_t pos, const Work& wk, Lds& S) {
    (void)step;
    (void)pos;
    TileRegs tr;
    tile_issue(p, 0, S, wk, tr);
    stage_tile0(tr, S);
    arrive(&S.cnt_t0);
    for (int l = 0; l < p.L; ++l) {
        flag_wait(p, S, &S.p1_done, (uint32_t)l + 1);  // h staged, tile 0 done (its partials are in)
        RK_TRACE(wave_id() == kM0, kTrPass2Start);
        tile_compute<1, kMaxTiles>(tr, wk, S);
        if (arrive_last(&S.cnt_p2, (uint32_t)kMW * (l + 1))) {
            act_epilogue(p, wk, S);
            flag_set(&S.act_ready, (uint32_t)l + 1);
            RK_TRACE(true, kTrActReady);
        }
        if (l + 1 < p.L) {
            tile_issue(p, l + 1, S, wk, tr);
            flag_wait(p, S, &S.cnt_p1, (uint32_t)kRW * (l + 1));  // the row waves are done with this layer's codes
            stage_tile0(tr, S);
            arrive(&S.cnt_t0);
        } else {
            head_issue(p, tr);
        }
    }
    flag_wait(p, S, &S.cnt_head, (uint32_t)kRW);
    head_compute(p, tr, S);
}

// W12..W15: per layer the row work (x phase, their part of tile 0), then this layer's down columns (issued only
// now: the x poll and the gather never wait behind weight loads, and a load issued into a full memory queue would
// stall the wave ahead of tile 0), act -> the down partials of the block's channels for all 2048 rows, and the
// row gather.
RK_DEV void down_main(const Params& p, uint32_t step, int64_t pos, int64_t tok, const Work& wk, Lds& S) {
    const int rho = row_index();
    for (int l = 0; l < p.L; ++l) {
        const uint32_t tag = tag_of(step, l);
        x_phase(p, l, step, pos, tok, rho, S);
        row_pass1(p, l, pos, tag, wk, rho, S);
        DownRegs dr;
        down_issue(p, l, wk, dr);
        flag_wait(p, S, &S.act_ready, (uint32_t)l + 1);
        down_compute(p, tag, wk, dr, S);
        RK_TRACE(rho == 4, kTrDownPublished);
        gather_phase(p, l, tag, rho, S);
    }
    x_final(p, step, pos, rho, S);
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
#ifdef RK_DECODE_TRACE
    for (int i = tid; i < 64 * kTrEvents; i += kThreads) (&S.trace[0][0])[i] = 0ull;
#endif
    if (tid == 0) {
        S.p1_done = S.act_ready = 0u;
        S.cnt_ln = S.cnt_h = S.cnt_g = S.cnt_head = S.cnt_t0 = S.cnt_p1 = S.cnt_p2 = S.cnt_att = S.cnt_comb = 0u;
        S.abort = 0u;
    }
    __syncthreads();
    if (tid < kALanes) {
        __builtin_amdgcn_s_setprio(2);  // the attention path is the step's critical path
        attention_main<REP>(p, step, pos, tok, work_of(p, S), S);
    } else if (tid < 64 * kD0) {
        tile_main(p, step, pos, work_of(p, S), S);
    } else {
        down_main(p, step, pos, tok, work_of(p, S), S);
    }
#ifdef RK_DECODE_TRACE
    __syncthreads();
    if (g_trace)
        for (int i = tid; i < 64 * kTrEvents; i += kThreads)
            g_trace[(size_t)blockIdx.x * 64 * kTrEvents + i] = (&S.trace[0][0])[i];
#endif
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
    if (p.n_audio <= 0 || p.n_audio > 64 * kMW * nblocks) return RK_ERR_SHAPE;  // head rows: <= 64 per tile wave
    if (nblocks <= 0 || nblocks * 8 != kH) return RK_ERR_BLOCK;  // block b owns rows [8b, 8b + 8)
    if (p.nsp <= 0 || p.nsp > kMaxSplits || p.NKV * p.nsp > nblocks || p.inter / 16 > kMaxSlices * nblocks ||
        (p.S + p.nsp - 1) / p.nsp > kAW * kSlotsPerWave)  // every cached slot of a split is in registers
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

#ifdef RK_DECODE_TRACE
// trace builds only: the stamp buffer ([nblocks][64][kTrEvents] uint64, or NULL) and the event count
extern "C" __attribute__((visibility("default"))) int rk_decode_trace_set(unsigned long long* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_trace), &buf, sizeof(buf)) == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
extern "C" __attribute__((visibility("default"))) int rk_decode_trace_events(void) { return kTrEvents; }
#endif

extern "C" int rk_decode_get_limits(rk_decode_limits* out) {
    if (!out) return RK_ERR_NULL;
    out->max_tiles = kMaxTiles;
    out->first_pass = kFirstPass;
    out->max_slices = kMaxSlices;
    out->work_stride = kWork;
    out->slice_begin_col = kSliceBegin;
    out->slice_end_col = kSliceEnd;
    out->x_copies = kXRep;
    out->max_splits = kMaxSplits;
    out->max_slots_per_split = kAW * kSlotsPerWave;
    return RK_OK;
}
