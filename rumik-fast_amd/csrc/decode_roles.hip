// One batch-1 decode step of the Rumik decoder in ONE kernel launch, the grid split by role (gfx950, MI355X).
//
// Why one launch: a step is ~36 x 3 dependent GEMVs plus glue; as separate kernels each pays a launch gap and a
// cold memory-latency ramp. A grid of one 1024-thread block per CU stays resident for the whole step.
//
// Why roles: a poll (a coherent load of another block's tagged words) returns only after the loads its CU issued
// before it; on a CU that streams weights it takes ~2.2 us one way, on a CU that does not ~0.6-0.9 us even with
// the rest of the chip streaming. So the step's latency chain (x -> LayerNorm -> q/k/v -> attention -> combine ->
// o -> residual sum -> x) runs on blocks that carry little weight traffic, and the bulk of the bytes is streamed
// by blocks that poll once per layer and have slack:
//   latency blocks (kNL = 64, 8 per XCD): latency block j owns residual rows [32j, 32j + 32) (it gathers their
//     o and down partials and publishes them), attention split j % (64 / NKV) of KV head j / (64 / NKV), and the
//     combine of head j / 4 with the o projection of that head for rows [512 (j % 4), + 512);
//   stream blocks (192): a run of 3-4 MLP slices (16 channels: their 16 gate and 16 up rows, and the w_down
//     columns) each; x -> LayerNorm -> gate / up -> act -> down partials for all 2048 rows.
// The q/k/v projection sits on either side, chosen per step from pos (see "the roles" below): at short contexts
// the latency blocks poll x, run the LayerNorm and compute their group's q/k/v tiles; at long ones the stream
// blocks compute them after their LayerNorm and the latency blocks start each layer at the q poll.
// Inside a block all 16 waves go through the same phases and meet at block barriers (every wave reaches every
// barrier, an aborted wait included, so no barrier can hang); wave w owns column group w (columns
// [128w, 128w + 128)) of every 2048-vector: its part of x, its LayerNorm statistics and its h fragments, and the
// K-split share of every w_in tile (group w), so the tile MFMAs read only h the wave staged itself.
//
// Synchronization between blocks is dataflow: every value one block hands to another is a tagged 32-bit word
// (fp16 value | tag << 16, the tag names the step and the layer) written with an agent-scope atomic store and
// polled by the consumer with agent-scope loads (coherent across the XCDs' L2s). Every exchange buffer has two
// halves, used by even and odd layers: a block writes a half again only two layers later, and by then every
// block has finished reading it (a block at layer l + 2 has polled x of layer l + 2, or with stream q/k/v the q/k/v
// that the stream blocks computed from it; every latency block published that x after its layer-(l + 1) gather,
// which needed every block's layer-(l + 1) partials).
//
// Every wait is bounded by wall-clock time (200 ms): on expiry the kernel sets an abort bit in `status`, every
// later wait returns at once and the grid drains with garbage results. A residual sum that leaves the fp16 range
// (or is NaN) sets a sticky status bit and the step runs on.
#include "dequant.h"

namespace {

constexpr int kWaves = 16;
constexpr int kThreads = 64 * kWaves;
constexpr int kH = 2048;
constexpr int kHD = 128;
constexpr int kNG = kH / 128;                 // column groups: one per wave
constexpr int kNB = 256;                      // blocks (one per CU)
constexpr int kNL = 64;                       // latency blocks
constexpr int kNS = kNB - kNL;                // stream blocks
constexpr int kLRows = kH / kNL;              // residual rows per latency block (32)
constexpr int kLPairs = kLRows / 2;           // 16
constexpr int kOQ = 4;                        // o row quarters per head (16 heads x 4 = 64 latency blocks)
constexpr int kOItems = kH / kOQ * 4;         // 2048 items of 16 bytes per (head, quarter): 2 per thread
constexpr int kMaxTiles = 8;                  // gate / up tiles per stream block
constexpr int kMaxQkv = 2;                    // q / k / v tiles per stream block
constexpr int kMaxSlices = 4;                 // w_down 16-column slices per stream block
constexpr int kSlotsPerWave = 8;
constexpr int kMaxRep = 4;
constexpr int kMaxSplits = 16;
constexpr int kXRep = 16;                     // copies of x (no 8 KB stretch serves more than 16 pollers)
constexpr int kHeadAhead = 6;                 // head rows per stream wave loaded before the final x poll
constexpr uint64_t kWaitTicks = 20000000ull;  // 200 ms at the 100 MHz wall clock
constexpr unsigned kAbort = 1u, kTimeout = 2u, kBadPos = 4u, kNonFinite = 8u;

static_assert(kNS * kLPairs == 3 * kThreads, "three down-partial qwords per thread in the gather");
static_assert(kMaxSplits * kSlotsPerWave <= kWaves * kSlotsPerWave, "a split's slots fit the block's waves");

typedef rk_decode_roles_params Params;

RK_DEV float h16(uint16_t b) { return f16_bits_to_f32(b); }
RK_DEV uint16_t f16b(float v) { return f32_to_f16_bits(v); }
RK_DEV float rnd16(float v) { return (float)(_Float16)v; }
RK_DEV uint32_t pack_h2(float a, float b) {
    h2_t v;
    v.x = (_Float16)a;
    v.y = (_Float16)b;
    return as_u32(v);
}

// lane / thread indices through an empty asm: every use recomputes its addresses instead of the optimizer hoisting
// dozens of 64-bit addresses out of the layer loop, where they would stay live (and spill) across the whole step
RK_DEV int lane_id() { return (int)opaque_vgpr(threadIdx.x & 63); }
// The launch parameters (the kernel's only argument, at offset 0 of the kernarg segment) through a pointer the
// optimizer cannot see through: each layer re-reads the fields it uses with scalar loads instead of keeping every
// field, and every pointer derived from one, live across the whole kernel, which overflows the SGPRs into VGPR lanes
// (a v_writelane / v_readlane pair around every use).
RK_DEV const rk_decode_roles_params& fresh() {
    auto q = __builtin_amdgcn_kernarg_segment_ptr();  // constant address space: scalar loads
    asm volatile("" : "+s"(q));
    return *(const rk_decode_roles_params*)q;
}
RK_DEV int tid() { return (int)opaque_vgpr(threadIdx.x); }
RK_DEV int wave_id() { return __builtin_amdgcn_readfirstlane(threadIdx.x >> 6); }

// An index kept when `on` and replaced by 0 otherwise, by integer masking: a select written as `on ? i : 0` around a
// load can be compiled as a branch with a load on each side, and the merge then waits for every load in flight
// (observed: the K / V prefetch serialized into one round trip per load).
RK_DEV size_t keep_if(bool on, size_t i) { return i & (size_t)0 - (size_t)on; }

// ---------------------------------------------------------------------------------------------- coherent access
RK_DEV void st_coh(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RK_DEV uint32_t ld_coh(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV uint64_t ld_coh64(const uint64_t* p) {
    return __hip_atomic_load(const_cast<uint64_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV void st_coh64(uint64_t* p, uint64_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

// Traffic inside a latency group (the 64 / NKV latency blocks of one KV head: its q / k / v words and its attention
// split partials, produced and consumed only inside the group). With p.local_xcd the role table puts each group on
// one XCD, so these words are written into that XCD's L2 (nontemporal store, no write-through) and the group's
// agent-scope polls hit them there: a coherent load refetches a line from memory unless this L2 holds it dirty,
// and a line written on this XCD is dirty here. Measured one way: ~0.3 us through the L2 against ~0.6 us through
// memory. Without p.local_xcd they go through memory like every other exchange. (The dispatcher deals a launch's
// blocks to the XCDs round robin, block b to XCD (b + c) % 8 for some c of the launch, so blocks with equal b % 8
// share an XCD; a group split over XCDs would not see its words and its waits would time out, not read stale data:
// every word carries the tag of its step and layer.)
RK_DEV void st_grp(uint32_t* a, uint32_t v, bool local) {
    if (local)
        __builtin_nontemporal_store(v, a);
    else
        st_coh(a, v);
}
RK_DEV void st_grp64(uint64_t* a, uint64_t v, bool local) {
    if (local)
        __builtin_nontemporal_store(v, a);
    else
        st_coh64(a, v);
}

// ---------------------------------------------------------------------------------------------- tagged words
RK_DEV uint32_t tag_of(uint32_t step, int l) { return 1u + (step * 64u + (uint32_t)l) % 65535u; }
RK_DEV uint32_t tword(float v, uint32_t tag) { return (uint32_t)f16b(v) | (tag << 16); }
RK_DEV uint64_t tpair(float a, float b, uint32_t tag) {
    return (uint64_t)tword(a, tag) | ((uint64_t)tword(b, tag) << 32);
}
RK_DEV bool pair_ok(uint64_t q, uint32_t tag) {
    return (uint32_t)((q >> 16) & 0xFFFFu) == tag && (uint32_t)(q >> 48) == tag;
}
RK_DEV uint32_t pair_val(uint64_t q) { return (uint32_t)(q & 0xFFFFu) | ((uint32_t)(q >> 16) & 0xFFFF0000u); }

// ---------------------------------------------------------------------------------------------- phase trace
// A build option (RK_ROLES_TRACE; off in the product library): wall-clock stamps per (layer, event) in LDS, copied
// out at the end of the step to the buffer rk_roles_trace_set names ([block][64 layers][kTrEvents] uint64).
enum TraceEvent {
    kTrXPolled,       // x of the layer polled (wave 0)
    kTrLnDone,        // h staged (after the LayerNorm barrier)
    kTrTilesDone,     // the block's w_in tiles computed (latency: q/k/v, stream: gate / up)
    kTrQkvPublished,  // latency: q / k / v published (wave 0)
    kTrQPolled,       // latency: the split's q / k / v polled
    kTrSplitPublished,// latency: the split partials published (wave 0)
    kTrCombDone,      // latency: the head's attention output formed (poll included)
    kTrOPublished,    // latency: o partials published (wave 0)
    kTrGatherPolled,  // latency: the rows' partials polled (wave 0)
    kTrXPublished,    // latency: x rows published
    kTrActReady,      // stream: act formed
    kTrDownPublished, // stream: down partials published (wave 0)
    kTrXPolledAll,    // x polled by the block's last wave (max over waves)
    kTrLnBarrier,     // the LayerNorm statistics barrier passed
    kTrLoadsIssued,   // latency: this layer's K / V and o loads issued (max over waves)
    kTrAttnStart,     // latency: the barrier after the q poll passed
    kTrAttnEnd,       // latency: attention computed (max over the attention waves)
    kTrGatherAll,     // latency: the rows' partials polled by the block's last wave
    kTrGatherSum,     // latency: the gather's wave sums in LDS (after the barrier)
    kTrCombFirst,     // latency: the combine's first poll round returned
    kTrCombRounds,    // latency: the combine's poll rounds (a count, not a time)
    kTrCombStart,     // latency: the combine's poll started
    kTrCombChecked,   // latency: the combine's first poll round checked without completing (its loads returned)
    kTrSplitAcked,    // latency: the split partial stores acknowledged (max over the publishing waves)
    kTrCombDrained,   // latency: wave 0's earlier memory operations all complete at the combine's start
    kTrEvents
};
#ifdef RK_ROLES_TRACE
__device__ unsigned long long* g_roles_trace;
#define RK_TRACE(cond, ev)                                                      \
    do {                                                                        \
        if ((cond) && threadIdx.x == 0) S.trace[l][(ev)] = wall_clock64();      \
    } while (0)
#define RK_TRACE_MAX(ev)                                                                        \
    do {                                                                                        \
        if ((threadIdx.x & 63) == 0) atomicMax(&S.trace[l][(ev)], (unsigned long long)wall_clock64()); \
    } while (0)
#else
#define RK_TRACE(cond, ev) \
    do {                   \
    } while (0)
#define RK_TRACE_MAX(ev) \
    do {                 \
    } while (0)
#endif

// ---------------------------------------------------------------------------------------------- LDS layout
struct Lds {
    uint4 hfrag[kH / 8];                      // MFMA A fragments of h (group g: entries 16g .. 16g + 15)
    float hsum[kNG];                          // per-group sums of h
    float hbias[kNG];                         // per group: 64 x the sum of its odd-column h (biased high nibbles)
    alignas(16) uint32_t hnat[kH / 2];        // the final h as natural fp16 pairs (the int8 head's input)
    float2 lnst[kWaves];                      // per wave: sum and squared deviations of its 128 x values
    float tpart[kWaves][kMaxTiles + kMaxQkv][16];  // K-split partial dots of the block's tiles (per wave = group):
                                              //   gate / up tiles in slots [0, 8), q / k / v tiles in [8, 10)
    float act[kMaxSlices * 16];               // stream: act of the block's MLP channels
    alignas(16) uint32_t qst[kMaxRep + 2][64];  // latency: q of the group's heads, then k and v at pos (pairs)
    float s_m[kWaves][kMaxRep], s_l[kWaves][kMaxRep];
    float2 s_acc[kWaves][kMaxRep][64];        // per-wave attention partials
    alignas(16) float s_p[kWaves][kMaxRep][kSlotsPerWave];  // per wave: exp(score - max) of its slots, per head
    uint32_t attn[kHD / 2];                   // the head's attention output, natural fp16 pairs
    float asum;                               //   and the sum of its 128 values (the o projection's min term)
    float2 gpart[kWaves][kLPairs];            // gather: per wave, down-partial sums of the row pairs
    float2 gopart[4][kLPairs];                //   and o-partial sums (waves 0..3)
    float xrow[kLRows];                       // latency: the block's residual rows
    float rcos[kHD / 2], rsin[kHD / 2];       // RoPE cos / sin of pair i at pos
    uint32_t abort;
#ifdef RK_ROLES_TRACE
    unsigned long long trace[64][kTrEvents];
#endif
};

// ---------------------------------------------------------------------------------------------- waits
// true while a wait may go on; on expiry raise the abort bit (globally and in this block). `status` is the status
// word loaded in the same batch as the poll it belongs to, every kStatusEvery-th round only: every polling wave of
// the grid reading that one word every round would make it the hottest address in the memory system. SLEEP: the
// pause between rounds in units of 64 clocks (long for pollers with slack, so that waiting does not flood the
// memory system with coherent reads).
constexpr int kStatusEvery = 16;
#ifndef RK_SB_XSLEEP
#define RK_SB_XSLEEP 20
#endif
constexpr int kStreamXSleep = RK_SB_XSLEEP;  // ~0.5 us

template <int SLEEP = 1>
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
    __builtin_amdgcn_s_sleep(SLEEP);
    return true;
}

RK_DEV uint32_t status_every(const Params& p, int round) {
    return (round % kStatusEvery) == kStatusEvery - 1 ? ld_coh(p.status) : 0u;
}

// Poll N tagged fp16 pairs per lane (qword addresses from addr(k); nullptr = not needed) until every tag matches;
// val[k] receives the packed pair. Each iteration loads only the words this lane still lacks, plus the status
// word, as one batch with a single wait; a word's first validated value is kept. Wave-uniform control flow;
// false after an abort or a timeout.
template <int N, int SLEEP = 1, class Addr>
RK_DEV bool poll_pairs(const Params& p, Lds& S, uint32_t tag, Addr addr, uint32_t (&val)[N]) {
    static_assert(N <= 32, "pending mask");
    uint32_t pending = 0;
#pragma unroll
    for (int k = 0; k < N; ++k) {
        val[k] = 0u;
        if (addr(k)) pending |= 1u << k;
    }
    const uint64_t t0 = wall_clock64();
    uint64_t q[N];
#pragma unroll
    for (int k = 0; k < N; ++k) q[k] = 0;
    for (int round = 0;; ++round) {
#pragma unroll
        for (int k = 0; k < N; ++k)
            if (pending & (1u << k)) q[k] = ld_coh64(addr(k));
        const uint32_t st = status_every(p, round);
#pragma unroll
        for (int k = 0; k < N; ++k)
            if ((pending & (1u << k)) && pair_ok(q[k], tag)) {
                val[k] = pair_val(q[k]);
                pending &= ~(1u << k);
            }
        if (__all(pending == 0)) return true;
        if (!wait_more<SLEEP>(p, S, t0, st)) return false;
    }
}

// ---------------------------------------------------------------------------------------------- x / LayerNorm / h
// Four waves (one per SIMD) hold the 2048-vector: x-wave w (< kXW) lane L holds columns 512w + 8L .. + 7 (four
// tagged qwords of x, eight fp16 values). Fewer waves than 16 because every wave pays the reductions' dependent
// instruction chains in full: 16 waves of two values each measured ~0.8 us per LayerNorm (4 waves per SIMD, each
// wave64 VALU instruction holding the SIMD for 4 cycles), four waves of eight values a quarter of that.
constexpr int kXW = 4;
constexpr int kXCols = kH / kXW;  // 512

struct XIn {
    u4_t x;  // eight fp16 (natural pairs)
    u4_t w;  // their LayerNorm weights
};

RK_DEV bool x_wave() { return wave_id() < kXW; }

RK_DEV u4_t x_embed(const Params& p, int64_t tok) {
    const float es = h16(p.emb_s[tok]);
    const u2_t c = *reinterpret_cast<const u2_t*>(p.emb_q + (size_t)tok * kH + kXCols * wave_id() + 8 * lane_id());
    u4_t v;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const uint32_t wd = c[e >> 1] >> (16 * (e & 1));
        v[e] = pack_h2((float)(int8_t)(wd & 0xFF) * es, (float)(int8_t)((wd >> 8) & 0xFF) * es);
    }
    return v;
}

// x of layer l (l >= 1; published by the latency blocks at the end of layer l - 1 into half l & 1), this block's copy
template <int SLEEP>
RK_DEV bool x_poll(const Params& p, Lds& S, int l, uint32_t step, u4_t& xv) {
    const uint64_t* tx = reinterpret_cast<const uint64_t*>(p.tx) +
                         ((size_t)(l & 1) * kXRep + blockIdx.x % kXRep) * (kH / 2) + kXCols / 2 * wave_id() + 4 * lane_id();
    uint32_t v[4];
    const bool ok = poll_pairs<4, SLEEP>(p, S, tag_of(step, l - 1), [&](int k) -> const uint64_t* { return tx + k; }, v);
#pragma unroll
    for (int e = 0; e < 4; ++e) xv[e] = v[e];
    return ok;
}

// the lane's eight LayerNorm weights, loaded before the x poll so that their round trip overlaps it
RK_DEV u4_t ln_w_issue(const uint16_t* w) {
    return *reinterpret_cast<const u4_t*>(w + kXCols * wave_id() + 8 * lane_id());
}

// LayerNorm (reference engine/rumik_int4.py:38-43: biased variance, no bias) of the 2048-vector the x-waves hold:
// each x-wave's sum and sum of squared deviations from its own mean go through LDS and every x-wave combines the
// four in the same order (Chan's pairwise update: no cancellation). Every wave of the block reaches the barrier.
// Returns h = round((x - mean) rstd w) as the lane's eight values in natural pairs (x-waves only).
RK_DEV u4_t layer_norm(const Params& p, Lds& S, int l, const XIn& in) {
    const int w = wave_id();
    float x[8];
    if (x_wave()) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const h2_t v = as_h2(in.x[e]);
            x[2 * e] = (float)v.x;
            x[2 * e + 1] = (float)v.y;
        }
        float s = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) s += x[e];
        const float sum = wave_sum(s);
        const float m = sum * (1.0f / kXCols);
        float d2 = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) d2 += (x[e] - m) * (x[e] - m);
        const float m2 = wave_sum(d2);
        if (lane_id() == 0) S.lnst[w] = make_float2(sum, m2);
    }
    __syncthreads();
    RK_TRACE(true, kTrLnBarrier);
    u4_t h = {0u, 0u, 0u, 0u};
    if (x_wave()) {
        float tot = 0.f;
#pragma unroll
        for (int r = 0; r < kXW; ++r) tot += S.lnst[r].x;
        const float mean = tot * (1.0f / kH);
        float M2 = 0.f;
#pragma unroll
        for (int r = 0; r < kXW; ++r) {
            const float2 st = S.lnst[r];
            const float dm = st.x * (1.0f / kXCols) - mean;
            M2 += st.y + (float)kXCols * dm * dm;
        }
        const float rstd = 1.0f / sqrtf(M2 * (1.0f / kH) + p.eps);
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const h2_t wh = as_h2(in.w[e]);
            h[e] = pack_h2((x[2 * e] - mean) * rstd * (float)wh.x, (x[2 * e + 1] - mean) * rstd * (float)wh.y);
        }
    }
    return h;
}

// x-wave w: h -> MFMA A fragments + group sums. The lane's 8 columns are one 8-column block (global block 64w + L:
// group g = 4w + L / 16, block m = L % 16 of the group); pair_permute gives its dequant-order pairs
// (x0,x4),(x1,x5),(x2,x6),(x3,x7). The codes' tile layout gives MFMA lane j + 16s of 32-column chunk t4 the columns
// 32s + 8 t4 .. + 7 (a lane's 16 bytes are the row's bytes [16s, 16s + 16), word t4 feeding chunk t4), so block
// m = 4s + t4 goes to entry 16g + 4 t4 + s = 16g + 4 (m % 4) + m / 4, where chunk t4's A operand reads it.
// The tiles' high-nibble codes stay biased by 64 (dequant_frag_hi64): hbias[g] = 64 x the sum of the group's
// odd-column h, the pairs (x1,x5), (x3,x7), is what the tile dots subtract.
RK_DEV void stage_h(const u4_t& h, Lds& S) {
    const int L = lane_id(), w = wave_id();
    const int g = 4 * w + (L >> 4), m = L & 15;
    uint32_t hp[4];
    pair_permute(h, hp);
    S.hfrag[16 * g + 4 * (m & 3) + (m >> 2)] = make_uint4(hp[0], hp[1], hp[2], hp[3]);
    float s = 0.f, a = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const h2_t v = as_h2(h[e]);
        s += (float)v.x + (float)v.y;
        a += (float)v.y;  // natural pairs (x_2e, x_2e+1): the odd column
    }
    s += dpp<0x128>(s);  // row_ror 8
    s += dpp<0x124>(s);  // row_ror 4
    s += dpp<0x122>(s);  // row_ror 2
    s += dpp<0x121>(s);  // row_ror 1: every lane of the 16-lane row holds the group's sum
    a += dpp<0x128>(a);
    a += dpp<0x124>(a);
    a += dpp<0x122>(a);
    a += dpp<0x121>(a);
    if (m == 0) {
        S.hsum[g] = s;
        S.hbias[g] = 64.f * a;
    }
}

// ---------------------------------------------------------------------------------------------- w_in tiles
// w_in rows are [q | k | v | per 8 MLP channels: 8 gate rows, 8 up rows]; tile T = rows [16T, 16T + 16). win_t
// holds per (layer, tile, group) the 16 rows x 64 bytes of codes in lane order (lane j + 16s: row j, bytes
// [16s, 16s + 16) of the group); win_sm per (layer, tile, group, row) the word scale | min << 16.
RK_DEV size_t n_tiles(const Params& p) { return ((size_t)(p.NH + 2 * p.NKV) * kHD + 2 * p.inter) / 16; }

template <int NT>
struct TileRegs {
    u4_t w[NT];
    uint32_t sm[NT];
};

// wave w: group w of tiles tile(0) .. tile(nt - 1). The load count is fixed and every load unconditional (entries past
// nt read one 16-byte word of the layer's tile 0 in every lane, a single broadcast request, and are ignored), so the
// compiler can wait for exactly the loads a computation needs: a load skipped on some path would make it wait for
// every load in flight at that point.
template <int NT, class TileOf>
RK_DEV void tile_issue(const Params& p, int l, TileOf tile, int nt, TileRegs<NT>& r) {
    const int w = wave_id(), L = lane_id();
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const bool on = t < nt;
        const size_t T = (size_t)l * n_tiles(p) + keep_if(on, (size_t)tile(t));
        r.w[t] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p.win_t) + (T * kNG + w) * 64 + keep_if(on, L));
        r.sm[t] = p.win_sm[(T * kNG + w) * 16 + keep_if(on, L & 15)];
    }
}

// the wave's group of tiles [0, nt) -> S.tpart[w][slot0 + t][row]; per 32-column chunk two tiles' MFMAs are in
// flight (the register entries past nt are not computed: the branches are wave-uniform and hold no memory access)
template <int NT>
RK_DEV void tile_compute(const TileRegs<NT>& r, int nt, Lds& S, int slot0) {
    const int w = wave_id(), L = lane_id(), s = L >> 4;
    const Int4Masks km = int4_masks();
    const float hs = S.hsum[w], hb = S.hbias[w];
#pragma unroll
    for (int t0 = 0; t0 < NT; t0 += 2) {
        if (t0 >= nt) break;
        const bool two = t0 + 1 < nt;
        f4_t d[2] = {f4_t{0.f, 0.f, 0.f, 0.f}, f4_t{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int t4 = 0; t4 < 4; ++t4) {
            const h8_t A = __builtin_bit_cast(h8_t, S.hfrag[16 * w + 4 * t4 + s]);
            d[0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, dequant_frag_hi64(r.w[t0][t4], km), d[0], 0, 0, 0);
            if (t0 + 1 < NT && two)
                d[1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(A, dequant_frag_hi64(r.w[t0 + 1][t4], km), d[1], 0, 0, 0);
            __builtin_amdgcn_sched_barrier(0);
        }
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const int t = t0 + e;
            if (t < NT && L < 16 && t < nt) {
                const uint32_t sm = r.sm[t];
                S.tpart[w][slot0 + t][L] = __builtin_fmaf(d[e][0] - hb, h16((uint16_t)sm), h16((uint16_t)(sm >> 16)) * hs);
            }
        }
    }
}

// the projection output of tile t, row j: the 16 groups' partials summed in group order, rounded to fp16 (the
// reference keeps the fused projection's output in the activation dtype)
RK_DEV float tile_out(const Lds& S, int t, int j) {
    float y = 0.f;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) y += S.tpart[w][t][j];
    return rnd16(y);
}

// ---------------------------------------------------------------------------------------------- latency block
struct Split {
    bool att;  // this block computes a split
    int g, sp, start, end, n;
};

// slots per split: n / nsp rounded up to 8, at least min_chunk (short contexts use fewer, fuller splits)
RK_DEV int split_chunk(const Params& p, int n) { return max(p.min_chunk, ((n + p.nsp - 1) / p.nsp + 7) & ~7); }

RK_DEV Split split_of(const Params& p, int j, int64_t pos) {
    const int per = kNL / p.NKV;
    Split s;
    s.g = j / per;
    s.sp = j % per;
    s.n = (int)min<int64_t>(pos + 1, (int64_t)p.S);
    const int ch = split_chunk(p, s.n);
    s.start = min(s.sp * ch, s.n);
    s.end = min(s.start + ch, s.n);
    s.att = s.sp < p.nsp && s.start < s.end;
    return s;
}

RK_DEV int comb_splits(const Params& p, int64_t pos) {
    const int n = (int)min<int64_t>(pos + 1, (int64_t)p.S);
    const int ch = split_chunk(p, n);
    return min(p.nsp, (n + ch - 1) / ch);
}

// The split's slots go to slot groups of 8 (sg: slots [start + 8 sg, + 8)); each slot group is computed for all
// REP heads by one wave, or, when there are at most 8 slot groups (contexts up to 1024 at 16 splits), for half the
// heads each by two waves (hg = head group), so twice the waves share the latency-bound softmax and PV chains. Attention wave a =
// (w + 15) % 16 (wave 1 first: wave 0, which polls, joins only when all 16 are needed) takes (sg, hg) =
// (a / nhg, a % nhg). Scores use the chunk layout: lane (u = L / 8, c = L % 8) holds dims [16c, 16c + 16) of slot
// u's key; the PV product the dim-pair layout (lane L: dims 2L, 2L + 1 of every slot's value).
struct AttnPlan {
    int nsg, nhg, nact;  // slot groups, head groups, attention waves (nsg * nhg)
};

template <int REP>
RK_DEV AttnPlan attn_plan(const Split& s) {
    AttnPlan a;
    a.nsg = s.att ? (s.end - s.start + kSlotsPerWave - 1) / kSlotsPerWave : 0;
    a.nhg = (2 * a.nsg <= kWaves && REP >= 2) ? 2 : 1;
    a.nact = a.nsg * a.nhg;
    return a;
}

RK_DEV int attn_wave() { return (wave_id() + kWaves - 1) % kWaves; }

struct KVRegs {
    u4_t k[2];
    uint32_t v[kSlotsPerWave];
};

// Called by every wave of every latency block at the same point; a wave outside the split (or a block without one)
// reads one word of slot 0 in every lane instead (a broadcast request), so the load count stays fixed.
RK_DEV void kv_issue(const Params& p, int l, const Split& s, const AttnPlan& ap, KVRegs& kv) {
    const int a = attn_wave(), L = lane_id();
    const bool on = a < ap.nact;
    const size_t base = (((size_t)l * p.NKV + s.g) * p.S) * kHD;
    const u4_t* kr = reinterpret_cast<const u4_t*>(p.kc + base);
    const uint32_t* vr = reinterpret_cast<const uint32_t*>(p.vc + base);
    const int s0 = s.start + kSlotsPerWave * (a / max(ap.nhg, 1));
    const size_t ko = keep_if(on, (size_t)min(s0 + (L >> 3), p.S - 1) * (kHD / 8) + 2 * (L & 7));
    kv.k[0] = kr[ko];
    kv.k[1] = kr[ko + keep_if(on, 1)];
#pragma unroll
    for (int u = 0; u < kSlotsPerWave; ++u) kv.v[u] = vr[keep_if(on, (size_t)min(s0 + u, p.S - 1) * (kHD / 2) + L)];
}

// wave 0: q of the split's KV head (REP heads) and, when the split holds pos, k / v at pos -> S.qst
template <int REP>
RK_DEV bool q_poll(const Params& p, Lds& S, int l, const Split& s, int64_t pos, uint32_t tag) {
    const int L = lane_id();
    const bool has_pos = s.start <= pos && pos < s.end;
    const uint64_t* tq = reinterpret_cast<const uint64_t*>(p.tq) + (size_t)(l & 1) * (p.NH * kHD / 2) + opaque_vgpr(0u);
    const uint64_t* tkv = reinterpret_cast<const uint64_t*>(p.tkv) + (size_t)(l & 1) * (p.NKV * kHD) + opaque_vgpr(0u);
    uint32_t v[REP + 2];
    const bool ok = poll_pairs<REP + 2>(
        p, S, tag,
        [&](int k) -> const uint64_t* {
            if (k < REP) return tq + (size_t)(s.g * REP + k) * (kHD / 2) + L;
            if (!has_pos) return nullptr;
            return tkv + (size_t)((k - REP) * p.NKV + s.g) * (kHD / 2) + L;
        },
        v);
#pragma unroll
    for (int k = 0; k < REP + 2; ++k) S.qst[k < REP ? k : kMaxRep + k - REP][L] = v[k];
    return ok;
}

// Attention wave (sg, hg): heads hg HPW .. + HPW - 1 over slot group sg (m = -inf, l = 0 where no slot is
// valid). Each lane dots its 16 key dims with the same 16 dims of the query heads (v_dot2, fp32 sums) and the eight
// chunk lanes of a slot reduce with three DPP steps; per head the max and the sum of exp over the slots reduce over
// lane bits 3..5; PV reads the slots' p back from LDS (one broadcast read per 4 slots). Slots past the split's end are selected away (never multiplied
// by p = 0), so a NaN left in a slot beyond pos cannot reach the result (the reference's masked loads, other = 0).
// Results per (slot group, head) in S.s_m / s_l / s_acc.
template <int HPW>
RK_DEV void attention(const Params& p, const Split& s, int64_t pos, const KVRegs& kv, int sg, int hg, Lds& S) {
    const int L = lane_id();
    const int s0 = s.start + kSlotsPerWave * sg;
    const int u = L >> 3, c = L & 7;
    const bool valid = s0 + u < s.end;
    u4_t kk[2] = {kv.k[0], kv.k[1]};
    if (s0 + u == pos) {  // slot pos: the tagged k (dims 16c .. 16c + 15 = pairs 8c .. 8c + 7)
        kk[0] = *reinterpret_cast<const u4_t*>(&S.qst[kMaxRep][8 * c]);
        kk[1] = *reinterpret_cast<const u4_t*>(&S.qst[kMaxRep][8 * c + 4]);
    }
#pragma unroll
    for (int r = 0; r < HPW; ++r) {
        const int hd = hg * HPW + r;
        const u4_t q0 = *reinterpret_cast<const u4_t*>(&S.qst[hd][8 * c]);
        const u4_t q1 = *reinterpret_cast<const u4_t*>(&S.qst[hd][8 * c + 4]);
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
        float ls = e + dpp<0x128>(e);
        ls = sum_xor<16>(ls);
        ls = sum_xor<32>(ls);
        if (c == 0) S.s_p[sg][hd][u] = e;  // the slot's weight, read back by every lane below
        if (L == 0) {
            S.s_m[sg][hd] = m;
            S.s_l[sg][hd] = ls;
        }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");  // the wave's weights in LDS before its lanes read them
    float2 acc[HPW];
    float pw[HPW][kSlotsPerWave];
#pragma unroll
    for (int r = 0; r < HPW; ++r) {
        acc[r] = make_float2(0.f, 0.f);
        const f4_t* src = reinterpret_cast<const f4_t*>(S.s_p[sg][hg * HPW + r]);  // one broadcast read per 4 slots
#pragma unroll
        for (int q = 0; q < kSlotsPerWave / 4; ++q) {
            const f4_t v = src[q];
#pragma unroll
            for (int e = 0; e < 4; ++e) pw[r][4 * q + e] = v[e];
        }
    }
#pragma unroll
    for (int uu = 0; uu < kSlotsPerWave; ++uu) {
        const int su = s0 + uu;
        const h2_t vp = as_h2(su == pos ? S.qst[kMaxRep + 1][L] : (su < s.end ? kv.v[uu] : 0u));
        const float v0 = (float)vp.x, v1 = (float)vp.y;
#pragma unroll
        for (int r = 0; r < HPW; ++r) {
            acc[r].x = __builtin_fmaf(pw[r][uu], v0, acc[r].x);
            acc[r].y = __builtin_fmaf(pw[r][uu], v1, acc[r].y);
        }
    }
#pragma unroll
    for (int r = 0; r < HPW; ++r) S.s_acc[sg][hg * HPW + r][L] = acc[r];
}

// attention wave r (< REP), after the block barrier: head r's merge over the slot groups, published as the split's
// normalized partial (o / l, m, l) into half l & 1 of tpo / tml
template <int REP>
RK_DEV void split_publish(const Params& p, int l, const Split& s, int nsg, uint32_t tag, const Lds& S) {
    const int L = lane_id(), r = attn_wave();
    float M = -INFINITY;
    for (int g = 0; g < nsg; ++g) M = fmaxf(M, S.s_m[g][r]);
    float Lt = 0.f, ax = 0.f, ay = 0.f;
    for (int g = 0; g < nsg; ++g) {
        const float wt = S.s_m[g][r] == -INFINITY ? 0.f : __expf(S.s_m[g][r] - M);
        Lt += wt * S.s_l[g][r];
        ax += wt * S.s_acc[g][r][L].x;
        ay += wt * S.s_acc[g][r][L].y;
    }
    const size_t pi = ((size_t)(l & 1) * p.NH + s.g * REP + r) * p.nsp + s.sp;
    const float inv = Lt > 0.f ? 1.0f / Lt : 0.f;
    const bool local = p.local_xcd != 0;
    st_grp64(reinterpret_cast<uint64_t*>(p.tpo + pi * kHD) + L, tpair(ax * inv, ay * inv, tag), local);
    if (L == 0) {
        st_grp64(reinterpret_cast<uint64_t*>(p.tml) + 2 * pi,
                 (uint64_t)__builtin_bit_cast(uint32_t, M) | ((uint64_t)tag << 32), local);
        st_grp64(reinterpret_cast<uint64_t*>(p.tml) + 2 * pi + 1,
                 (uint64_t)__builtin_bit_cast(uint32_t, Lt) | ((uint64_t)tag << 32), local);
    }
}

// Wave 0: head h's combine out = sum_i w_i o_i / sum_i w_i, w_i = exp(m_i - max m) l_i over the cnt splits holding at
// least one slot (<= 16: one poll batch per iteration, lane L = dim pair, lane j % 16 also split j's (m, l)); the
// sums run in split order. The output, rounded to fp16, goes to S.attn as natural pairs, its sum to S.asum.
RK_DEV bool combine(const Params& p, Lds& S, int l, int h, int cnt, uint32_t tag) {
    const int L = lane_id();
    RK_TRACE(true, kTrCombStart);
#ifdef RK_ROLES_TRACE
    __builtin_amdgcn_s_waitcnt(0);
    RK_TRACE(true, kTrCombDrained);
#endif
    int rounds = 0;
    const size_t hb = ((size_t)(l & 1) * p.NH + h) * p.nsp;
    const uint32_t z = opaque_vgpr(0u);
    const uint64_t* po = reinterpret_cast<const uint64_t*>(p.tpo + hb * kHD) + L + z;
    const int jl = L % kMaxSplits;
    const uint64_t* tml = reinterpret_cast<const uint64_t*>(p.tml) + 2 * (hb + min(jl, p.nsp - 1)) + z;
    const uint64_t t0 = wall_clock64();
    uint32_t pending = cnt >= 32 ? 0xFFFFFFFFu : ((1u << cnt) - 1);
    bool ml_done = jl >= cnt;
    float mi = -INFINITY, li = 0.f;
    uint32_t val[kMaxSplits];
    uint64_t q[kMaxSplits], qm = 0, ql = 0;
#pragma unroll
    for (int k = 0; k < kMaxSplits; ++k) {
        val[k] = 0u;
        q[k] = 0;
    }
    bool ok = true;
    while (true) {
#pragma unroll
        for (int k = 0; k < kMaxSplits; ++k)
            if (pending & (1u << k)) q[k] = ld_coh64(po + (size_t)k * (kHD / 2));
        if (!ml_done) {
            qm = ld_coh64(tml);
            ql = ld_coh64(tml + 1);
        }
        const uint32_t st = status_every(p, rounds);
        if (rounds == 0) RK_TRACE(true, kTrCombFirst);
        ++rounds;
#pragma unroll
        for (int k = 0; k < kMaxSplits; ++k)
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
        RK_TRACE(rounds == 1, kTrCombChecked);
        if (!wait_more(p, S, t0, st)) {
            ok = false;
            break;
        }
    }
#ifdef RK_ROLES_TRACE
    if (threadIdx.x == 0) S.trace[l][kTrCombRounds] = (unsigned long long)rounds * 100ull;  // shown as "us" = rounds
#endif
    float mv = jl < cnt ? mi : -INFINITY;
    mv = fmaxf(mv, dpp<0x128>(mv));  // row_ror 8
    mv = fmaxf(mv, dpp<0x124>(mv));  // row_ror 4
    mv = fmaxf(mv, dpp<0x122>(mv));  // row_ror 2
    const float M = fmaxf(mv, dpp<0x121>(mv));  // row_ror 1
    const float wl = (jl < cnt && mi != -INFINITY) ? __expf(mi - M) * li : 0.f;
    float ax = 0.f, ay = 0.f, Ls = 0.f;
#pragma unroll
    for (int k = 0; k < kMaxSplits; ++k) {
        const float wk = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, wl), k));
        const h2_t o = as_h2(val[k]);
        ax = __builtin_fmaf(wk, (float)o.x, ax);
        ay = __builtin_fmaf(wk, (float)o.y, ay);
        Ls += wk;
    }
    const float inv = Ls > 0.f ? 1.0f / Ls : 0.f;
    const float a0 = rnd16(ax * inv), a1 = rnd16(ay * inv);
    S.attn[L] = pack_h2(a0, a1);
    const float as = wave_sum(a0 + a1);
    if (L == 0) S.asum = as;
    return ok;
}

// ---------------------------------------------------------------------------------------------- o slice
// Latency block (head h, quarter r) computes the o projection of head h's attention output for rows
// [512r, 512r + 512): 2048 items (row 512r + i / 4, 32-column chunk i % 4 of the head's 128 columns), one
// 16-byte load each, thread g taking items g and g + 1024. The head's columns are one quantization group, so each
// row has one scale | min word (wo_sm[layer][head][row]: a block's 512 words are contiguous).
struct ORegs {
    u4_t w[2];
    uint32_t sm[2];
};

RK_DEV void o_issue(const Params& p, int l, int h, int r, ORegs& o) {
    const int g = tid();
    const u4_t* base = reinterpret_cast<const u4_t*>(p.wo_q) + ((size_t)(l * p.NH + h) * kOQ + r) * kOItems;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = g + kThreads * k;
        o.w[k] = __builtin_nontemporal_load(base + i);
        o.sm[k] = p.wo_sm[((size_t)l * p.NH + h) * kH + (kH / kOQ) * r + (i >> 2)];
    }
}

// the items' dots, summed per row over the 4 lanes of its chunks; lanes i % 8 == 0 publish rows (i/4, i/4 + 1) as
// one tagged pair to top[half][consumer latency block][head][32 rows]
RK_DEV void o_publish(const Params& p, int l, uint32_t tag, int h, int r, const ORegs& o, const Lds& S) {
    const int g = tid(), L = lane_id();
    const Int4Masks km = int4_masks();
    float vals[2];
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int c = (g + kThreads * k) & 3;
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
        vals[k] = __builtin_fmaf(v, h16((uint16_t)o.sm[k]), h16((uint16_t)(o.sm[k] >> 16)) * S.asum);
    }
    asm volatile("" ::"v"(vals[0]), "v"(vals[1]));  // both items before either store
    uint64_t* top = reinterpret_cast<uint64_t*>(p.top) + (size_t)(l & 1) * kNL * p.NH * kLPairs;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
        const int i = g + kThreads * k;
        const float nxt = dpp<0x104>(vals[k]);  // row_shl 4: the next row's total (lane + 4, same 16-lane row)
        if ((L & 7) == 0) {
            const int row = (kH / kOQ) * r + (i >> 2);  // even
            st_coh64(top + ((size_t)(row / kLRows) * p.NH + h) * kLPairs + (row % kLRows) / 2, tpair(vals[k], nxt, tag));
        }
    }
}

// ---------------------------------------------------------------------------------------------- gather (latency)
// Latency block j polls its rows' partials in one batch per iteration: thread g takes the down-partial qwords
// g, g + 1024, g + 2048 of its run tdp[half][j][192 producers][16 pairs] (producer q / 16, row pair q % 16 = g % 16)
// and, g < 256, the o-partial qword g of top[half][j][16 heads][16 pairs]. Sums per row pair: the four lanes of a
// wave sharing L % 16, then the 16 waves through LDS, each in a fixed order (the result does not depend on arrival
// order). Wave 0 then forms x = round(x + round(o) + round(d)) (as add_ln) and publishes the 32 rows in kXRep copies.
RK_DEV void gather(const Params& p, Lds& S, int l, uint32_t tag, int j) {
    const int g = tid(), L = lane_id(), w = wave_id();
    const uint64_t* dp = reinterpret_cast<const uint64_t*>(p.tdp) + ((size_t)(l & 1) * kNL + j) * kNS * kLPairs + g;
    const uint64_t* op = reinterpret_cast<const uint64_t*>(p.top) + ((size_t)(l & 1) * kNL + j) * p.NH * kLPairs + g;
    const bool with_o = g < p.NH * kLPairs;
    uint32_t v[4];
    poll_pairs<4>(p, S, tag,
                  [&](int k) -> const uint64_t* {
                      if (k < 3) return dp + kThreads * k;
                      return with_o ? op : nullptr;
                  },
                  v);
    RK_TRACE(true, kTrGatherPolled);
    RK_TRACE_MAX(kTrGatherAll);
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const h2_t hv = as_h2(v[k]);
        d0 += (float)hv.x;
        d1 += (float)hv.y;
    }
    const h2_t ov = as_h2(v[3]);  // zero where not polled
    float o0 = (float)ov.x, o1 = (float)ov.y;
    d0 = sum_xor<16>(sum_xor<32>(d0));
    d1 = sum_xor<16>(sum_xor<32>(d1));
    o0 = sum_xor<16>(sum_xor<32>(o0));
    o1 = sum_xor<16>(sum_xor<32>(o1));
    if (L < kLPairs) {
        S.gpart[w][L] = make_float2(d0, d1);
        if (w < 4) S.gopart[w][L] = make_float2(o0, o1);
    }
    __syncthreads();
    RK_TRACE(true, kTrGatherSum);
    if (w != 0) return;
    bool bad = false;
    if (L < kLPairs) {
        float2 d = make_float2(0.f, 0.f), o = make_float2(0.f, 0.f);
#pragma unroll
        for (int r = 0; r < kWaves; ++r) {
            d.x += S.gpart[r][L].x;
            d.y += S.gpart[r][L].y;
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            o.x += S.gopart[r][L].x;
            o.y += S.gopart[r][L].y;
        }
        const float x0 = rnd16(S.xrow[2 * L] + rnd16(o.x) + rnd16(d.x));
        const float x1 = rnd16(S.xrow[2 * L + 1] + rnd16(o.y) + rnd16(d.y));
        S.xrow[2 * L] = x0;
        S.xrow[2 * L + 1] = x1;
        bad = !(__builtin_isfinite(x0) && __builtin_isfinite(x1));  // beyond 65504 the fp16 sum is inf
    }
    if (__ballot(bad) != 0ull && L == 0) atomicOr(p.status, kNonFinite);
    __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");  // the 16 lanes' rows before every lane reads them
    const int pr = L & (kLPairs - 1);
    const uint64_t word = tpair(S.xrow[2 * pr], S.xrow[2 * pr + 1], tag);
    uint64_t* tx = reinterpret_cast<uint64_t*>(p.tx) + (size_t)((l + 1) & 1) * kXRep * (kH / 2) + kLPairs * j + pr;
#pragma unroll
    for (int c = 0; c < kXRep / 4; ++c) st_coh64(tx + (size_t)(4 * c + (L >> 4)) * (kH / 2), word);
    RK_TRACE(true, kTrXPublished);
}

// ---------------------------------------------------------------------------------------------- stream block
// w_down by 16-column slices: wd_t per (layer, slice) 2048 rows x 8 bytes, so thread g's 16 bytes of a slice are
// rows 2g, 2g + 1; wd_sm per (layer, 128-column group) the 2048 rows' scale | min << 16 (a block's 3-4 slices
// span at most two groups).
struct DownRegs {
    u4_t c[kMaxSlices];
    u2_t sm[2];
};

RK_DEV void down_issue(const Params& p, int l, int sb, int se, DownRegs& d) {
    const int g = tid();
    const int nsl = p.inter / 16, ngd = p.inter / 128, gb = sb / 8;
#pragma unroll
    for (int i = 0; i < kMaxSlices; ++i) {  // slices past se: one broadcast word of the layer's slice 0, ignored
        const bool on = sb + i < se;
        d.c[i] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p.wd_t) +
                                            ((size_t)l * nsl + keep_if(on, sb + i)) * (kH / 2) + keep_if(on, g));
    }
#pragma unroll
    for (int q = 0; q < 2; ++q)
        d.sm[q] = *reinterpret_cast<const u2_t*>(p.wd_sm + ((size_t)l * ngd + min(gb + q, ngd - 1)) * kH + 2 * g);
}

// rows 2g, 2g + 1 of the down projection over the block's channels, published as one tagged pair into the run of
// the latency block that owns them: tdp[half][g / 16][stream index][g % 16]
RK_DEV void down_publish(const Params& p, int l, uint32_t tag, int si, int sb, int se, const DownRegs& dr,
                         const Lds& S) {
    const int g = tid();
    const Int4Masks km = int4_masks();
    const int gb = sb / 8;
    float d0 = 0.f, d1 = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxSlices; ++i) {
        if (sb + i >= se) continue;
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
        const int q = (sb + i) / 8 - gb;
        float dd[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {  // row 2g + hh: dwords 2hh, 2hh + 1
            float dot = 0.f;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                h2_t pr[4];
                dequant_pairs(dr.c[i][2 * hh + e], km, pr);
#pragma unroll
                for (int kk = 0; kk < 4; ++kk) dot = dot2(pr[kk], as_h2(xp[4 * e + kk]), dot);
            }
            const uint32_t sm = q == 0 ? dr.sm[0][hh] : dr.sm[1][hh];
            dd[hh] = __builtin_fmaf(dot, h16((uint16_t)sm), h16((uint16_t)(sm >> 16)) * asum);
        }
        d0 += dd[0];
        d1 += dd[1];
    }
    uint64_t* out = reinterpret_cast<uint64_t*>(p.tdp) + ((size_t)(l & 1) * kNL + g / kLPairs) * kNS * kLPairs +
                    (size_t)si * kLPairs + g % kLPairs;
    st_coh64(out, tpair(d0, d1, tag));
}

// wave 0, after the tile barrier: lane (tile t = L / 8, channel j = L % 8): gate row j and up row j + 8 of the
// block's tile t -> act of channel 8t + j of the block (silu(gate) * up with gate and up rounded first, as post)
RK_DEV void act_epilogue(int nt, Lds& S) {
    const int L = lane_id();
    const int t = L >> 3, j = L & 7;
    if (t >= nt) return;
    const float gt = tile_out(S, t, j), up = tile_out(S, t, j + 8);
    S.act[8 * t + j] = rnd16(gt / (1.0f + __expf(-gt)) * up);
}

// ---------------------------------------------------------------------------------------------- head
// int8 audio head rows si + 192 (w + 16k) (k = 0, 1, ...) of stream block si, wave w (the stream blocks' registers
// are free once their last down slices are computed, early in the last layer, so the head's 33.6 MB stream runs
// under the rest of that layer); the first kHeadAhead rows are loaded then, the rest when used. Lane k keeps the
// wave's k-th logit (<= 64 rows per wave: checked on the host); the stores come after the loop.
struct HeadRegs {
    u4_t w[2 * kHeadAhead];
    uint16_t s;  // lane k: the fp16 scale of the wave's k-th row (loaded with the rows, not one round trip per row)
};

RK_DEV int head_row(int si, int k) { return si + kNS * (wave_id() + kWaves * k); }

RK_DEV void head_issue(const Params& p, int si, HeadRegs& hr) {
    const int L = lane_id();
#pragma unroll
    for (int k = 0; k < kHeadAhead; ++k) {
        const int r = min(head_row(si, k), p.n_audio - 1);
        const u4_t* qr = reinterpret_cast<const u4_t*>(p.head_q + (size_t)r * kH);
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) hr.w[2 * k + jj] = __builtin_nontemporal_load(qr + L + 64 * jj);
    }
    hr.s = p.head_s[min(head_row(si, L), p.n_audio - 1)];
}

RK_DEV void head_compute(const Params& p, int si, const HeadRegs& hr, const Lds& S) {
    const int L = lane_id();
    float res = 0.f;
    int nrows = 0;
    for (int k = 0;; ++k) {
        const int r = head_row(si, k);
        if (r >= p.n_audio) break;
        u4_t q[2];
        if (k < kHeadAhead) {
            q[0] = hr.w[0];
            q[1] = hr.w[1];
#pragma unroll
            for (int kk = 1; kk < kHeadAhead; ++kk)
                if (k == kk) {
                    q[0] = hr.w[2 * kk];
                    q[1] = hr.w[2 * kk + 1];
                }
        } else {
            const u4_t* qr = reinterpret_cast<const u4_t*>(p.head_q + (size_t)r * kH);
            q[0] = qr[L];
            q[1] = qr[L + 64];
        }
        float acc = 0.f;
#pragma unroll
        for (int jj = 0; jj < 2; ++jj) {  // 128 chunks of 16 columns
            const int c = L + 64 * jj;
            uint32_t xp[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) xp[e] = S.hnat[8 * c + e];
            acc += chunk_dot_int8<true>(q[jj], xp);
        }
        acc = wave_sum(acc);
        if (L == k) res = acc * h16(hr.s);
        ++nrows;
    }
    if (L < nrows) p.logits[head_row(si, L)] = res;
}

// after the last layer, every stream block: the final LayerNorm -> h as natural pairs (and, stream block 0, the
// exported final hidden state), then the block's head rows
RK_DEV void final_phase(const Params& p, Lds& S, uint32_t step, int64_t pos, int si, const HeadRegs& hr) {
    XIn in;
    in.x = u4_t{0u, 0u, 0u, 0u};
    in.w = in.x;
    if (x_wave()) {
        in.w = ln_w_issue(p.norm_w);
        x_poll<1>(p, S, p.L, step, in.x);
        if (p.L == 1 && si == 0 && threadIdx.x == 0) p.pos[0] = pos + 1;  // every block has read pos
    }
    const u4_t h = layer_norm(p, S, p.L, in);
    if (x_wave()) {
        const int c = 64 * wave_id() + lane_id();  // the lane's 8-column block: natural pairs 4c .. 4c + 3
        *reinterpret_cast<uint4*>(&S.hnat[4 * c]) = make_uint4(h[0], h[1], h[2], h[3]);
        if (p.hn && si == 0) reinterpret_cast<uint4*>(p.hn)[c] = make_uint4(h[0], h[1], h[2], h[3]);
    }
    __syncthreads();
    head_compute(p, si, hr, S);
}

// the start of layer l in a stream block: x (the embedding at layer 0, else polled) and the LayerNorm weights, in
// the x-waves (the other waves return at once). Stream block 0 advances pos once x of layer 1 is in: that x needed
// every latency block's gather of layer 0, which needed every block's partials, so every block has read pos.
// XSLEEP: the x poll's pause between rounds, in units of 64 clocks.
template <int XSLEEP>
RK_DEV XIn x_fetch(const Params& p, Lds& S, int l, uint32_t step, int64_t pos, int64_t tok, int si) {
    XIn in;
    in.x = u4_t{0u, 0u, 0u, 0u};
    in.w = in.x;
    if (!x_wave()) return in;
    in.w = ln_w_issue(p.ln_w + (size_t)l * kH);
    if (l == 0) {
        in.x = x_embed(p, tok);
    } else {
        x_poll<XSLEEP>(p, S, l, step, in.x);
        if (l == 1 && si == 0 && threadIdx.x == 0) p.pos[0] = pos + 1;
    }
    RK_TRACE(true, kTrXPolled);
    RK_TRACE_MAX(kTrXPolledAll);
    return in;
}

// -> LayerNorm -> h staged
RK_DEV void x_norm(const Params& p, Lds& S, int l, const XIn& in) {
    const u4_t h = layer_norm(p, S, l, in);
    if (x_wave()) stage_h(h, S);
    __syncthreads();
    RK_TRACE(true, kTrLnDone);
}

// ---------------------------------------------------------------------------------------------- the roles
// Two placements of the q / k / v projection, chosen per step from pos (the same in every block):
//   latency q/k/v (pos < p.stream_qkv_from): every latency block polls x, runs the LayerNorm and computes nq =
//     (NH + 2 NKV) * 8 / 64 q/k/v tiles of its own group's list, [q tiles of heads g REP .. g REP + REP - 1 | k
//     tiles of KV head g | v tiles of KV head g], member i = j % (64 / NKV) taking entries [i nq, i nq + nq), so the
//     group's q/k/v exchange stays in the group's XCD;
//   stream q/k/v (pos >= p.stream_qkv_from): stream block si computes w_in tiles [qkv_first(si), qkv_first(si + 1))
//     of the first NQT = (NH + 2 NKV) * 8 ([q of every head | k | v]) right after its LayerNorm and publishes them
//     written through; the latency blocks skip x, the LayerNorm and the tiles, and start each layer at the q poll.
// Measured (36 layers, us per token at ctx 256 / 512 / 1024 / 2048): latency q/k/v 500 / 520 / 539 / 585, stream
// q/k/v 510 / 499 / 500 / 522. The second takes ~4 us of x / LayerNorm / tiles per layer off the latency chain; at
// short contexts that gain is spent in the stream blocks, whose MLP then ends later and whose next-layer weight
// burst lands on the gather's polls.
RK_DEV int qkv_tile(const Params& p, int j, int u) {
    constexpr int kTH = kHD / 16;  // tiles per head
    const int per = kNL / p.NKV, rep = p.NH / p.NKV, nq = (rep + 2) * kTH / per;
    const int g = j / per, t = (j % per) * nq + u, qt = rep * kTH;
    if (t < qt) return g * qt + t;
    if (t < qt + kTH) return p.NH * kTH + g * kTH + (t - qt);
    return (p.NH + p.NKV) * kTH + g * kTH + (t - qt - kTH);
}

RK_DEV int qkv_first(const Params& p, int si) {
    return (int)((long)si * ((p.NH + 2 * p.NKV) * (kHD / 16)) / kNS);
}

// q/k/v tile epilogue, wave 0 lane (tile t = L / 16, row j = L % 16; the tile's partials in S.tpart slot slot0 + t,
// its w_in tile index tile(t)): RoPE on q / k rows (pairs 2i, 2i + 1 sit in adjacent lanes), published tagged (into
// the group's L2 when local, else written through); k and v also written into the cache at pos
template <class TileOf>
RK_DEV void qkv_epilogue(const Params& p, int l, int64_t pos, uint32_t tag, TileOf tile, int nq, int slot0,
                         bool local, const Lds& S) {
    const int L = lane_id();
    const int t = L >> 4, j = L & 15;
    const float y = t < nq ? tile_out(S, slot0 + t, j) : 0.f;
    const float partner = dpp<0xB1>(y);  // row j ^ 1 (quad_perm [1,0,3,2])
    if (t >= nq) return;
    const int NH = p.NH, NKV = p.NKV;
    const int row = tile(t) * 16 + j;
    const int qk_rows = (NH + NKV) * kHD;
    uint32_t* tq = p.tq + (size_t)(l & 1) * NH * kHD;
    uint32_t* tkv = p.tkv + (size_t)(l & 1) * 2 * NKV * kHD;
    if (row < qk_rows) {
        float out = y;
        if ((p.sliding >> l) & 1ull) {  // interleaved RoPE: pairs (2i, 2i + 1)
            const int dd = row % kHD;
            const float c = S.rcos[dd >> 1], sn = S.rsin[dd >> 1];
            out = (dd & 1) ? (y * c + partner * sn) : (y * c - partner * sn);
        }
        out = rnd16(out);
        if (row < NH * kHD) {
            st_grp(tq + row, tword(out, tag), local);
        } else {
            const int r2 = row - NH * kHD;
            st_grp(tkv + r2, tword(out, tag), local);
            p.kc[(((size_t)l * NKV + r2 / kHD) * p.S + pos) * kHD + r2 % kHD] = f16b(out);
        }
    } else {
        const int r2 = row - qk_rows;
        st_grp(tkv + NKV * kHD + r2, tword(y, tag), local);
        p.vc[(((size_t)l * NKV + r2 / kHD) * p.S + pos) * kHD + r2 % kHD] = f16b(y);
    }
}

// Latency block j, one layer: [latency q/k/v: x -> LayerNorm -> its q/k/v tiles, published] the split's q poll ->
// attention -> split partials; the head's combine -> o slice -> o partials; the rows' gather -> x rows. The block's
// residual rows live in S.xrow (the gather updates them).
// Load placement: vector-memory results return in issue order per wave, and a CU's loads share one queue, so a
// poll waits for the loads issued before it; each load is therefore issued right after a poll and needed before
// (or long after) the next one. Stream q/k/v: this layer's K / V slots and o items are issued by every wave at the
// layer's start and drain while the stream blocks compute q/k/v. Latency q/k/v: they are issued right after the x
// poll (by the x-waves after the LayerNorm: issued before it, they queue ahead of the statistics), the next layer's
// tiles once this layer's are computed, by wave 0 (which polls q and the combine) only after its combine poll.
// (Every load sequence is unconditional and in the same place for all layers: a load skipped or moved on some path
// makes the compiler's counter waits on that path's merge conservative.) LAST: the last layer, which issues no
// next-layer loads (the loop is peeled so that every load sequence is straight-line code: see tile_issue).
template <int REP>
struct LatencyRegs {
    static constexpr int NQ = REP == 4 ? 3 : 4;  // latency q/k/v tiles per block (16 q heads, 64 / REP kv heads)
    TileRegs<NQ> tr;
    KVRegs kv;
    ORegs orr;
};

template <int REP, bool SQ, bool LAST>
RK_DEV void latency_layer(const Params& p_in, Lds& S, uint32_t step, int64_t pos, int64_t tok, int j, int l,
                          const Split& s, int cnt, LatencyRegs<REP>& R) {
    const Params& p = fresh();
    (void)p_in;
    constexpr int NQ = LatencyRegs<REP>::NQ;
    const int w = wave_id();
    const uint32_t tag = tag_of(step, l);
    const int h = j / kOQ, r = j % kOQ;
    const AttnPlan ap = attn_plan<REP>(s);
    if constexpr (SQ) {
        kv_issue(p, l, s, ap, R.kv);
        o_issue(p, l, h, r, R.orr);
        RK_TRACE_MAX(kTrLoadsIssued);
        if (w == 0 && s.att) q_poll<REP>(p, S, l, s, pos, tag);
        RK_TRACE(true, kTrQPolled);
    } else {
        const auto qt = [&](int u) { return qkv_tile(p, j, u); };
        const XIn in = x_fetch<1>(p, S, l, step, pos, tok, -1);
        if (!x_wave()) {
            kv_issue(p, l, s, ap, R.kv);
            o_issue(p, l, h, r, R.orr);
        }
        x_norm(p, S, l, in);
        if (x_wave()) {
            kv_issue(p, l, s, ap, R.kv);
            o_issue(p, l, h, r, R.orr);
        }
        RK_TRACE_MAX(kTrLoadsIssued);
        tile_compute<NQ>(R.tr, NQ, S, 0);
        __syncthreads();
        RK_TRACE(true, kTrTilesDone);
        if (w == 0) {
            qkv_epilogue(p, l, pos, tag, qt, NQ, 0, p.local_xcd != 0, S);
            RK_TRACE(true, kTrQkvPublished);
            if (s.att) q_poll<REP>(p, S, l, s, pos, tag);
            RK_TRACE(true, kTrQPolled);
        } else if constexpr (!LAST) {
            tile_issue<NQ>(p, l + 1, qt, NQ, R.tr);
        }
    }
    __syncthreads();
    RK_TRACE(true, kTrAttnStart);
    if (s.att) {
        const int a = attn_wave();
        if (a < ap.nact) {
            if (ap.nhg == 2)
                attention<REP / 2>(p, s, pos, R.kv, a / 2, a % 2, S);
            else
                attention<REP>(p, s, pos, R.kv, a, 0, S);
            RK_TRACE_MAX(kTrAttnEnd);
        }
        __syncthreads();
        if (attn_wave() < REP) {
            split_publish<REP>(p, l, s, ap.nsg, tag, S);
#ifdef RK_ROLES_TRACE
            __builtin_amdgcn_s_waitcnt(0);
            RK_TRACE_MAX(kTrSplitAcked);
#endif
        }
        RK_TRACE(true, kTrSplitPublished);
    }
    if (w == 0) {
        combine(p, S, l, h, cnt, tag);
        RK_TRACE(true, kTrCombDone);
        // latency q/k/v: wave 0 polls, so its share of the next layer's tiles goes out only now, after its q and
        // combine polls (a poll returns only after the wave's earlier loads), and lands before its gather poll
        if constexpr (!SQ && !LAST) tile_issue<NQ>(p, l + 1, [&](int u) { return qkv_tile(p, j, u); }, NQ, R.tr);
    }
    __syncthreads();
    o_publish(p, l, tag, h, r, R.orr, S);
    RK_TRACE(true, kTrOPublished);
    gather(p, S, l, tag, j);
    __syncthreads();
}

// layer 0's residual rows of latency block j: the embedding rows 32j .. 32j + 31, rounded to fp16 as x_embed does
RK_DEV void x_rows_init(const Params& p, Lds& S, int64_t tok, int j) {
    const int t = threadIdx.x;
    if (t < kLRows) {
        const float es = h16(p.emb_s[tok]);
        S.xrow[t] = rnd16((float)p.emb_q[(size_t)tok * kH + kLRows * j + t] * es);
    }
}

template <int REP, bool SQ>
RK_DEV void latency_run(const Params& p, Lds& S, uint32_t step, int64_t pos, int64_t tok, int j) {
    LatencyRegs<REP> R;
    x_rows_init(p, S, tok, j);  // read by the first gather, several barriers later
    const Split s = split_of(p, j, pos);  // the same for every layer of the step
    const int cnt = comb_splits(p, pos);
    if constexpr (!SQ)
        tile_issue<LatencyRegs<REP>::NQ>(p, 0, [&](int u) { return qkv_tile(p, j, u); }, LatencyRegs<REP>::NQ, R.tr);
    for (int l = 0; l + 1 < p.L; ++l) latency_layer<REP, SQ, false>(p, S, step, pos, tok, j, l, s, cnt, R);
    latency_layer<REP, SQ, true>(p, S, step, pos, tok, j, p.L - 1, s, cnt, R);
}

// Stream block si (slices [sb, se)), one layer: x -> LayerNorm -> [stream q/k/v: its q / k / v tiles, published]
// -> gate / up tiles -> act -> down partials for all 2048 rows -> the next layer's tiles issued (the last layer
// issues the block's head rows instead). Stream q/k/v: wave 0's q / k / v stores go out before any wave issues this
// layer's down columns (a barrier between them), so they do not queue behind them; the down columns then load
// under the gate / up tiles. Latency q/k/v: the down columns are issued right after the LayerNorm. Either way the
// block's ~200 KB per layer goes out in two parts a few microseconds apart, and the tiles, issued last, land before
// the block's next x poll (results return in issue order), which therefore does not re-poll while the chip streams.
struct StreamRegs {
    TileRegs<kMaxTiles> tr;
    TileRegs<kMaxQkv> qr;
    DownRegs dr;
    HeadRegs hr;
};

template <bool SQ, bool LAST>
RK_DEV void stream_layer(const Params& p_in, Lds& S, uint32_t step, int64_t pos, int64_t tok, int si, int sb, int se,
                         int l, StreamRegs& R) {
    const Params& p = fresh();
    (void)p_in;
    const int w = wave_id();
    const uint32_t tag = tag_of(step, l);
    const int t0 = (int)(n_tiles(p) - (size_t)p.inter / 8) + 2 * sb, nt = 2 * (se - sb);
    const int q0 = qkv_first(p, si), nq = qkv_first(p, si + 1) - q0;
    const auto mlp_tiles = [&](int t) { return t0 + t; };
    const auto qkv_tiles = [&](int t) { return q0 + t; };
    const XIn in = x_fetch<kStreamXSleep>(p, S, l, step, pos, tok, si);
    x_norm(p, S, l, in);
    if constexpr (SQ) {
        tile_compute<kMaxQkv>(R.qr, nq, S, kMaxTiles);
        __syncthreads();
        if (w == 0) qkv_epilogue(p, l, pos, tag, qkv_tiles, nq, kMaxTiles, false, S);
        RK_TRACE(true, kTrQkvPublished);
        __syncthreads();  // wave 0's q / k / v stores are in the queue before this layer's down columns
    }
    down_issue(p, l, sb, se, R.dr);
    tile_compute<kMaxTiles>(R.tr, nt, S, 0);
    __syncthreads();
    RK_TRACE(true, kTrTilesDone);
    if (w == 0) act_epilogue(nt, S);
    __syncthreads();
    RK_TRACE(true, kTrActReady);
    down_publish(p, l, tag, si, sb, se, R.dr, S);
    RK_TRACE(true, kTrDownPublished);
    if constexpr (!LAST) {
        if constexpr (SQ) tile_issue<kMaxQkv>(p, l + 1, qkv_tiles, nq, R.qr);
        tile_issue<kMaxTiles>(p, l + 1, mlp_tiles, nt, R.tr);
    } else {
        head_issue(p, si, R.hr);
    }
}

template <bool SQ>
RK_DEV void stream_run(const Params& p, Lds& S, uint32_t step, int64_t pos, int64_t tok, int si, int sb, int se) {
    StreamRegs R;
    const int t0 = (int)(n_tiles(p) - (size_t)p.inter / 8) + 2 * sb;
    const int q0 = qkv_first(p, si);
    if constexpr (SQ) tile_issue<kMaxQkv>(p, 0, [&](int t) { return q0 + t; }, qkv_first(p, si + 1) - q0, R.qr);
    tile_issue<kMaxTiles>(p, 0, [&](int t) { return t0 + t; }, 2 * (se - sb), R.tr);
    for (int l = 0; l + 1 < p.L; ++l) stream_layer<SQ, false>(p, S, step, pos, tok, si, sb, se, l, R);
    stream_layer<SQ, true>(p, S, step, pos, tok, si, sb, se, p.L - 1, R);
    final_phase(p, S, step, pos, si, R.hr);
}

template <int REP>
__global__ __launch_bounds__(kThreads) void decode_roles_kernel(Params p) {
    extern __shared__ __align__(16) uint8_t smem_raw[];
    Lds& S = *reinterpret_cast<Lds*>(smem_raw);
    const int t = threadIdx.x;
    const int64_t pos = p.pos[0];
    const int64_t tok = p.tok[0];
    if (pos < 0 || pos >= p.S) {  // no cache slot for this position: every block leaves at once
        if (blockIdx.x == 0 && t == 0) atomicOr(p.status, kBadPos);
        return;
    }
    const uint32_t step = p.ctr[blockIdx.x];
    const int16_t* role = p.role + 4 * blockIdx.x;
    const int kind = role[0], idx = role[1], sb = role[2], se = role[3];
    if (t < kHD / 2) {  // the table holds each angle twice (pair elements 2i, 2i + 1)
        S.rcos[t] = h16(p.cos_t[(size_t)pos * kHD + 2 * t]);
        S.rsin[t] = h16(p.sin_t[(size_t)pos * kHD + 2 * t]);
    }
#ifdef RK_ROLES_TRACE
    for (int i = t; i < 64 * kTrEvents; i += kThreads) (&S.trace[0][0])[i] = 0ull;
#endif
    if (t == 0) S.abort = 0u;
    __syncthreads();
    const bool sq = pos >= p.stream_qkv_from;  // the same in every block: the step's q/k/v placement
    if (kind == 0) {
        if (sq)
            latency_run<REP, true>(p, S, step, pos, tok, idx);
        else
            latency_run<REP, false>(p, S, step, pos, tok, idx);
    } else {
        if (sq)
            stream_run<true>(p, S, step, pos, tok, idx, sb, se);
        else
            stream_run<false>(p, S, step, pos, tok, idx, sb, se);
    }
#ifdef RK_ROLES_TRACE
    __syncthreads();
    if (g_roles_trace)
        for (int i = t; i < 64 * kTrEvents; i += kThreads)
            g_roles_trace[(size_t)blockIdx.x * 64 * kTrEvents + i] = (&S.trace[0][0])[i];
#endif
    if (t == 0) p.ctr[blockIdx.x] = step + 1;
}

// can kNB blocks of the kernel be resident on the current device at the same time?
bool co_resident(int rep) {
    constexpr int kMaxDev = 64;
    static int cached[kMaxDev][2];  // resident blocks per device and rep (0: not yet asked)
    const int ri = rep == 2 ? 0 : 1;
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    if (dev >= 0 && dev < kMaxDev && cached[dev][ri] > 0) return kNB <= cached[dev][ri];
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
    const void* fn = rep == 2 ? (const void*)decode_roles_kernel<2> : (const void*)decode_roles_kernel<4>;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fn, kThreads, sizeof(Lds)) != hipSuccess) return false;
    if (dev >= 0 && dev < kMaxDev) cached[dev][ri] = per_cu * cus;
    return kNB <= per_cu * cus;
}

}  // namespace

extern "C" int rk_decode_step_roles(const rk_decode_roles_params* params, rk_stream_t stream) {
    if (!params) return RK_ERR_NULL;
    const Params& p = *params;
    if (p.L <= 0 || p.L > 64 || p.NH * kHD != kH || p.NKV <= 0 || p.NH % p.NKV || p.S <= 0) return RK_ERR_SHAPE;
    const int rep = p.NH / p.NKV;
    if (!(rep == 2 || rep == 4)) return RK_ERR_SHAPE;  // NKV 8 or 4: 64 / NKV latency blocks per KV head
    if (p.inter <= 0 || p.inter % 128 || (p.inter / 16 + kNS - 1) / kNS > kMaxSlices) return RK_ERR_SHAPE;
    if (((p.NH + 2 * p.NKV) * kHD / 16) % kNL) return RK_ERR_SHAPE;                // latency q/k/v: spread evenly
    if ((p.NH + 2 * p.NKV) * (kHD / 16) > kMaxQkv * kNS) return RK_ERR_SHAPE;  // stream q/k/v tiles per block
    if (p.n_audio <= 0 || p.n_audio > kNS * kWaves * 64) return RK_ERR_SHAPE;  // <= 64 head rows per wave
    if (p.nsp <= 0 || p.nsp > kNL / p.NKV || p.nsp > kMaxSplits || p.min_chunk <= 0 || p.min_chunk % 8 ||
        (p.S + p.nsp - 1) / p.nsp > kWaves * kSlotsPerWave)  // every slot of a split is in some wave's registers
        return RK_ERR_BLOCK;
    if (!p.tok || !p.pos || !p.emb_q || !p.emb_s || !p.win_t || !p.win_sm || !p.wo_q || !p.wo_sm || !p.wd_t ||
        !p.wd_sm || !p.ln_w || !p.norm_w || !p.cos_t || !p.sin_t || !p.kc || !p.vc || !p.head_q || !p.head_s ||
        !p.logits || !p.role || !p.tx || !p.tq || !p.tkv || !p.top || !p.tdp || !p.tpo || !p.tml || !p.ctr ||
        !p.status)
        return RK_ERR_NULL;
    if (!co_resident(rep)) return RK_ERR_BLOCK;  // the waits need every block resident at once
    hipStream_t st = (hipStream_t)stream;
    if (rep == 2)
        hipLaunchKernelGGL(decode_roles_kernel<2>, dim3(kNB), dim3(kThreads), sizeof(Lds), st, p);
    else
        hipLaunchKernelGGL(decode_roles_kernel<4>, dim3(kNB), dim3(kThreads), sizeof(Lds), st, p);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

namespace {
__global__ __launch_bounds__(kThreads) void placement_kernel(int32_t* xcc) {
    if (threadIdx.x == 0) xcc[blockIdx.x] = (int32_t)__builtin_amdgcn_s_getreg(20 | (0 << 6) | (3 << 11));
}
}  // namespace

extern "C" int rk_decode_roles_placement(int32_t* xcc, rk_stream_t stream) {
    if (!xcc) return RK_ERR_NULL;
    hipLaunchKernelGGL(placement_kernel, dim3(kNB), dim3(kThreads), 0, (hipStream_t)stream, xcc);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_decode_roles_params_size(void) { return (int)sizeof(Params); }

extern "C" int rk_decode_roles_get_limits(rk_decode_roles_limits* out) {
    if (!out) return RK_ERR_NULL;
    out->blocks = kNB;
    out->latency_blocks = kNL;
    out->max_slices = kMaxSlices;
    out->x_copies = kXRep;
    out->max_splits = kMaxSplits;
    out->slots_per_wave = kSlotsPerWave;
    out->waves = kWaves;
    return RK_OK;
}

#ifdef RK_ROLES_TRACE
// trace builds only: the stamp buffer ([256][64][kTrEvents] uint64, or NULL) and the event count
extern "C" __attribute__((visibility("default"))) int rk_roles_trace_set(unsigned long long* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_roles_trace), &buf, sizeof(buf)) == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
extern "C" __attribute__((visibility("default"))) int rk_roles_trace_events(void) { return kTrEvents; }
#endif
