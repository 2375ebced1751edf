// One decoder layer's four decode projections in one launch (the benchmark's config 1 workload): the input
// projection w_in = [q | k | v | gate | up] over x with act = silu(gate) * up, the o projection over a given
// attention output, and the down projection over act. The reference runs them as separate calls with the SiLU in
// between (engine/rumik_fused.py:100-101 and 115-116: gemv(h, w_in), the MLP part of fused.post, gemv(ob, w_o),
// gemv(act, w_down)); all are int4 g128 GEMVs, y[n] = sum_g scale[n,g] * dot(codes, x)_g + min[n,g] * sum(x)_g
// (kernels/int4_gemv.py:1-4).
//
// Why one launch: the two-launch form (w_in with the SiLU fused, then o + down) pays two ramps and drains of the
// memory stream; one grid streams all ~41.6 MB back to back. down needs all of act, which every block produces a
// slice of, so the grid meets once, in the middle:
//   * one block of 8 waves per CU (its LDS request keeps a second block off the CU); every wait is bounded;
//   * block b owns gate / up pairs [b*pb, b*pb + pb), q/k/v rows [b*qb, ...), o rows [b*ob, ...) and down rows
//     [b*db, ...). K = 2048 is one 16-byte code chunk (32 columns) per lane, so a wave reads a row with one load;
//     x and the attention output are read once per block and shared through LDS in dot order;
//   * two wave roles with streams of about equal length: the down waves (2..7) take up to 6 gate / up pair slots
//     and then the 8 down rows' chunk 64 (w - 2) + lane (thread-per-chunk), the q/o waves (0, 1) 6 pair slots and
//     then the q/k/v and o rows. The q/o waves, whose streams are the longest, are the oldest: a CU issues its
//     waves' memory requests oldest first, so they no longer trail the others and the down waves' act read, which
//     queues behind every load the CU has in flight, starts sooner. Each wave keeps kAhead load units in flight and
//     computes a row as soon as it lands;
//   * act values are published as tagged 32-bit words (value bits | launch tag << 16) with agent-scope stores, so a
//     reader on any XCD takes a word only once it carries this launch's tag: no fences. A per-block flag (also the
//     tag) follows the words; the tag comes from a per-block launch counter in the workspace that the block
//     advances at its end, so graph replays need no reset;
//   * the down codes are dequantized to fp16 pairs as they land; then each down-wave lane reads its act chunk's 32
//     words (waiting on the flags only if some are not there yet), computes its chunk of the 8 down rows
//     (v_dot2, fp32 accumulation, the group affine per chunk), and the rows are reduced over the wave in
//     registers and over the 6 waves through LDS.
#include "internal.h"
#include "dequant.h"

#include <type_traits>

namespace {

constexpr int kWaves = 8;
constexpr int kThreads = 64 * kWaves;
constexpr int kH = 2048;            // hidden size: one 32-column chunk per lane in phase 1
constexpr int kDownWaves = 6;       // waves 2..7: gate / up and down; waves 0, 1: gate / up, q/k/v and o
constexpr int kQoWaves = kWaves - kDownWaves;
constexpr int kPairRot = 3;         // pair slot owner index of wave w: (w + 3) % 8
constexpr int kPairSlots = 6;       // gate / up pair slots per wave: local pairs w + 8s
constexpr int kPlainSlots = 6;      // q/k/v rows per q/o wave
constexpr int kOSlots = 4;          // o rows per q/o wave
constexpr int kDownRows = 8;        // down rows per block
constexpr int kAhead = 6;           // load units a wave keeps in flight
constexpr int kMaxInter = 64 * kDownWaves * 32;  // one down chunk per down-wave lane
constexpr int kMaxPairs = kWaves * kPairSlots;   // 48 gate / up pairs per block
constexpr size_t kLdsBytes = 82 * 1024;  // more than half of the CU's 160 KB: one block per CU
constexpr uint64_t kWaitTicks = 20000000ull;  // 200 ms at the 100 MHz wall clock
constexpr uint32_t kTimeout = 1u;      // status bit: an act poll ran out of time
constexpr int kMaxBlocks = 256;    // one block per CU, at most 256 (MI355X has 256 CUs)
constexpr int kCtrWords = kMaxBlocks;  // per-block launch counters and flags
constexpr int kHdrWords = 64;       // status word and padding


struct LayerArgs {
    const void* x;   // w_in's input [H]
    const void* ob;  // o's input [H]
    int xdt;
    const uint8_t* q_in;  // w_in [n_plain + 2 * inter, H]
    const uint16_t* s_in;
    const uint16_t* m_in;
    const uint8_t* q_o;  // w_o [H, H]
    const uint16_t* s_o;
    const uint16_t* m_o;
    const uint8_t* q_d;  // w_down [H, inter]
    const uint16_t* s_d;
    const uint16_t* m_d;
    void* y_plain;  // [n_plain]
    void* act;      // [inter]
    void* y_o;      // [H]
    void* y_down;   // [H]
    int ydt;
    int n_plain, inter;
    int pb, qb, obr, db;  // gate / up pairs, q/k/v rows, o rows, down rows per block
    uint32_t* ws;  // [0] status, [kHdrWords, +kCtrWords) launch counters, [.., +kCtrWords) flags, inter act words
};

RK_DEV void st_coh(uint32_t* p, uint32_t v) { __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
RK_DEV uint32_t ld_coh(const uint32_t* p) {
    return __hip_atomic_load(const_cast<uint32_t*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// the value an output of dtype dt (RK_F16 / RK_BF16) holds for v, and its bits
RK_DEV uint16_t bits_as(int dt, float v) { return dt == RK_F16 ? f32_to_f16_bits(v) : f32_to_bf16_bits(v); }
RK_DEV float from_bits(int dt, uint16_t b) { return dt == RK_F16 ? f16_bits_to_f32(b) : bf16_bits_to_f32(b); }

// A build option (RK_LAYER_TRACE; off in the product library, where RK_LTR is empty): wall-clock stamps per (block,
// wave, event) in registers, stored at the end of the launch to the buffer rk_layer_trace_set names
// ([block][8 waves][8 events] uint64, 100 MHz ticks); rumik-fast_amd/layer_trace.py builds and reads it.
#ifdef RK_LAYER_TRACE
__device__ unsigned long long* g_layer_trace;
#define RK_LTR(i) (T_[i] = wall_clock64())
#else
#define RK_LTR(i) ((void)0)
#endif

// A barrier for LDS traffic only: waits for this wave's LDS operations but not for its outstanding global loads
// (which __syncthreads would), and keeps the compiler from moving memory accesses across it.
RK_DEV void lds_barrier() {
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    asm volatile("s_barrier" ::: "memory");
}

// f(integral_constant<int, i>) for i in [B, E), each i a compile-time constant
template <int B, int E, class F>
RK_DEV void static_for(F&& f) {
    if constexpr (B < E) {
        f(std::integral_constant<int, B>{});
        static_for<B + 1, E>(f);
    }
}

// 16 dot-ordered pairs and their sum, from an LDS row written by process_x_chunk's caller
RK_DEV void load_pairs(const uint32_t* src, uint32_t (&p)[16], float& s) {
    const u4_t* v = reinterpret_cast<const u4_t*>(src);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const u4_t t = v[i];
        p[4 * i] = t.x;
        p[4 * i + 1] = t.y;
        p[4 * i + 2] = t.z;
        p[4 * i + 3] = t.w;
    }
    s = __builtin_bit_cast(float, src[16]);
}

// row `row`'s code chunk `lane`; when !ok, a line of `spare` (a cached 4 KB vector) instead
RK_DEV u4_t issue_row(const uint8_t* q, int row, bool ok, const void* spare, int lane) {
    const u4_t* wp = ok ? reinterpret_cast<const u4_t*>(q + (size_t)row * (kH / 2)) + lane
                        : reinterpret_cast<const u4_t*>(spare) + lane;
    return __builtin_nontemporal_load(wp);
}

// one row's share of this lane from its codes and its group's packed scale | min << 16
RK_DEV float row_part_sm(u4_t w, uint32_t sm, const uint32_t (&xp)[16], float xs, const Int4Masks& km) {
    const h2_t v = as_h2(sm);
    return __builtin_fmaf(chunk_dot_int4(w, xp, km), (float)v.x, (float)v.y * xs);
}

// The block's scales and mins, packed per group as scale | min << 16 in LDS: gate rows, up rows, q/k/v rows and o
// rows (16 groups each, K = 2048), then the down rows (inter / 128 groups each). Regions in groups.
constexpr int kTabG = 0;
constexpr int kTabU = kTabG + kWaves * kPairSlots * 16;
constexpr int kTabQ = kTabU + kWaves * kPairSlots * 16;
constexpr int kTabO = kTabQ + 2 * kPlainSlots * 16;
constexpr int kTabD = kTabO + 2 * kOSlots * 16;
constexpr int kTabWords = kTabD + kDownRows * (kMaxInter / 128);
constexpr int kTabIter = (kTabWords / 2 + kThreads - 1) / kThreads;  // group pairs per thread

__global__ __launch_bounds__(kThreads) void gemv_layer_kernel(LayerArgs a) {
    __shared__ uint32_t wave_bad[kWaves];          // a down wave whose wait ran out
    __shared__ uint32_t pub[kWaves * kPairSlots];  // this block's act values (bits), by local channel
    __shared__ float red[kDownWaves][kDownRows];   // down partial sums per wave
    __shared__ __align__(16) uint32_t xq[2][64][20];  // x, then the attention output: chunk pairs + sum
    __shared__ uint32_t tab[kTabWords];                // the block's scales | mins, by region
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int b = blockIdx.x;
#ifdef RK_LAYER_TRACE
    uint64_t T_[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#endif
    RK_LTR(0);
    const int nch2 = a.inter >> 5;  // down's 32-column chunks
    const int ng2 = a.inter >> 7;
    uint32_t* status = a.ws;
    uint32_t* ctr = a.ws + kHdrWords;
    uint32_t* flags = a.ws + kHdrWords + kCtrWords;  // per-block "act slice published" flags (the tag)
    uint32_t* xw = a.ws + kHdrWords + 2 * kCtrWords;  // tagged act words, channel 32c + i at i * nch2 + c
    const int p0 = b * a.pb, q0 = b * a.qb, o0 = b * a.obr, d0 = b * a.db;
    const int dw = wave - kQoWaves;         // down waves: 0 .. 5
    const int dchunk = 64 * dw + lane;      // down waves: this lane's down chunk (valid below nch2)

    // x and the attention output are read once per block (wave 0; lane = chunk) and shared through LDS in dot order:
    // a CU serves its waves' memory requests in issue order, so they go out before any weight request of the block
    XChunk xc, oc;
    if (wave == 0) {
        load_x_raw(a.x, lane, xc);
        load_x_raw(a.ob, lane, oc);
    }
    // the block's scale / min rows are contiguous per region: copied as dwords (two groups each)
    const int npb = max(0, min(a.pb, a.inter - p0)), nq = max(0, min(a.qb, a.n_plain - q0));
    const int no = max(0, min(a.obr, kH - o0)), nd = max(0, min(a.db, kH - d0));
    const int cG = npb * 8, cU = cG + npb * 8, cQ = cU + nq * 8, cO = cQ + no * 8, cD = cO + nd * ng2 / 2;
    uint32_t ts[kTabIter], tm[kTabIter];
    int tdst[kTabIter];
#pragma unroll
    for (int it = 0; it < kTabIter; ++it) {
        const int i = threadIdx.x + it * kThreads;  // group pair
        const uint32_t* sp = reinterpret_cast<const uint32_t*>(a.x);  // spare (cached) for pairs past the tables
        const uint32_t* mp = sp;
        int dst = -1;
        if (i < cG) {
            sp = reinterpret_cast<const uint32_t*>(a.s_in + (size_t)(a.n_plain + p0) * 16) + i;
            mp = reinterpret_cast<const uint32_t*>(a.m_in + (size_t)(a.n_plain + p0) * 16) + i;
            dst = kTabG + 2 * i;
        } else if (i < cU) {
            sp = reinterpret_cast<const uint32_t*>(a.s_in + (size_t)(a.n_plain + a.inter + p0) * 16) + (i - cG);
            mp = reinterpret_cast<const uint32_t*>(a.m_in + (size_t)(a.n_plain + a.inter + p0) * 16) + (i - cG);
            dst = kTabU + 2 * (i - cG);
        } else if (i < cQ) {
            sp = reinterpret_cast<const uint32_t*>(a.s_in + (size_t)q0 * 16) + (i - cU);
            mp = reinterpret_cast<const uint32_t*>(a.m_in + (size_t)q0 * 16) + (i - cU);
            dst = kTabQ + 2 * (i - cU);
        } else if (i < cO) {
            sp = reinterpret_cast<const uint32_t*>(a.s_o + (size_t)o0 * 16) + (i - cQ);
            mp = reinterpret_cast<const uint32_t*>(a.m_o + (size_t)o0 * 16) + (i - cQ);
            dst = kTabO + 2 * (i - cQ);
        } else if (i < cD) {
            sp = reinterpret_cast<const uint32_t*>(a.s_d + (size_t)d0 * ng2) + (i - cO);
            mp = reinterpret_cast<const uint32_t*>(a.m_d + (size_t)d0 * ng2) + (i - cO);
            dst = kTabD + 2 * (i - cO);
        }
        ts[it] = *sp;
        tm[it] = *mp;
        tdst[it] = dst;
    }
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);

    const Int4Masks km = int4_masks();
    uint32_t step = 0, tag = 0;
    h2_t dq[kDownRows][16];  // down waves: chunk dchunk of the block's down rows, as fp16 pairs

    // ---- phase 1. Two wave roles with streams of about equal length, in the order they are consumed:
    //   down waves (2..7):  up to 6 gate / up pair slots (gate, then up), then the 8 down rows' chunk of each lane;
    //   q/o waves (0, 1):   6 gate / up pair slots, then 6 q/k/v rows and 4 o rows.
    // kAhead units stay in flight: a wave computes a row as soon as it lands and issues the unit kAhead places
    // further on, so the rows are computed while the rest streams. Units past the block's share load a line of x
    // instead (cached; the result is dropped).
    auto phase1 = [&](auto down_c) __attribute__((always_inline)) {
        constexpr bool kDown = decltype(down_c)::value;
        constexpr int kP = kPairSlots;  // pair slots
        constexpr int kGU = 2 * kP;
        constexpr int kUnits = kGU + (kDown ? kDownRows : kPlainSlots + kOSlots);
        u4_t rl[kDown ? kGU : kGU + kPlainSlots + kOSlots];
        u4_t wd[kDownRows];
        const int qw = wave;  // q/o waves: 0, 1
        // local pair index of slot s: o + 8s with the wave's owner index o = (w + 3) % 8 (the block's waves read 8
        // consecutive rows per slot). A block's pairs (43 at inter = 11008) leave slot 5 to owners 0..2 only; the
        // rotation gives those extra pairs to down waves 5..7, so the q/o waves, whose streams are the longest, carry
        // five pairs
        auto pair_of = [&](int s) { return (wave + kPairRot) % kWaves + kWaves * s; };
        auto issue = [&](auto kc) __attribute__((always_inline)) {  // unit number as a compile-time constant
            constexpr int k = decltype(kc)::value;
            if constexpr (k >= kUnits) {
            } else if constexpr (k < kGU) {
                const int pl = pair_of(k >> 1);
                const bool ok = pl < a.pb && p0 + pl < a.inter;
                rl[k] = issue_row(a.q_in, a.n_plain + (k & 1) * a.inter + p0 + pl, ok, a.x, lane);
            } else if constexpr (kDown) {
                constexpr int r = k - kGU;
                const bool ok = r < a.db && d0 + r < kH && dchunk < nch2;
                const size_t row = ok ? (size_t)(d0 + r) : 0;
                const u4_t* wp = ok ? reinterpret_cast<const u4_t*>(a.q_d + row * (a.inter >> 1)) + dchunk
                                    : reinterpret_cast<const u4_t*>(a.x) + lane;
                wd[r] = __builtin_nontemporal_load(wp);
            } else if constexpr (k < kGU + kPlainSlots) {
                const int ql = qw + 2 * (k - kGU);
                const bool ok = ql < a.qb && q0 + ql < a.n_plain;
                rl[k] = issue_row(a.q_in, q0 + ql, ok, a.x, lane);
            } else {
                const int ol = qw + 2 * (k - kGU - kPlainSlots);
                const bool ok = ol < a.obr && o0 + ol < kH;
                rl[k] = issue_row(a.q_o, o0 + ol, ok, a.x, lane);
            }
        };
        static_for<0, kAhead>([&](auto kc) __attribute__((always_inline)) { issue(kc); });
        // this block's launch count (the tag of this launch's act words), behind the first rows; a VGPR load, so
        // nothing waits for it until it is used
        step = ld_coh(ctr + b + opaque_vgpr(0u));
        tag = 1u + step % 65535u;

        if (wave == 0) {
            uint32_t p[16];
            float ps;
            process_x_chunk(xc, a.xdt, p, ps);
            u4_t* dst = reinterpret_cast<u4_t*>(xq[0][lane]);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = u4_t{p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]};
            xq[0][lane][16] = __builtin_bit_cast(uint32_t, ps);
            process_x_chunk(oc, a.xdt, p, ps);
            dst = reinterpret_cast<u4_t*>(xq[1][lane]);
#pragma unroll
            for (int i = 0; i < 4; ++i) dst[i] = u4_t{p[4 * i], p[4 * i + 1], p[4 * i + 2], p[4 * i + 3]};
            xq[1][lane][16] = __builtin_bit_cast(uint32_t, ps);
        }
#pragma unroll
        for (int it = 0; it < kTabIter; ++it)
            if (tdst[it] >= 0) {
                tab[tdst[it]] = (ts[it] & 0xFFFFu) | (tm[it] << 16);
                tab[tdst[it] + 1] = (ts[it] >> 16) | (tm[it] & 0xFFFF0000u);
            }
        lds_barrier();
        uint32_t xp[16];
        float xs;
        load_pairs(xq[0][lane], xp, xs);
        RK_LTR(1);

        // gate / up: slot s of each in vg[s] / vu[s]; after the reductions lanes 8s..8s+7 hold slot s of both
        {
            float vg[8], vu[8];
#pragma unroll
            for (int s = 0; s < 8; ++s) vg[s] = vu[s] = 0.f;
            static_for<0, kGU>([&](auto kc) __attribute__((always_inline)) {
                constexpr int k = decltype(kc)::value;
                const int pl = min(pair_of(k >> 1), kWaves * kPairSlots - 1);
                const uint32_t sm = tab[((k & 1) ? kTabU : kTabG) + pl * 16 + (lane >> 2)];
                const float r = row_part_sm(rl[k], sm, xp, xs, km);
                if constexpr (k & 1) vu[k >> 1] = r; else vg[k >> 1] = r;
                issue(std::integral_constant<int, k + kAhead>{});
            });
            wave_reduce_rows<8>(vg);
            wave_reduce_rows<8>(vu);
            const int s = lane >> 3;
            const int pl = pair_of(s);
            if (s < kP && (lane & 7) == 0 && pl < a.pb && p0 + pl < a.inter) {
                const float gr = from_bits(a.ydt, bits_as(a.ydt, vg[0]));
                const float ur = from_bits(a.ydt, bits_as(a.ydt, vu[0]));
                pub[pl] = bits_as(a.ydt, gr / (1.0f + __expf(-gr)) * ur);
            }
        }
        // the last q/o wave publishes the block's act slice and then the block's flag (one store stream: the flag
        // usually lands after the words; readers check the words' tags in any case)
        lds_barrier();
        if (wave == kQoWaves - 1) {
            const int np = min(a.pb, a.inter - p0);
            for (int l = lane; l < np; l += 64) {
                const int c = p0 + l;
                const uint32_t hb = pub[l];
                reinterpret_cast<uint16_t*>(a.act)[c] = (uint16_t)hb;
                st_coh(xw + (size_t)(c & 31) * nch2 + (c >> 5), hb | (tag << 16));
            }
            if (lane == 0) st_coh(flags + b, tag);
        }
        RK_LTR(2);

        if constexpr (kDown) {
            // the down chunks to fp16 pairs, kept for phase 2
            static_for<kGU, kUnits>([&](auto kc) __attribute__((always_inline)) {
                constexpr int r = decltype(kc)::value - kGU;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    h2_t p[4];
                    dequant_pairs(wd[r][i], km, p);
#pragma unroll
                    for (int e = 0; e < 4; ++e) dq[r][4 * i + e] = p[e];
                }
                issue(std::integral_constant<int, decltype(kc)::value + kAhead>{});
            });
        } else {
            // q/k/v rows in slots 0..5, o rows in 8..11; after the reduction lanes 4s..4s+3 hold slot s
            uint32_t op[16];
            float os;
            load_pairs(xq[1][lane], op, os);
            float v[16];
#pragma unroll
            for (int s = 0; s < 16; ++s) v[s] = 0.f;
            static_for<kGU, kUnits>([&](auto kc) __attribute__((always_inline)) {
                constexpr int k = decltype(kc)::value;
                if constexpr (k < kGU + kPlainSlots) {
                    const int ql = qw + 2 * (k - kGU);
                    v[k - kGU] = row_part_sm(rl[k], tab[kTabQ + ql * 16 + (lane >> 2)], xp, xs, km);
                } else {
                    const int ol = qw + 2 * (k - kGU - kPlainSlots);
                    v[8 + k - kGU - kPlainSlots] = row_part_sm(rl[k], tab[kTabO + ol * 16 + (lane >> 2)], op, os, km);
                }
                issue(std::integral_constant<int, k + kAhead>{});
            });
            wave_reduce_rows<16>(v);
            const int s = lane >> 2;
            if ((lane & 3) == 0) {
                if (s < kPlainSlots) {
                    const int ql = qw + 2 * s;
                    if (ql < a.qb && q0 + ql < a.n_plain) store_act(a.y_plain, a.ydt, (size_t)(q0 + ql), v[0]);
                } else if (s >= 8 && s < 8 + kOSlots) {
                    const int ol = qw + 2 * (s - 8);
                    if (ol < a.obr && o0 + ol < kH) store_act(a.y_o, a.ydt, (size_t)(o0 + ol), v[0]);
                }
            }
        }
    };
    if (wave >= kQoWaves) phase1(std::true_type{});
    else phase1(std::false_type{});
    RK_LTR(3);

    // ---- phase 2 on the down waves, while the q/o waves finish their streams: take act chunk t (32 tagged words,
    // one per channel) into registers in dot order, and compute chunk t of the block's down rows (v_dot2, fp32
    // accumulation, the group affine); rows are reduced over the wave, then over the waves. By the time a down wave
    // gets here most blocks have published, so the words are read at once; if some are not there yet the wave
    // waits on the blocks' flags (nb words per poll: the blocks still streaming are not slowed by the waiting ones)
    // before it reads the words again.
    if (wave >= kQoWaves && 64 * dw < nch2) {
        bool bad = false;
        const uint64_t t0 = wall_clock64();
        const int nb = gridDim.x;
        const bool mine = dchunk < nch2;
        const int cc = min(dchunk, nch2 - 1);
        uint32_t wv[32];
        RK_LTR(4);
        while (true) {
#pragma unroll
            for (int i = 0; i < 32; ++i) wv[i] = ld_coh(xw + (size_t)i * nch2 + cc);
            bool have = true;
#pragma unroll
            for (int i = 0; i < 32; ++i) have = have && (wv[i] >> 16) == tag;
            if (__all(have || !mine)) break;
            while (true) {  // not all there: wait for every flag, then read again
                uint32_t f[kMaxBlocks / 64];
#pragma unroll
                for (int k = 0; k < kMaxBlocks / 64; ++k) f[k] = ld_coh(flags + min(k * 64 + lane, nb - 1));
                bool all = true;
#pragma unroll
                for (int k = 0; k < kMaxBlocks / 64; ++k) all = all && f[k] == tag;
                if (__all(all)) break;
                if (wall_clock64() - t0 > kWaitTicks) break;
                __builtin_amdgcn_s_sleep(2);
            }
            if (wall_clock64() - t0 > kWaitTicks) {  // a block never arrived: record it, compute no down row
                if (lane == 0) atomicOr(status, kTimeout);
                bad = true;
                break;
            }
        }
        RK_LTR(5);
        if (!bad) {
            XChunk ac;
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    ac.d[i][e] = (wv[8 * i + 2 * e] & 0xFFFFu) | (wv[8 * i + 2 * e + 1] << 16);
            uint32_t ap[16];
            float as;
            process_x_chunk(ac, a.ydt, ap, as);
            float acc[kDownRows];
#pragma unroll
            for (int r = 0; r < kDownRows; ++r) {
                float a0 = 0.f, a1 = 0.f;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    a0 = dot2(dq[r][4 * i + 0], as_h2(ap[4 * i + 0]), a0);
                    a1 = dot2(dq[r][4 * i + 1], as_h2(ap[4 * i + 1]), a1);
                    a0 = dot2(dq[r][4 * i + 2], as_h2(ap[4 * i + 2]), a0);
                    a1 = dot2(dq[r][4 * i + 3], as_h2(ap[4 * i + 3]), a1);
                }
                const h2_t sm = as_h2(tab[kTabD + r * ng2 + (cc >> 2)]);
                const float v = __builtin_fmaf(a0 + a1, (float)sm.x, (float)sm.y * as);
                acc[r] = mine ? v : 0.f;
            }
            wave_reduce_rows<kDownRows>(acc);  // lanes 8r..8r+7 hold row r
            if ((lane & 7) == 0) red[dw][lane >> 3] = acc[0];
        }
        if (lane == 0) wave_bad[dw] = bad ? 1u : 0u;
        RK_LTR(6);
    }
    __syncthreads();
    if (wave == 0 && lane < kDownRows) {
        bool any_bad = false;
        float v = 0.f;
#pragma unroll
        for (int w = 0; w < kDownWaves; ++w)
            if (64 * w < nch2) {
                any_bad = any_bad || wave_bad[w] != 0u;
                v += red[w][lane];
            }
        const int row = d0 + lane;
        if (!any_bad && lane < a.db && row < kH) store_act(a.y_down, a.ydt, (size_t)row, v);
    }
    RK_LTR(7);
#ifdef RK_LAYER_TRACE
    if (g_layer_trace && lane == 0)
        for (int i = 0; i < 8; ++i) g_layer_trace[((size_t)b * kWaves + wave) * 8 + i] = T_[i];
#endif
    // the counter is kept reduced modulo 65535, so consecutive launches always carry different tags (a plain
    // uint32 counter would wrap from 2^32 - 1 to 0, and both values give tag 1)
    if (threadIdx.x == 0) st_coh(ctr + b, (step + 1u) % 65535u);
}

int layer_blocks() {
    constexpr int kMaxDev = 64;
    static int cached[kMaxDev];  // co-resident blocks per device (0: not yet asked)
    int dev = 0, cus = 0, per_cu = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 0;
    if (dev >= 0 && dev < kMaxDev && cached[dev] > 0) return cached[dev];
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gemv_layer_kernel, kThreads, kLdsBytes) != hipSuccess ||
        per_cu < 1)
        return 0;
    const int nb = min(cus, kMaxBlocks);  // one block per CU; the LDS request keeps a second one off
    if (dev >= 0 && dev < kMaxDev) cached[dev] = nb;
    return nb;
}

int cdiv(int a, int b) { return (a + b - 1) / b; }

}  // namespace

extern "C" size_t rk_gemv_int4_g128_layer_ws_bytes(int inter) {
    if (inter <= 0) return 0;
    return (size_t)(kHdrWords + 2 * kCtrWords + inter) * 4;
}

extern "C" int rk_gemv_int4_g128_layer(const void* x, const void* ob, int x_dtype, const uint8_t* q_in,
                                       const uint16_t* s_in, const uint16_t* m_in, const uint8_t* q_o,
                                       const uint16_t* s_o, const uint16_t* m_o, const uint8_t* q_down,
                                       const uint16_t* s_down, const uint16_t* m_down, void* y_plain, void* act,
                                       void* y_o, void* y_down, int y_dtype, int n_plain, int inter, int H,
                                       void* ws, size_t ws_bytes, rk_stream_t stream) {
    if (!x || !ob || !q_in || !s_in || !m_in || !q_o || !s_o || !m_o || !q_down || !s_down || !m_down || !act ||
        !y_o || !y_down || !ws || (n_plain > 0 && !y_plain))
        return RK_ERR_NULL;
    if (x_dtype != RK_F16 && x_dtype != RK_BF16) return RK_ERR_DTYPE;
    if (y_dtype != RK_F16 && y_dtype != RK_BF16) return RK_ERR_DTYPE;
    if (H != kH || n_plain < 0 || inter <= 0 || inter % 128 || inter > kMaxInter) return RK_ERR_SHAPE;
    if (ws_bytes < rk_gemv_int4_g128_layer_ws_bytes(inter)) return RK_ERR_SHAPE;
    if (((uintptr_t)x & 15) || ((uintptr_t)ob & 15) || ((uintptr_t)q_in & 15) || ((uintptr_t)q_o & 15) ||
        ((uintptr_t)q_down & 15) || ((uintptr_t)ws & 3) || ((uintptr_t)act & 1) || ((uintptr_t)s_in & 3) ||
        ((uintptr_t)m_in & 3) || ((uintptr_t)s_o & 3) || ((uintptr_t)m_o & 3) || ((uintptr_t)s_down & 3) ||
        ((uintptr_t)m_down & 3))
        return RK_ERR_ALIGN;
    const int nb = layer_blocks();
    if (nb <= 0 || nb > kMaxBlocks) return RK_ERR_BLOCK;
    LayerArgs a;
    a.x = x; a.ob = ob; a.xdt = x_dtype;
    a.q_in = q_in; a.s_in = s_in; a.m_in = m_in;
    a.q_o = q_o; a.s_o = s_o; a.m_o = m_o;
    a.q_d = q_down; a.s_d = s_down; a.m_d = m_down;
    a.y_plain = y_plain; a.act = act; a.y_o = y_o; a.y_down = y_down; a.ydt = y_dtype;
    a.n_plain = n_plain; a.inter = inter;
    a.pb = cdiv(inter, nb);
    a.qb = cdiv(n_plain, nb);
    a.obr = cdiv(H, nb);
    a.db = cdiv(H, nb);
    a.ws = reinterpret_cast<uint32_t*>(ws);
    // the per-wave slots: pairs (wave + 3) % 8 + 8s (s < 6); q/k/v and o rows on the two q/o waves; the down rows
    if (a.pb > kMaxPairs || a.qb > 2 * kPlainSlots || a.obr > 2 * kOSlots || a.db > kDownRows)
        return RK_ERR_SHAPE;
    hipLaunchKernelGGL(gemv_layer_kernel, dim3(nb), dim3(kThreads), kLdsBytes, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

#ifdef RK_LAYER_TRACE
// trace builds only: the stamp buffer ([blocks][8][8] uint64, or NULL)
extern "C" __attribute__((visibility("default"))) int rk_layer_trace_set(unsigned long long* buf) {
    return hipMemcpyToSymbol(HIP_SYMBOL(g_layer_trace), &buf, sizeof(buf)) == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
#endif
