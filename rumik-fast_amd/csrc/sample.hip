// The tail of a decode step on gfx950: stop predictor + top-k + Gumbel-max sampling + token counters
// (reference engine/sample.py, whose three Triton kernels replace ~25 PyTorch kernels of
// RumikInt4._logits_and_stop / _pick, engine/rumik_int4.py:174-198).
//
//   stop   = sigmoid(w2 . gelu(W1 . LayerNorm(h) + b1) + b2) > 0.5  (<=> the stop logit > 0), only from min_new on
//   logits = the audio head's output; index end_idx (</audio>) is masked to -inf for the first min_new tokens
//   token  = ids[argmax over the top-k logits of (logit / T + Gumbel(u))]  == a sample from softmax(top-k / T)
//
// Top-k ordering (the reference's, sample.py:7-11): each logit and its index are one int64 key,
//   key = sortable(bits(x)) << 32 | index,  sortable(b) = b ^ ((b >> 31) & 0x7FFFFFFF)
// so key order is value order (monotonic also for -inf) with ties broken by the larger index; keys are unique.
// Stage 1: four waves per chunk of 512 logits sort the chunk with a bitonic network held in registers (2 keys per
// lane, element 2 t + i): partners at distance 1 stay inside a lane, at 2 .. 64 are one 64-bit shuffle away, and
// the three stages at distance 128 / 256 exchange through LDS between the waves. Stage 2: the chunks' top-32
// lists are merged pairwise in a tree, one wave per merge (a 32-key list and the other reversed form a bitonic
// sequence of 64, one key per lane; 6 shuffle stages keep the top 32 in order), 16 waves per level. An LDS bitonic
// sort of the whole chunk / candidate list (what the Triton code's tl.sort does) measured ~1 us per network stage
// here (98 us per call); a 64-step radix bisection over ballots 48 us; 32 rounds of a 64-bit wave maximum 34 us.
//
// Buffers: keys[512c .. 512c + 512) = chunk c sorted in key order (the reference's contents) and scratch[0 .. 32) =
// the global top 32 in key order, which is what the reference's pick and its sampler check read of the candidate
// list (sample.py:69-72, check_sample.py:44); the rest of scratch is not written.
//
// Entry points: the reference's three kernels one to one (rk_stop_hidden, rk_topk_partial, rk_pick), and
// rk_sample_tail, the same work in ONE launch: blocks [0, nzb) compute the stop predictor's hidden layer, the next
// blocks sort one chunk each (wave 0); every block then bumps a completion counter and the last block to arrive
// does the pick. The exchanged results (keys, z1) are stored and read at agent scope and each block's stores are
// acknowledged before its count goes up (a device-scope __threadfence per wave writes back L2 and measured 3x
// slower here). No block waits for another, so the grid needs no co-residency, and the last block resets the
// counter, so replays need no memset.
#include <algorithm>

#include "common.h"

namespace {

constexpr int kCH = 512;       // logits per chunk (reference CH)
constexpr int kKeep = 32;      // survivors per chunk (reference KEEP, >= top_k)
constexpr int kMaxNC = 4096;   // candidate slots of the pick (at most 128 chunks)
constexpr int kThreads = 1024;
constexpr int kWaves = kThreads / 64;
constexpr int kStopRows = kWaves;  // stop-predictor rows per block (one per wave)

RK_DEV int32_t sortable(float x) {
    const int32_t b = __builtin_bit_cast(int32_t, x);
    return b ^ ((b >> 31) & 0x7FFFFFFF);
}
RK_DEV float unsortable(int32_t k) { return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7FFFFFFF)); }
RK_DEV int64_t make_key(float x, int i) {
    return (int64_t)(((uint64_t)(uint32_t)sortable(x) << 32) | (uint64_t)(uint32_t)i);
}

constexpr int64_t kPad = -(int64_t(1) << 62);  // below every real key (the reference's padding value)

// Results another block of the same launch reads (rk_sample_tail) are stored and loaded at agent scope (coherent
// across the XCDs' L2s, no cache-wide fence needed): the writer waits for its stores' acknowledgements before the
// block's count goes up, and the last block reads them with agent-scope loads.
RK_DEV void st_agent(int64_t* p, int64_t v) {
    __hip_atomic_store(reinterpret_cast<uint64_t*>(p), (uint64_t)v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV int64_t ld_agent(const int64_t* p) {
    return (int64_t)__hip_atomic_load(reinterpret_cast<uint64_t*>(const_cast<int64_t*>(p)), __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV void st_agent(float* p, float v) {
    __hip_atomic_store(reinterpret_cast<uint32_t*>(p), __builtin_bit_cast(uint32_t, v), __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_AGENT);
}
RK_DEV float ld_agent(const float* p) {
    return __builtin_bit_cast(float, __hip_atomic_load(reinterpret_cast<uint32_t*>(const_cast<float*>(p)),
                                                       __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT));
}

// v of lane i ^ m (m a power of two below 64, a constant once the callers' loops are unrolled), both halves by
// VALU lane moves (no LDS round trip)
template <int M>
RK_DEV int64_t xor64(int64_t v) {
    const uint32_t lo = xor_lanes<M>((uint32_t)v), hi = xor_lanes<M>((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}
RK_DEV int64_t shfl_xor64(int64_t v, int m) {
    switch (m) {
        case 1: return xor64<1>(v);
        case 2: return xor64<2>(v);
        case 4: return xor64<4>(v);
        case 8: return xor64<8>(v);
        case 16: return xor64<16>(v);
        default: return xor64<32>(v);
    }
}

// Waves 0..3 of the block (one per SIMD) sort the 512 keys of chunk c descending and store them to out[0 .. 512):
// element e = 2 t + i of thread t < 256 (two keys per lane). Partners at distance 1 sit in the same lane, at 2 .. 64
// in another lane of the same wave (one 64-bit shuffle per key), at 128 and 256 in another wave (through xs, 512
// keys of LDS). Every thread of the block runs the loop and reaches its barriers (the other waves and a block
// without a chunk, `active` false, only pass them), so the block's barriers always pair up. (One wave with eight keys
// per lane measured ~7 us per chunk: the network's dependent compare / select / shuffle chain on one SIMD.)
RK_DEV void chunk_sort(const void* logits, int ldt, bool early, int nv, int end_idx, int c, bool active, int64_t* out,
                       int64_t* xs) {
    const int t = threadIdx.x;
    const bool on = active && t < 256;
    int64_t v[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int e = c * kCH + 2 * t + i;
        float x = on && e < nv ? load_act(logits, ldt, (size_t)e) : -INFINITY;
        if (early && e == end_idx) x = -INFINITY;  // no </audio> during the first min_new tokens
        v[i] = make_key(x, e);
    }
#pragma unroll
    for (int k = 2; k <= kCH; k <<= 1) {
        const bool desc = ((2 * t) & k) == 0;  // the direction of both of the lane's elements (k >= 2)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            if (j == 1) {
                const bool sw = desc ? v[0] < v[1] : v[0] > v[1];
                const int64_t a = v[0], b = v[1];
                v[0] = sw ? b : a;
                v[1] = sw ? a : b;
            } else if (j < 128) {  // partner lane t ^ (j / 2), same wave, same slot
                const int m = j >> 1;
                const bool keep_max = ((t & m) == 0) == desc;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int64_t o = shfl_xor64(v[i], m);
                    v[i] = keep_max ? (o > v[i] ? o : v[i]) : (o < v[i] ? o : v[i]);
                }
            } else {  // partner in another wave
                __syncthreads();  // the previous exchange's reads are done
                if (on) {
                    xs[2 * t] = v[0];
                    xs[2 * t + 1] = v[1];
                }
                __syncthreads();
                const bool keep_max = (((2 * t) & j) == 0) == desc;
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int64_t o = on ? xs[(2 * t + i) ^ j] : v[i];
                    v[i] = keep_max ? (o > v[i] ? o : v[i]) : (o < v[i] ? o : v[i]);
                }
            }
        }
    }
    if (on) {
        st_agent(out + 2 * t, v[0]);
        st_agent(out + 2 * t + 1, v[1]);
    }
}

// one wave: the top 32 of two descending 32-key lists a, b (LDS) into dst[0 .. 32) in order (dst may alias a)
RK_DEV void merge_top32(const int64_t* a, const int64_t* b, int64_t* dst) {
    const int lane = threadIdx.x & 63;
    int64_t x = lane < 32 ? a[lane] : b[63 - lane];  // descending then ascending: bitonic
#pragma unroll
    for (int j = 32; j > 0; j >>= 1) {
        const int64_t o = shfl_xor64(x, j);
        const bool lower = (lane & j) == 0;
        x = lower ? (o > x ? o : x) : (o < x ? o : x);
    }
    __builtin_amdgcn_wave_barrier();
    if (lane < 32) dst[lane] = x;
}

RK_DEV float block_sum(float v, float* red) {  // red: >= 4 floats of LDS; every thread gets the sum
    v = wave_sum(v);
    const int w = threadIdx.x >> 6, nw = blockDim.x >> 6;
    __syncthreads();
    if ((threadIdx.x & 63) == 0) red[w] = v;
    __syncthreads();
    float t = 0.f;
    for (int i = 0; i < nw; ++i) t += red[i];
    return t;
}

// ---- stop predictor, hidden layer (reference stop_hidden, sample.py:34-49): z1[r] = gelu(W1[r] . LN(h) + b1[r])
// for rows [r0, r0 + kStopRows); every block recomputes the (cheap) LayerNorm of h into LDS. One wave per row.
RK_DEV void stop_rows(const void* h, int hdt, const float* lnw, const float* lnb, const void* w1, int wdt,
                      const float* b1, float* z1, float eps, int H, int nz, int r0, float* z, float* red) {
    const int lane = threadIdx.x & 63, r = r0 + (threadIdx.x >> 6);
    // this wave's W1 row first (up to kRowRegs 16-byte pieces per lane), so its HBM latency overlaps the LayerNorm
    constexpr int kRowRegs = 8;  // H <= 8192 with 16-bit weights
    const bool vec = H % 512 == 0 && H <= 64 * 8 * kRowRegs && wdt != RK_F32;
    uint4 wv[kRowRegs];
    if (vec) {
        const uint4* wr = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w1) + (size_t)min(r, nz - 1) * H);
#pragma unroll
        for (int k = 0; k < kRowRegs; ++k) wv[k] = wr[min(lane + 64 * k, H / 8 - 1)];
    }
    float s = 0.f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const float v = load_act(h, hdt, (size_t)i);
        z[i] = v;
        s += v;
    }
    const float mean = block_sum(s, red) / (float)H;
    float ss = 0.f;
    for (int i = threadIdx.x; i < H; i += blockDim.x) {
        const float d = z[i] - mean;
        ss += d * d;
    }
    const float rstd = rsqrtf(block_sum(ss, red) / (float)H + eps);
    for (int i = threadIdx.x; i < H; i += blockDim.x) z[i] = (z[i] - mean) * rstd * lnw[i] + lnb[i];
    __syncthreads();
    if (r >= nz) return;
    float acc = 0.f;
    if (vec) {  // 8 weights (16 bytes) per lane per piece
#pragma unroll
        for (int k = 0; k < kRowRegs; ++k) {
            const int c = lane + 64 * k;
            if (c < H / 8) {
                const uint32_t d[4] = {wv[k].x, wv[k].y, wv[k].z, wv[k].w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float lo = wdt == RK_BF16 ? bf16_bits_to_f32((uint16_t)d[e]) : f16_bits_to_f32((uint16_t)d[e]);
                    const float hi = wdt == RK_BF16 ? bf16_bits_to_f32((uint16_t)(d[e] >> 16))
                                                    : f16_bits_to_f32((uint16_t)(d[e] >> 16));
                    acc = __builtin_fmaf(lo, z[8 * c + 2 * e], acc);
                    acc = __builtin_fmaf(hi, z[8 * c + 2 * e + 1], acc);
                }
            }
        }
    } else {
        for (int k = lane; k < H; k += 64) acc = __builtin_fmaf(load_act(w1, wdt, (size_t)r * H + k), z[k], acc);
    }
    acc = wave_sum(acc) + b1[r];
    if (lane == 0) st_agent(z1 + r, 0.5f * acc * (1.0f + erff(acc * 0.7071067811865476f)));  // exact GELU (F.gelu)
}

// ---- stage 1 (reference topk_partial, sample.py:53-61): block blk sorts chunk blk (waves 0..3; every thread of
// the block calls in, for the barriers)
RK_DEV void topk_chunks(const void* logits, int ldt, const int64_t* step, int64_t* keys, int nv, int end_idx,
                        int min_new, int blk) {
    __shared__ int64_t xs[kCH];
    const int c = blk;
    const bool early = step[0] < (int64_t)min_new;
    chunk_sort(logits, ldt, early, nv, end_idx, c, c * kCH < nv, keys + (size_t)c * kCH, xs);
}

// ---- stage 2 (reference pick, sample.py:65-93): the top 32 of the chunks' lists, sample, stop rule, counters.
// The block stages the lists (nch x 32 keys) and computes the stop logit; wave 0 selects and samples.
RK_DEV void pick_block(const int64_t* keys, int64_t* scratch, const float* u, const float* z1, const float* w2,
                       const float* b2, const int64_t* ids, int64_t* step_p, int64_t* tok, int64_t* out,
                       float inv_temp, int64_t end_id, int min_new, int nch, int topk, int nz, int64_t* cand,
                       float* red) {
    for (int c = threadIdx.x; c < nch * kKeep; c += blockDim.x)
        cand[c] = ld_agent(keys + (size_t)(c / kKeep) * kCH + c % kKeep);
    float part = 0.f;
    for (int r = threadIdx.x; r < nz; r += blockDim.x) part = __builtin_fmaf(ld_agent(z1 + r), w2[r], part);
    const float stop_logit = block_sum(part, red) + b2[0];  // sigmoid(.) > 0.5  <=>  stop_logit > 0
    __syncthreads();
    // merge tree over the lists (in place): level d merges list i and list i + 2^d for i a multiple of 2^(d+1)
    const int w = threadIdx.x >> 6;
    for (int d = 1; d < nch; d <<= 1) {
        for (int i = 2 * d * w; i < nch; i += 2 * d * kWaves)
            if (i + d < nch) merge_top32(cand + i * kKeep, cand + (i + d) * kKeep, cand + i * kKeep);
        __syncthreads();
    }
    if (threadIdx.x >= 64) return;
    const int lane = threadIdx.x;
    const int64_t top = lane < kKeep ? cand[lane] : kPad;
    if (lane < kKeep) scratch[lane] = top;
    const int j = lane;  // candidate rank (lanes 0..31 hold the top 32, best first)
    const int64_t t = __shfl(top, j & 31);
    const float val = unsortable((int32_t)(t >> 32));
    const int idx = (int)(uint32_t)(t & 0xFFFFFFFF);
    const float uu = j < topk ? u[j] : 0.5f;
    const float g = -logf(-logf(fminf(fmaxf(uu, 1e-10f), 1.0f)));
    const float score = j < topk ? val * inv_temp + g : -INFINITY;
    const float best = wave_max(score);
    const uint64_t hit = __ballot(score == best);  // the first (highest-ranked) candidate holding the maximum
    const int bj = hit ? __builtin_ctzll(hit) : 0;
    const int choice = __shfl(idx, bj);
    if (j == 0) {
        const int64_t step = step_p[0];
        int64_t nxt = ids[choice];
        if (stop_logit > 0.f && step >= (int64_t)min_new) nxt = end_id;
        out[step] = nxt;
        tok[0] = nxt;
        step_p[0] = step + 1;
    }
}

__global__ __launch_bounds__(kThreads) void stop_hidden_kernel(const void* h, int hdt, const float* lnw,
                                                               const float* lnb, const void* w1, int wdt,
                                                               const float* b1, float* z1, float eps, int H, int nz) {
    extern __shared__ __align__(16) float zsm[];
    __shared__ float red[16];
    stop_rows(h, hdt, lnw, lnb, w1, wdt, b1, z1, eps, H, nz, blockIdx.x * kStopRows, zsm, red);
}

__global__ __launch_bounds__(kThreads) void topk_partial_kernel(const void* logits, int ldt, const int64_t* step,
                                                                int64_t* keys, int nv, int end_idx, int min_new) {
    topk_chunks(logits, ldt, step, keys, nv, end_idx, min_new, blockIdx.x);
}

__global__ __launch_bounds__(kThreads) void pick_kernel(const int64_t* keys, int64_t* scratch, const float* u,
                                                        const float* z1, const float* w2, const float* b2,
                                                        const int64_t* ids, int64_t* step_p, int64_t* tok,
                                                        int64_t* out, float inv_temp, int64_t end_id, int min_new,
                                                        int nch, int topk, int nz) {
    extern __shared__ __align__(16) int64_t ssm[];
    __shared__ float red[16];
    pick_block(keys, scratch, u, z1, w2, b2, ids, step_p, tok, out, inv_temp, end_id, min_new, nch, topk, nz, ssm,
               red);
}

struct TailArgs {
    const void* h;
    const float *lnw, *lnb;
    const void* w1;
    const float *b1, *w2, *b2, *u;
    const void* logits;
    const int64_t* ids;
    int64_t *keys, *scratch, *step, *tok, *out;
    float* z1;
    unsigned* counter;
    float eps, inv_temp;
    int64_t end_id;
    int hdt, wdt, ldt, H, nz, nv, end_idx, min_new, nch, topk, nzb;
};

__global__ __launch_bounds__(kThreads) void sample_tail_kernel(TailArgs a) {
    extern __shared__ __align__(16) uint8_t raw[];
    __shared__ float red[16];
    __shared__ unsigned last;
    const int b = blockIdx.x;
    if (b < a.nzb)
        stop_rows(a.h, a.hdt, a.lnw, a.lnb, a.w1, a.wdt, a.b1, a.z1, a.eps, a.H, a.nz, b * kStopRows,
                  reinterpret_cast<float*>(raw), red);
    else
        topk_chunks(a.logits, a.ldt, a.step, a.keys, a.nv, a.end_idx, a.min_new, b - a.nzb);
    __builtin_amdgcn_s_waitcnt(0);  // this wave's agent-scope stores are acknowledged
    __syncthreads();                // ... and every other wave's of the block
    if (threadIdx.x == 0)
        last = __hip_atomic_fetch_add(a.counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    if (threadIdx.x == 0)  // ready for the next call (stream order)
        __hip_atomic_store(a.counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    pick_block(a.keys, a.scratch, a.u, a.z1, a.w2, a.b2, a.ids, a.step, a.tok, a.out, a.inv_temp, a.end_id,
               a.min_new, a.nch, a.topk, a.nz, reinterpret_cast<int64_t*>(raw), red);
}

bool pow2(int n) { return n > 0 && (n & (n - 1)) == 0; }

int check_pick(int nch, int nc, int topk, int nz) {
    if (nch <= 0 || topk <= 0 || topk > kKeep || nz <= 0) return RK_ERR_SHAPE;
    if (!pow2(nc) || nc < nch * kKeep || nc > kMaxNC) return RK_ERR_SHAPE;
    return RK_OK;
}

int check_stop(int hdt, int wdt, int H, int nz) {
    if (hdt != RK_F16 && hdt != RK_BF16 && hdt != RK_F32) return RK_ERR_DTYPE;
    if (wdt != RK_F16 && wdt != RK_BF16 && wdt != RK_F32) return RK_ERR_DTYPE;
    if (H <= 0 || H > 16384 || nz <= 0) return RK_ERR_SHAPE;
    return RK_OK;
}

}  // namespace

extern "C" int rk_stop_hidden(const void* h, int h_dtype, const float* lnw, const float* lnb, const void* w1,
                              int w1_dtype, const float* b1, float* z1, float eps, int H, int nz,
                              rk_stream_t stream) {
    if (!h || !lnw || !lnb || !w1 || !b1 || !z1) return RK_ERR_NULL;
    if (const int e = check_stop(h_dtype, w1_dtype, H, nz)) return e;
    if (((uintptr_t)w1 & 15) && w1_dtype != RK_F32) return RK_ERR_ALIGN;
    hipLaunchKernelGGL(stop_hidden_kernel, dim3((nz + kStopRows - 1) / kStopRows), dim3(kThreads),
                       (size_t)H * sizeof(float), (hipStream_t)stream, h, h_dtype, lnw, lnb, w1, w1_dtype, b1, z1,
                       eps, H, nz);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_topk_partial(const void* logits, int logits_dtype, const int64_t* step, int64_t* keys, int nv,
                               int end_idx, int min_new, rk_stream_t stream) {
    if (!logits || !step || !keys) return RK_ERR_NULL;
    if (logits_dtype != RK_F16 && logits_dtype != RK_BF16 && logits_dtype != RK_F32) return RK_ERR_DTYPE;
    if (nv <= 0) return RK_ERR_SHAPE;
    const int nch = (nv + kCH - 1) / kCH;
    hipLaunchKernelGGL(topk_partial_kernel, dim3(nch), dim3(kThreads), 0,
                       (hipStream_t)stream, logits, logits_dtype, step, keys, nv, end_idx, min_new);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_pick(const int64_t* keys, int64_t* scratch, const float* u, const float* z1, const float* w2,
                       const float* b2, const int64_t* ids, int64_t* step, int64_t* tok, int64_t* out,
                       float inv_temp, int64_t end_id, int min_new, int nch, int nc, int topk, int nz,
                       rk_stream_t stream) {
    if (!keys || !scratch || !u || !z1 || !w2 || !b2 || !ids || !step || !tok || !out) return RK_ERR_NULL;
    if (const int e = check_pick(nch, nc, topk, nz)) return e;
    hipLaunchKernelGGL(pick_kernel, dim3(1), dim3(kThreads), (size_t)nch * kKeep * sizeof(int64_t),
                       (hipStream_t)stream, keys, scratch, u, z1, w2, b2, ids, step, tok, out, inv_temp, end_id,
                       min_new, nch, topk, nz);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_sample_tail(const void* h, int h_dtype, const float* lnw, const float* lnb, const void* w1,
                              int w1_dtype, const float* b1, const float* w2, const float* b2, float eps, int H,
                              int nz, const void* logits, int logits_dtype, int nv, int end_idx, const float* u,
                              const int64_t* ids, int64_t* step, int64_t* tok, int64_t* out, float inv_temp,
                              int64_t end_id, int min_new, int topk, int64_t* keys, int64_t* scratch, int nc,
                              float* z1, unsigned* counter, rk_stream_t stream) {
    if (!h || !lnw || !lnb || !w1 || !b1 || !w2 || !b2 || !logits || !u || !ids || !step || !tok || !out || !keys ||
        !scratch || !z1 || !counter)
        return RK_ERR_NULL;
    if (const int e = check_stop(h_dtype, w1_dtype, H, nz)) return e;
    if (logits_dtype != RK_F16 && logits_dtype != RK_BF16 && logits_dtype != RK_F32) return RK_ERR_DTYPE;
    if (nv <= 0) return RK_ERR_SHAPE;
    const int nch = (nv + kCH - 1) / kCH;
    if (const int e = check_pick(nch, nc, topk, nz)) return e;
    if (((uintptr_t)w1 & 15) && w1_dtype != RK_F32) return RK_ERR_ALIGN;
    TailArgs a;
    a.h = h; a.lnw = lnw; a.lnb = lnb; a.w1 = w1; a.b1 = b1; a.w2 = w2; a.b2 = b2; a.u = u;
    a.logits = logits; a.ids = ids; a.keys = keys; a.scratch = scratch; a.step = step; a.tok = tok; a.out = out;
    a.z1 = z1; a.counter = counter; a.eps = eps; a.inv_temp = inv_temp; a.end_id = end_id;
    a.hdt = h_dtype; a.wdt = w1_dtype; a.ldt = logits_dtype; a.H = H; a.nz = nz; a.nv = nv; a.end_idx = end_idx;
    a.min_new = min_new; a.nch = nch; a.topk = topk; a.nzb = (nz + kStopRows - 1) / kStopRows;
    const size_t lds = std::max((size_t)H * sizeof(float), (size_t)nch * kKeep * sizeof(int64_t));
    const int chunk_blocks = nch;  // one block per chunk
    hipLaunchKernelGGL(sample_tail_kernel, dim3(a.nzb + chunk_blocks), dim3(kThreads), lds, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
