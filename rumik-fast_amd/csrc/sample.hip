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
// so sorting keys sorts values (monotonic also for -inf) and breaks ties by the larger index. Stage 1 sorts each
// chunk of 512 keys (descending) in LDS with a bitonic network; stage 2 gathers the first 32 of every chunk, sorts
// them and samples from the first top_k.
//
// Entry points: the reference's three kernels one to one (rk_stop_hidden, rk_topk_partial, rk_pick; buffers and
// their contents as the reference's: keys = every chunk sorted, scratch = the sorted candidate list), and
// rk_sample_tail, the same work in ONE launch: blocks [0, nzb) compute the stop predictor's hidden layer, blocks
// [nzb, nzb + nch) sort one chunk each; every block then bumps a completion counter (release fence + device-scope
// atomic) and the last block to arrive does the pick (acquire fence first). No block waits for another, so the
// grid needs no co-residency, and the last block resets the counter, so replays need no memset.
#include <algorithm>

#include "common.h"

namespace {

constexpr int kCH = 512;       // logits per chunk (reference CH)
constexpr int kKeep = 32;      // survivors per chunk (reference KEEP, >= top_k)
constexpr int kMaxNC = 4096;   // candidate slots of the pick (32 KB of LDS)
constexpr int kStopRows = 4;   // stop-predictor rows per block (one per wave)
constexpr int kThreads = 256;

RK_DEV int32_t sortable(float x) {
    const int32_t b = __builtin_bit_cast(int32_t, x);
    return b ^ ((b >> 31) & 0x7FFFFFFF);
}
RK_DEV float unsortable(int32_t k) { return __builtin_bit_cast(float, k ^ ((k >> 31) & 0x7FFFFFFF)); }
RK_DEV int64_t make_key(float x, int i) {
    return (int64_t)(((uint64_t)(uint32_t)sortable(x) << 32) | (uint64_t)(uint32_t)i);
}

// descending bitonic sort of n (a power of two) keys in LDS by the whole block
RK_DEV void bitonic_desc(int64_t* s, int n) {
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < n; i += blockDim.x) {
                const int p = i ^ j;
                if (p > i) {
                    const int64_t a = s[i], b = s[p];
                    const bool desc = (i & k) == 0;  // this half of the k-block runs descending
                    if (desc ? a < b : a > b) {
                        s[i] = b;
                        s[p] = a;
                    }
                }
            }
            __syncthreads();
        }
    }
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
    const int lane = threadIdx.x & 63, r = r0 + (threadIdx.x >> 6);
    if (r >= nz) return;
    float acc = 0.f;
    if (H % 512 == 0 && wdt != RK_F32) {  // 8 weights (16 bytes) per lane per step
        const uint4* wr = reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(w1) + (size_t)r * H);
        for (int c = lane; c < H / 8; c += 64) {
            const uint4 q = wr[c];
            const uint32_t d[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float lo = wdt == RK_BF16 ? bf16_bits_to_f32((uint16_t)d[e]) : f16_bits_to_f32((uint16_t)d[e]);
                const float hi = wdt == RK_BF16 ? bf16_bits_to_f32((uint16_t)(d[e] >> 16))
                                                : f16_bits_to_f32((uint16_t)(d[e] >> 16));
                acc = __builtin_fmaf(lo, z[8 * c + 2 * e], acc);
                acc = __builtin_fmaf(hi, z[8 * c + 2 * e + 1], acc);
            }
        }
    } else {
        for (int k = lane; k < H; k += 64) acc = __builtin_fmaf(load_act(w1, wdt, (size_t)r * H + k), z[k], acc);
    }
    acc = wave_sum(acc) + b1[r];
    if (lane == 0) z1[r] = 0.5f * acc * (1.0f + erff(acc * 0.7071067811865476f));  // exact GELU (F.gelu)
}

// ---- stage 1 (reference topk_partial, sample.py:53-61): chunk c's keys, sorted descending, into keys[c * 512 ..]
RK_DEV void topk_chunk(const void* logits, int ldt, const int64_t* step, int64_t* keys, int nv, int end_idx,
                       int min_new, int c, int64_t* s) {
    const bool early = step[0] < (int64_t)min_new;
    for (int e = threadIdx.x; e < kCH; e += blockDim.x) {
        const int i = c * kCH + e;
        float x = i < nv ? load_act(logits, ldt, (size_t)i) : -INFINITY;
        if (early && i == end_idx) x = -INFINITY;  // no </audio> during the first min_new tokens
        s[e] = make_key(x, i);
    }
    __syncthreads();
    bitonic_desc(s, kCH);
    for (int e = threadIdx.x; e < kCH; e += blockDim.x) keys[(size_t)c * kCH + e] = s[e];
}

// ---- stage 2 (reference pick, sample.py:65-93): merge the chunks' top 32, sample, stop rule, counters
RK_DEV void pick_block(const int64_t* keys, int64_t* scratch, const float* u, const float* z1, const float* w2,
                       const float* b2, const int64_t* ids, int64_t* step_p, int64_t* tok, int64_t* out,
                       float inv_temp, int64_t end_id, int min_new, int nch, int nc, int topk, int nz, int64_t* s,
                       float* red) {
    for (int c = threadIdx.x; c < nc; c += blockDim.x) {
        const int ch = c / kKeep;
        s[c] = ch < nch ? keys[(size_t)ch * kCH + c % kKeep] : -(int64_t(1) << 62);
    }
    float part = 0.f;
    for (int r = threadIdx.x; r < nz; r += blockDim.x) part = __builtin_fmaf(z1[r], w2[r], part);
    const float stop_logit = block_sum(part, red) + b2[0];  // sigmoid(.) > 0.5  <=>  stop_logit > 0
    __syncthreads();
    bitonic_desc(s, nc);
    for (int c = threadIdx.x; c < nc; c += blockDim.x) scratch[c] = s[c];
    if (threadIdx.x >= 64) return;
    const int j = threadIdx.x;  // candidate rank (lanes 0..31 hold the top 32, best first)
    const int64_t top = s[j & 31];
    const float val = unsortable((int32_t)(top >> 32));
    const int idx = (int)(uint32_t)(top & 0xFFFFFFFF);
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
    __shared__ int64_t s[kCH];
    topk_chunk(logits, ldt, step, keys, nv, end_idx, min_new, blockIdx.x, s);
}

__global__ __launch_bounds__(kThreads) void pick_kernel(const int64_t* keys, int64_t* scratch, const float* u,
                                                        const float* z1, const float* w2, const float* b2,
                                                        const int64_t* ids, int64_t* step_p, int64_t* tok,
                                                        int64_t* out, float inv_temp, int64_t end_id, int min_new,
                                                        int nch, int nc, int topk, int nz) {
    extern __shared__ __align__(16) int64_t ssm[];
    __shared__ float red[16];
    pick_block(keys, scratch, u, z1, w2, b2, ids, step_p, tok, out, inv_temp, end_id, min_new, nch, nc, topk, nz,
               ssm, red);
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
    int hdt, wdt, ldt, H, nz, nv, end_idx, min_new, nch, nc, topk, nzb;
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
        topk_chunk(a.logits, a.ldt, a.step, a.keys, a.nv, a.end_idx, a.min_new, b - a.nzb,
                   reinterpret_cast<int64_t*>(raw));
    __threadfence();  // release: every thread's z1 / keys stores are visible device-wide before the count
    __syncthreads();
    if (threadIdx.x == 0) last = atomicAdd(a.counter, 1u) == gridDim.x - 1;
    __syncthreads();
    if (!last) return;
    __threadfence();  // acquire: the other blocks' z1 / keys
    if (threadIdx.x == 0) *a.counter = 0u;  // ready for the next call (stream order)
    pick_block(a.keys, a.scratch, a.u, a.z1, a.w2, a.b2, a.ids, a.step, a.tok, a.out, a.inv_temp, a.end_id,
               a.min_new, a.nch, a.nc, a.topk, a.nz, reinterpret_cast<int64_t*>(raw), red);
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
    hipLaunchKernelGGL(topk_partial_kernel, dim3((nv + kCH - 1) / kCH), dim3(kThreads), 0, (hipStream_t)stream,
                       logits, logits_dtype, step, keys, nv, end_idx, min_new);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

extern "C" int rk_pick(const int64_t* keys, int64_t* scratch, const float* u, const float* z1, const float* w2,
                       const float* b2, const int64_t* ids, int64_t* step, int64_t* tok, int64_t* out,
                       float inv_temp, int64_t end_id, int min_new, int nch, int nc, int topk, int nz,
                       rk_stream_t stream) {
    if (!keys || !scratch || !u || !z1 || !w2 || !b2 || !ids || !step || !tok || !out) return RK_ERR_NULL;
    if (const int e = check_pick(nch, nc, topk, nz)) return e;
    hipLaunchKernelGGL(pick_kernel, dim3(1), dim3(kThreads), (size_t)nc * sizeof(int64_t), (hipStream_t)stream,
                       keys, scratch, u, z1, w2, b2, ids, step, tok, out, inv_temp, end_id, min_new, nch, nc, topk,
                       nz);
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
    a.min_new = min_new; a.nch = nch; a.nc = nc; a.topk = topk; a.nzb = (nz + kStopRows - 1) / kStopRows;
    const size_t lds = std::max(std::max((size_t)H * sizeof(float), (size_t)kCH * sizeof(int64_t)),
                                (size_t)nc * sizeof(int64_t));
    hipLaunchKernelGGL(sample_tail_kernel, dim3(a.nzb + nch), dim3(kThreads), lds, (hipStream_t)stream, a);
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
