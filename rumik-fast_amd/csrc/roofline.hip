// Read-only ceiling for the int4 weight stream (a measurement kernel, counterpart of the reference's
// kernels/roofline.py:20-33 `read_only`): it reads exactly the bytes an int4 GEMV launch reads from HBM (the codes,
// the scales and the mins: three buffers) and does no arithmetic beyond one 32-bit wrapping sum per block, so its
// time is what one launch of that many bytes costs on this part, and its result can be checked bit for bit.
//
// The three buffers are one logical range of 16-byte items (a's, then b's, then c's) walked in ONE grid-stride
// pass: every thread keeps UNROLL 16-byte nontemporal loads (the GEMV's own load width and hint) in flight per loop
// step, and no part of the grid waits at a buffer boundary while the rest of the range is still unread. `threads`
// (256 / 512 / 1024 per block), `blocks` and `unroll` are the launch-shape knobs a caller sweeps for the best case.
#include "common.h"

namespace {

struct Range3 {
    const u4_t* p[3];
    size_t end0, end1, n;  // item boundaries: [0, end0) in a, [end0, end1) in b, [end1, n) in c
};

RK_DEV const u4_t* item(const Range3& r, size_t i) {
    return i < r.end0 ? r.p[0] + i : (i < r.end1 ? r.p[1] + (i - r.end0) : r.p[2] + (i - r.end1));
}

template <int THREADS, int UNROLL>
__global__ __launch_bounds__(THREADS) void read_only_kernel(Range3 r, uint32_t* sink) {
    __shared__ uint32_t part[THREADS / 64];
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * THREADS;
    size_t i = (size_t)blockIdx.x * THREADS + threadIdx.x;
    for (; i + (UNROLL - 1) * stride < r.n; i += UNROLL * stride) {
        u4_t v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(item(r, i + u * stride));
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc += v[u][0] + v[u][1] + v[u][2] + v[u][3];
    }
    for (; i < r.n; i += stride) {
        const u4_t v = __builtin_nontemporal_load(item(r, i));
        acc += v[0] + v[1] + v[2] + v[3];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < THREADS / 64; ++w) s += part[w];
        sink[blockIdx.x] = s;
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

template <int THREADS>
int launch(const Range3& r, int blocks, int unroll, uint32_t* sink, hipStream_t st) {
    switch (unroll) {
        case 1: hipLaunchKernelGGL((read_only_kernel<THREADS, 1>), dim3(blocks), dim3(THREADS), 0, st, r, sink); break;
        case 2: hipLaunchKernelGGL((read_only_kernel<THREADS, 2>), dim3(blocks), dim3(THREADS), 0, st, r, sink); break;
        case 4: hipLaunchKernelGGL((read_only_kernel<THREADS, 4>), dim3(blocks), dim3(THREADS), 0, st, r, sink); break;
        case 8: hipLaunchKernelGGL((read_only_kernel<THREADS, 8>), dim3(blocks), dim3(THREADS), 0, st, r, sink); break;
        default: return RK_ERR_BLOCK;
    }
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}

}  // namespace

extern "C" int rk_read_only_ex(const void* a, size_t na, const void* b, size_t nb, const void* c, size_t nc,
                               int threads, int blocks, int unroll, uint32_t* sink, rk_stream_t stream) {
    if (!sink || (na && !a) || (nb && !b) || (nc && !c)) return RK_ERR_NULL;
    if (na % 16 || nb % 16 || nc % 16) return RK_ERR_SHAPE;
    if (!aligned16(a) || !aligned16(b) || !aligned16(c)) return RK_ERR_ALIGN;
    if (blocks <= 0 || blocks > 65536) return RK_ERR_BLOCK;
    if (!(unroll == 1 || unroll == 2 || unroll == 4 || unroll == 8)) return RK_ERR_BLOCK;
    Range3 r;
    r.p[0] = (const u4_t*)a;
    r.p[1] = (const u4_t*)b;
    r.p[2] = (const u4_t*)c;
    r.end0 = na / 16;
    r.end1 = r.end0 + nb / 16;
    r.n = r.end1 + nc / 16;
    hipStream_t st = (hipStream_t)stream;
    switch (threads) {
        case 256: return launch<256>(r, blocks, unroll, sink, st);
        case 512: return launch<512>(r, blocks, unroll, sink, st);
        case 1024: return launch<1024>(r, blocks, unroll, sink, st);
        default: return RK_ERR_BLOCK;
    }
}

extern "C" int rk_read_only(const void* a, size_t na, const void* b, size_t nb, const void* c, size_t nc, int blocks,
                            int unroll, uint32_t* sink, rk_stream_t stream) {
    return rk_read_only_ex(a, na, b, nb, c, nc, 256, blocks, unroll, sink, stream);
}
