// Read-only ceiling for the int4 weight stream (a measurement kernel, counterpart of the reference's
// kernels/roofline.py:20-33 `read_only`): it reads exactly the bytes an int4 GEMV launch reads from HBM (the codes,
// the scales and the mins: three buffers) and does no arithmetic beyond one 32-bit wrapping sum per block, so its
// time is what one launch of that many bytes costs on this part, and its result can be checked bit for bit.
//
// Every thread streams 16-byte nontemporal loads (the GEMV's own load width and hint), UNROLL of them in flight
// per loop step, grid-stride over each buffer in turn; `blocks` and `unroll` are the launch-shape knobs a caller
// sweeps for the best case.
#include "common.h"

namespace {

constexpr int kThreads = 256;

template <int UNROLL>
RK_DEV uint32_t stream_sum(const uint4* p, size_t n16) {
    uint32_t acc = 0;
    const size_t stride = (size_t)gridDim.x * kThreads;
    size_t i = (size_t)blockIdx.x * kThreads + threadIdx.x;
    for (; i + (UNROLL - 1) * stride < n16; i += UNROLL * stride) {
        u4_t v[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) v[u] = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p) + i + u * stride);
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) acc += v[u][0] + v[u][1] + v[u][2] + v[u][3];
    }
    for (; i < n16; i += stride) {
        const u4_t v = __builtin_nontemporal_load(reinterpret_cast<const u4_t*>(p) + i);
        acc += v[0] + v[1] + v[2] + v[3];
    }
    return acc;
}

template <int UNROLL>
__global__ __launch_bounds__(kThreads) void read_only_kernel(const uint4* a, size_t na, const uint4* b, size_t nb,
                                                             const uint4* c, size_t nc, uint32_t* sink) {
    __shared__ uint32_t part[kThreads / 64];
    uint32_t acc = stream_sum<UNROLL>(a, na) + stream_sum<UNROLL>(b, nb) + stream_sum<UNROLL>(c, nc);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) acc += __shfl_xor(acc, o);
    if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t s = 0;
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) s += part[w];
        sink[blockIdx.x] = s;
    }
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace

extern "C" int rk_read_only(const void* a, size_t na, const void* b, size_t nb, const void* c, size_t nc, int blocks,
                            int unroll, uint32_t* sink, rk_stream_t stream) {
    if (!sink || (na && !a) || (nb && !b) || (nc && !c)) return RK_ERR_NULL;
    if (na % 16 || nb % 16 || nc % 16) return RK_ERR_SHAPE;
    if (!aligned16(a) || !aligned16(b) || !aligned16(c)) return RK_ERR_ALIGN;
    if (blocks <= 0 || blocks > 65536) return RK_ERR_BLOCK;
    hipStream_t st = (hipStream_t)stream;
    const uint4 *pa = (const uint4*)a, *pb = (const uint4*)b, *pc = (const uint4*)c;
    switch (unroll) {
        case 1: hipLaunchKernelGGL(read_only_kernel<1>, dim3(blocks), dim3(kThreads), 0, st, pa, na / 16, pb, nb / 16, pc, nc / 16, sink); break;
        case 2: hipLaunchKernelGGL(read_only_kernel<2>, dim3(blocks), dim3(kThreads), 0, st, pa, na / 16, pb, nb / 16, pc, nc / 16, sink); break;
        case 4: hipLaunchKernelGGL(read_only_kernel<4>, dim3(blocks), dim3(kThreads), 0, st, pa, na / 16, pb, nb / 16, pc, nc / 16, sink); break;
        case 8: hipLaunchKernelGGL(read_only_kernel<8>, dim3(blocks), dim3(kThreads), 0, st, pa, na / 16, pb, nb / 16, pc, nc / 16, sink); break;
        default: return RK_ERR_BLOCK;
    }
    return hipGetLastError() == hipSuccess ? RK_OK : RK_ERR_LAUNCH;
}
