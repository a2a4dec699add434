// HBM read ceiling of one launch on gfx950: the bench's yardstick for the
// decode GEMVs (bench.py "hbm_read_ceiling"), built as its own library
// (libomni_read_ceiling.so) and not part of the operator ABI.
//
// One launch streams `bytes` (a multiple of 16) from a buffer with
// nontemporal 16-byte loads: thread t of block b loads the U 16-byte chunks
// b * U * T + u * T + t (u < U; each load instruction of a wave reads 1 KiB
// of consecutive bytes), every load of a thread issued before any result is
// used, then XORs them into one word that is stored to
// the sink only if it equals `never`, so the loads cannot be dropped while
// the launch writes at most that one word. A GEMV of the same bytes also
// reads its activations, does its dot products and reduces across lanes;
// this is the bare streaming read it cannot beat.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int U, int T>
__global__ __launch_bounds__(T) void read_kernel(const u32x4* __restrict__ src, int64_t chunks, uint32_t never,
                                                 uint32_t* sink) {
    const int64_t first = (int64_t)blockIdx.x * U * T + threadIdx.x;
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int64_t c = first + (int64_t)u * T < chunks ? first + (int64_t)u * T : chunks - 1;
        v[u] = __builtin_nontemporal_load(src + c);
    }
    uint32_t fold = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) fold ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (fold == never) sink[0] = fold;
}

template <int U, int T>
hipError_t launch(const void* src, int64_t chunks, uint32_t never, uint32_t* sink, hipStream_t stream) {
    const int64_t per_block = (int64_t)U * T;
    const int64_t blocks = (chunks + per_block - 1) / per_block;
    hipLaunchKernelGGL((read_kernel<U, T>), dim3((unsigned)blocks), dim3(T), 0, stream,
                       static_cast<const u32x4*>(src), chunks, never, sink);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Launch shapes: 0..8 = (U, T) in {1, 2, 4} x {256, 512, 1024}.
int omni_read_ceiling_shapes(void) { return 9; }

// One streaming read of `bytes` (> 0, a multiple of 16; `src` 16-byte
// aligned) with launch shape `shape`; `sink` is a device word the kernel
// writes only if the fold of every loaded word equals `never`. 0 on success,
// -1 on a bad argument, else the HIP error code.
int omni_read_ceiling(const void* src, int64_t bytes, int shape, uint32_t never, uint32_t* sink, void* stream) {
    if (!src || !sink || bytes <= 0 || bytes % 16 != 0 || reinterpret_cast<uintptr_t>(src) % 16 != 0 ||
        shape < 0 || shape >= 9)
        return -1;
    const int64_t chunks = bytes / 16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e;
    switch (shape) {
        case 0: e = launch<1, 256>(src, chunks, never, sink, s); break;
        case 1: e = launch<1, 512>(src, chunks, never, sink, s); break;
        case 2: e = launch<1, 1024>(src, chunks, never, sink, s); break;
        case 3: e = launch<2, 256>(src, chunks, never, sink, s); break;
        case 4: e = launch<2, 512>(src, chunks, never, sink, s); break;
        case 5: e = launch<2, 1024>(src, chunks, never, sink, s); break;
        case 6: e = launch<4, 256>(src, chunks, never, sink, s); break;
        case 7: e = launch<4, 512>(src, chunks, never, sink, s); break;
        default: e = launch<4, 1024>(src, chunks, never, sink, s); break;
    }
    return e == hipSuccess ? 0 : (int)e;
}

}  // extern "C"
