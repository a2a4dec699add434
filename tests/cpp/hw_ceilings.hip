// Hardware ceilings of MI355X (gfx950) that bound the int8 hot path's kernels.
// Measurement infrastructure, not a test: each mode prints one line per case.
//
//   hw_ceilings mfma    v_mfma_i32_32x32x32_i8 and v_mfma_scale_f32_32x32x64_f8f6f4
//                       back to back from registers, no memory traffic, one
//                       4-wave workgroup per CU, on random and on zero operands:
//                       TOPS and the shader clock (cycle counter against the
//                       100 MHz real-time counter) — the power-managed ceiling.
//   hw_ceilings ladder  the W8A8 ring kernel's K loop rebuilt one ingredient at a
//                       time, operands from LDS/L2 only: 24 MFMAs per 64-byte K
//                       tile per wave, + 14 fragment reads, + one barrier, + 7
//                       global->LDS copies per wave issued between MFMAs, + the
//                       same copies issued by 4 separate producer waves.
//   hw_ceilings read    one launch streaming 58.7 MB (the decode GEMV's weight
//                       bytes) over 19 rotating copies, for several grid sizes:
//                       the single-launch HBM read ceiling.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#define CK(x)                                                                       \
    do {                                                                            \
        hipError_t e_ = (x);                                                        \
        if (e_ != hipSuccess) {                                                     \
            printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);   \
            exit(1);                                                                \
        }                                                                           \
    } while (0)

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define LDS_AS __attribute__((address_space(3)))

// ---------------------------------------------------------------- mfma --
template <bool FP8>
__global__ __launch_bounds__(256, 1) void mfma_loop(const v8i* src, int iters, int* out,
                                                     unsigned long long* clk) {
    const int lane = threadIdx.x & 63;
    const int w = blockIdx.x * 4 + (threadIdx.x >> 6);
    v8i a[4], b[4];
    for (int i = 0; i < 4; ++i) {
        a[i] = src[(w * 8 + i) * 64 + lane];
        b[i] = src[(w * 8 + 4 + i) * 64 + lane];
    }
    const unsigned long long t0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
    int res = 0;
    if constexpr (!FP8) {
        v16i acc[4][4] = {};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const v4i aa = {a[i][0], a[i][1], a[i][2], a[i][3]};
                    const v4i bb = {b[j][0], b[j][1], b[j][2], b[j][3]};
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(aa, bb, acc[i][j], 0, 0, 0);
                }
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j)
                for (int e = 0; e < 16; ++e) res ^= acc[i][j][e];
    } else {
        v16f acc[4][4] = {};
        for (int it = 0; it < iters; ++it)
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[i], b[j], acc[i][j], 0, 0,
                                                                                0, 127, 0, 127);
        for (int i = 0; i < 4; ++i)
            for (int j = 0; j < 4; ++j)
                for (int e = 0; e < 16; ++e) res ^= __float_as_int(acc[i][j][e]);
    }
    const unsigned long long t1 = __builtin_readcyclecounter(), r1 = __builtin_amdgcn_s_memrealtime();
    out[blockIdx.x * 256 + threadIdx.x] = res;
    if (threadIdx.x == 0) {
        clk[blockIdx.x * 2] = t1 - t0;
        clk[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

double mean_mhz(const std::vector<unsigned long long>& c, int n) {
    double mhz = 0;
    for (int i = 0; i < n; ++i) mhz += (double)c[2 * i] / (double)c[2 * i + 1] * 100.0;
    return mhz / n;
}

void run_mfma(int cus) {
    const size_t n = (size_t)cus * 4 * 8 * 64 * 8;  // ints
    std::vector<int> h(n);
    uint64_t s = 1;
    for (auto& v : h) {
        s = s * 6364136223846793005ULL + 1442695040888963407ULL;
        uint32_t r = (uint32_t)(s >> 32), o = 0;
        for (int k = 0; k < 4; ++k) {
            uint32_t byte = (r >> (8 * k)) & 0xff;
            if ((byte & 0x7f) == 0x7f) byte ^= 1;  // no fp8 NaN codes
            o |= byte << (8 * k);
        }
        v = (int)o;
    }
    v8i *rnd, *zero;
    int* out;
    unsigned long long* clk;
    CK(hipMalloc(&rnd, n * 4));
    CK(hipMalloc(&zero, n * 4));
    CK(hipMalloc(&out, (size_t)cus * 256 * 4));
    CK(hipMalloc(&clk, (size_t)cus * 16));
    CK(hipMemcpy(rnd, h.data(), n * 4, hipMemcpyHostToDevice));
    CK(hipMemset(zero, 0, n * 4));
    const int iters = 20000;
    for (int fp8 = 0; fp8 < 2; ++fp8)
        for (int z = 0; z < 2; ++z) {
            const v8i* src = z ? zero : rnd;
            auto launch = [&] {
                if (fp8)
                    hipLaunchKernelGGL(mfma_loop<true>, dim3(cus), dim3(256), 0, 0, src, iters, out, clk);
                else
                    hipLaunchKernelGGL(mfma_loop<false>, dim3(cus), dim3(256), 0, 0, src, iters, out, clk);
            };
            launch();
            CK(hipGetLastError());
            CK(hipDeviceSynchronize());
            hipEvent_t a, b;
            CK(hipEventCreate(&a));
            CK(hipEventCreate(&b));
            CK(hipEventRecord(a));
            for (int r = 0; r < 3; ++r) launch();
            CK(hipEventRecord(b));
            CK(hipEventSynchronize(b));
            float ms;
            CK(hipEventElapsedTime(&ms, a, b));
            ms /= 3;
            std::vector<unsigned long long> c((size_t)cus * 2);
            CK(hipMemcpy(c.data(), clk, c.size() * 8, hipMemcpyDeviceToHost));
            const double ops = (double)cus * 4 * iters * 16 * (fp8 ? 131072.0 : 65536.0);
            printf("mfma %-28s operands %-6s: %7.3f ms  %6.0f TOPS  clock %5.0f MHz  %.1f cycles/MFMA\n",
                   fp8 ? "f8f6f4 32x32x64 (fp8)" : "i32_32x32x32_i8", z ? "zero" : "random", ms,
                   ops / (ms * 1e-3) / 1e12, mean_mhz(c, cus), (double)c[0] / (iters * 16.0));
        }
    CK(hipFree(rnd));
    CK(hipFree(zero));
    CK(hipFree(out));
    CK(hipFree(clk));
}

// -------------------------------------------------------------- ladder --
// The ring kernel's per-wave K-tile work: a 128 x 96 block of 32x32 int32
// accumulators (4 x 3 MFMAs per 32-byte k step, two k steps per 64-byte tile),
// fragment reads from a 4-stage LDS ring of 256 + 192 rows of 64 bytes, and
// 7 one-KiB global->LDS copies per wave per tile from an L2-resident buffer.
// RUNG 0: MFMAs only; 1: + fragment reads; 2: + one barrier per tile;
// 3: + copies between MFMAs; 4: 4 more waves do the copies (512 threads).
constexpr int kStage = (256 + 192) * 64;

template <int RUNG>
__global__ __launch_bounds__(RUNG == 4 ? 512 : 256, 1) void ladder(const uint8_t* __restrict__ src,
                                                                   int iters, int* out,
                                                                   unsigned long long* clk) {
    __shared__ __attribute__((aligned(1024))) uint8_t lds[4][kStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave_id = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wave = wave_id & 3;
    const bool producer = RUNG == 4 && wave_id >= 4;
    for (int i = (tid & 255) * 16; i < 4 * kStage; i += 256 * 16) {
        const uint32_t h = (uint32_t)(i + blockIdx.x * 7919) * 2654435761u;
        const v4i v = {(int)h, (int)(h * 2246822519u), (int)(h * 3266489917u), (int)(h ^ 0x9e3779b9u)};
        *reinterpret_cast<v4i*>(&lds[0][0] + i) = v;
    }
    __syncthreads();
    const int fr = lane & 31, fh = lane >> 5, fq = (fr >> 2) & 3;
    const int wm = wave >> 1, wn = wave & 1;
    const int fa0 = (wm * 128 + fr) * 64 + ((fh ^ fq) << 4);
    const int fa1 = (wm * 128 + fr) * 64 + (((2 + fh) ^ fq) << 4);
    const int fb0 = 256 * 64 + (wn * 96 + fr) * 64 + ((fh ^ fq) << 4);
    const int fb1 = 256 * 64 + (wn * 96 + fr) * 64 + (((2 + fh) ^ fq) << 4);
    v4i fa[4], fb[3];
    for (int i = 0; i < 4; ++i) fa[i] = *reinterpret_cast<const v4i*>(&lds[0][0] + fa0 + i * 2048);
    for (int j = 0; j < 3; ++j) fb[j] = *reinterpret_cast<const v4i*>(&lds[0][0] + fb0 + j * 2048);
    v16i acc[4][3] = {};
    // Copy c of a wave: 64 lanes x 16 bytes of tile rows, from a 2 MB window.
    const int cp_row = lane >> 2, cp_chunk = (lane & 3) ^ ((lane >> 4) & 3);
    const uint8_t* cs = src + ((size_t)(blockIdx.x % 64) * 448 + wave * 112 + cp_row) * 64 + cp_chunk * 16;
    (void)cs;  // used by the device pass only
    auto copy = [&](int it, int c) {
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_global_load_lds(cs + (size_t)(it & 31) * kStage + c * 1024,
                                         (LDS_AS void*)(&lds[(it + 3) & 3][0] + wave * 7168 + c * 1024), 16, 0, 0);
#endif
    };
    const unsigned long long t0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
    if (producer) {
        for (int it = 0; it < iters; ++it) {
#pragma unroll
            for (int c = 0; c < 7; ++c) copy(it, c);
            __builtin_amdgcn_s_waitcnt((14 & 15) | (7 << 4) | (15 << 8));  // vmcnt(14)
            asm volatile("s_barrier" ::: "memory");
        }
    } else {
        for (int it = 0; it < iters; ++it) {
            const int st = it & 3;
#pragma unroll
            for (int ks = 0; ks < 2; ++ks) {
#pragma unroll
                for (int q = 0; q < 12; ++q) {
                    const int i = q / 3, j = q % 3;
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
                    if constexpr (RUNG == 3)
                        if (ks == 1 && q < 7) copy(it, q);
                    if constexpr (RUNG >= 1)
                        if (q < 7) {
                            const uint8_t* base = &lds[st][0];
                            if (q < 4)
                                fa[q] = *reinterpret_cast<const v4i*>(base + (ks ? fa1 : fa0) + q * 2048);
                            else
                                fb[q - 4] = *reinterpret_cast<const v4i*>(base + (ks ? fb1 : fb0) + (q - 4) * 2048);
                        }
                    __builtin_amdgcn_sched_barrier(0);
                }
                if constexpr (RUNG >= 2)
                    if (ks == 0) {
                        if constexpr (RUNG == 3)
                            __builtin_amdgcn_s_waitcnt((14 & 15) | (7 << 4) | (0 << 8));  // vmcnt(14) lgkmcnt(0)
                        else
                            __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));  // lgkmcnt(0)
                        asm volatile("s_barrier" ::: "memory");
                    }
            }
        }
    }
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned long long t1 = __builtin_readcyclecounter(), r1 = __builtin_amdgcn_s_memrealtime();
    int res = 0;
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 3; ++j)
            for (int e = 0; e < 16; ++e) res ^= acc[i][j][e];
    if (tid < 256) out[blockIdx.x * 256 + tid] = res;
    if (tid == 0) {
        clk[blockIdx.x * 2] = t1 - t0;
        clk[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

void run_ladder(int cus) {
    // 64 windows of 448 rows, plus 32 K tiles of stride: every copy stays inside.
    const size_t bytes = (size_t)64 * 448 * 64 + (size_t)32 * kStage + 4096;
    std::vector<uint8_t> h(bytes);
    uint32_t s = 1;
    for (auto& b : h) {
        s = s * 1664525u + 1013904223u;
        b = (uint8_t)(s >> 24);
    }
    uint8_t* src;
    int* out;
    unsigned long long* clk;
    CK(hipMalloc(&src, bytes));
    CK(hipMalloc(&out, (size_t)cus * 256 * 4));
    CK(hipMalloc(&clk, (size_t)cus * 16));
    CK(hipMemcpy(src, h.data(), bytes, hipMemcpyHostToDevice));
    const int iters = 4000;
    const char* names[] = {"MFMAs only", "+ LDS fragment reads", "+ barrier per K tile",
                           "+ 7 LDS-DMA copies/wave between MFMAs", "copies by 4 producer waves"};
    for (int rep = 0; rep < 2; ++rep)
        for (int rung = 0; rung < 5; ++rung) {
            auto launch = [&] {
                switch (rung) {
                    case 0: hipLaunchKernelGGL(ladder<0>, dim3(cus), dim3(256), 0, 0, src, iters, out, clk); break;
                    case 1: hipLaunchKernelGGL(ladder<1>, dim3(cus), dim3(256), 0, 0, src, iters, out, clk); break;
                    case 2: hipLaunchKernelGGL(ladder<2>, dim3(cus), dim3(256), 0, 0, src, iters, out, clk); break;
                    case 3: hipLaunchKernelGGL(ladder<3>, dim3(cus), dim3(256), 0, 0, src, iters, out, clk); break;
                    default: hipLaunchKernelGGL(ladder<4>, dim3(cus), dim3(512), 0, 0, src, iters, out, clk);
                }
            };
            launch();
            CK(hipGetLastError());
            CK(hipDeviceSynchronize());
            hipEvent_t a, b;
            CK(hipEventCreate(&a));
            CK(hipEventCreate(&b));
            CK(hipEventRecord(a));
            for (int r = 0; r < 5; ++r) launch();
            CK(hipEventRecord(b));
            CK(hipEventSynchronize(b));
            float ms;
            CK(hipEventElapsedTime(&ms, a, b));
            ms /= 5;
            std::vector<unsigned long long> c((size_t)cus * 2);
            CK(hipMemcpy(c.data(), clk, c.size() * 8, hipMemcpyDeviceToHost));
            double cyc = 0;
            for (int i = 0; i < cus; ++i) cyc += (double)c[2 * i];
            cyc /= cus;
            const double mfmas = (double)iters * 24;
            printf("ladder pass %d rung %d %-40s: %6.0f TOPS  clock %5.0f MHz  %5.1f cycles/MFMA  MFMA busy %5.1f%%\n",
                   rep, rung, names[rung], (double)cus * 4 * mfmas * 65536 / (ms * 1e-3) / 1e12,
                   mean_mhz(c, cus), cyc / mfmas, 3200.0 / (cyc / mfmas));
        }
    CK(hipFree(src));
    CK(hipFree(out));
    CK(hipFree(clk));
}

// ---------------------------------------------------------------- read --
__global__ __launch_bounds__(256) void stream_read(const uint4* __restrict__ p, int64_t n16, unsigned* out) {
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    unsigned x = 0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += stride) {
        const uint4 v = p[i];
        x ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (x == 0x12345678u) out[0] = x;  // keeps the loads
}

void run_read() {
    const int64_t bytes = 4096LL * 14336, n16 = bytes / 16;
    const int copies = 19;
    uint4* buf;
    unsigned* out;
    CK(hipMalloc(&buf, bytes * copies));
    CK(hipMalloc(&out, 64));
    CK(hipMemset(buf, 1, bytes * copies));
    hipStream_t s;
    CK(hipStreamCreate(&s));
    for (int grid : {512, 1024, 2048, 4096, 8192}) {
        const int iters = copies * 10;
        hipGraph_t g;
        hipGraphExec_t ge;
        CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
        for (int i = 0; i < iters; ++i)
            hipLaunchKernelGGL(stream_read, dim3(grid), dim3(256), 0, s, buf + (int64_t)(i % copies) * n16, n16, out);
        CK(hipStreamEndCapture(s, &g));
        CK(hipGraphInstantiate(&ge, g, nullptr, nullptr, 0));
        CK(hipGraphLaunch(ge, s));
        CK(hipStreamSynchronize(s));
        float best = 1e30f;
        for (int rep = 0; rep < 3; ++rep) {
            hipEvent_t a, b;
            CK(hipEventCreate(&a));
            CK(hipEventCreate(&b));
            CK(hipEventRecord(a, s));
            CK(hipGraphLaunch(ge, s));
            CK(hipEventRecord(b, s));
            CK(hipEventSynchronize(b));
            float ms;
            CK(hipEventElapsedTime(&ms, a, b));
            best = std::min(best, ms);
        }
        const double us = best * 1000.0 / iters;
        printf("read 58.7 MB per launch, grid %5d x 256: %6.2f us  %5.0f GB/s\n", grid, us, bytes / us / 1e3);
        CK(hipGraphExecDestroy(ge));
        CK(hipGraphDestroy(g));
    }
    CK(hipFree(buf));
    CK(hipFree(out));
}

int main(int argc, char** argv) {
    const char* mode = argc > 1 ? argv[1] : "all";
    int cus = 0;
    CK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
    hipDeviceProp_t prop;
    CK(hipGetDeviceProperties(&prop, 0));
    if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0) {
        printf("device 0 is %s, not gfx950\n", prop.gcnArchName);
        return 1;
    }
    printf("device %s, %d CUs\n", prop.gcnArchName, cus);
    if (!strcmp(mode, "all") || !strcmp(mode, "mfma")) run_mfma(cus);
    if (!strcmp(mode, "all") || !strcmp(mode, "ladder")) run_ladder(cus);
    if (!strcmp(mode, "all") || !strcmp(mode, "read")) run_read();
    return 0;
}
