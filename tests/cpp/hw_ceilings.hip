// Hardware ceilings of MI355X (gfx950) that bound the int8 hot path's kernels.
// Measurement infrastructure, not a test: each mode prints one line per case.
//
//   hw_ceilings mfma    v_mfma_i32_32x32x32_i8 and v_mfma_scale_f32_32x32x64_f8f6f4
//                       back to back from registers, no memory traffic, one
//                       4-wave workgroup per CU, on random and on zero operands:
//                       TOPS and the shader clock (cycle counter against the
//                       100 MHz real-time counter) — the power-managed ceiling.
//   hw_ceilings ladder  the W8A8 ring kernel's K loop rebuilt one ingredient at a
//                       time (MFMAs, + double-buffered fragment reads, + one
//                       barrier, + global->LDS copies from L2, + the copies
//                       streaming the real kernel's operands from HBM), for
//                       128 x 96 and 128 x 128 per wave; then the fp16 ring's
//                       K loop (+ the int8 -> f16 weight conversion).
//   hw_ceilings read    one launch streaming 58.7 MB (the decode GEMV's weight
//                       bytes) over 19 rotating copies, every load of a thread
//                       issued up front, for several loads per thread and
//                       block sizes: the single-launch HBM read ceiling.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <type_traits>
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
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
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
// The int8 ring kernel's per-wave K-tile work, one ingredient at a time: a
// 128 x WN block of 32x32 int32 accumulators (two 32-byte k steps per 64-byte
// K tile), fragments double-buffered (the reads of the next k step are issued
// behind the current step's MFMAs, one per MFMA), and per K tile one barrier
// and (256 + 2 WN) / 64 one-KiB global->LDS copies per wave.
// RUNG 0: MFMAs only; 1: + fragment reads; 2: + one barrier per K tile;
// 3: + copies from an L2-resident window; 4: the copies stream the real
// kernel's operands instead: tile (m, n) of a 16 x 16 grid over A [4096][12288]
// and W [16 * 2 WN][12288], random bytes, K advancing 64 bytes per tile.
template <int WN, int RUNG>
__global__ __launch_bounds__(256, 1) void ladder8(const uint8_t* __restrict__ src, const uint8_t* __restrict__ big,
                                                  int iters, int* out, unsigned long long* clk) {
    constexpr int BN = 2 * WN;
    constexpr int kStage = (256 + BN) * 64;
    constexpr int kCpw = (256 + BN) / 64;
    constexpr int FM = 4, FN = WN / 32, PER = FM * FN;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[4][kStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int i = tid * 16; i < 4 * kStage; i += 256 * 16) {
        const uint32_t h = (uint32_t)(i + blockIdx.x * 7919) * 2654435761u;
        const v4i v = {(int)h, (int)(h * 2246822519u), (int)(h * 3266489917u), (int)(h ^ 0x9e3779b9u)};
        *reinterpret_cast<v4i*>(&lds[0][0] + i) = v;
    }
    __syncthreads();
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 31, fk = lane >> 5;
    int offA[FM], offB[FN];
    for (int i = 0; i < FM; ++i) offA[i] = (wm * 128 + i * 32 + fr) * 64 + fk * 16;
    for (int j = 0; j < FN; ++j) offB[j] = 256 * 64 + (wn * WN + j * 32 + fr) * 64 + fk * 16;
    v4i fa[2][FM], fb[2][FN];
    for (int i = 0; i < FM; ++i) fa[0][i] = fa[1][i] = *reinterpret_cast<const v4i*>(&lds[0][0] + offA[i]);
    for (int j = 0; j < FN; ++j) fb[0][j] = fb[1][j] = *reinterpret_cast<const v4i*>(&lds[0][0] + offB[j]);
    v16i acc[FM][FN];
    for (int i = 0; i < FM; ++i)
        for (int j = 0; j < FN; ++j) acc[i][j] = v16i{};
    const int cp_row = lane >> 2, cp_chunk = lane & 3;
    const uint8_t* cs = src + ((size_t)(blockIdx.x % 64) * 512 + wave * 128 + cp_row) * 64 + cp_chunk * 16;
    const int tm = (blockIdx.x / 16) % 16, tn = blockIdx.x % 16;
    const uint8_t* big_a = big + (size_t)(tm * 256) * 12288;
    const uint8_t* big_w = big + (size_t)4096 * 12288 + (size_t)(tn * BN) * 12288;
    const uint8_t* rsrc[kCpw];
    for (int c = 0; c < kCpw; ++c) {
        const int r16 = (wave * kCpw + c) * 16;
        rsrc[c] = (r16 < 256 ? big_a + (size_t)(r16 + cp_row) * 12288
                             : big_w + (size_t)(r16 - 256 + cp_row) * 12288) + cp_chunk * 16;
    }
    (void)cs;
    (void)rsrc;
    auto copy = [&](int it, int c) {
#if defined(__HIP_DEVICE_COMPILE__)
        LDS_AS void* dst = (LDS_AS void*)(&lds[(it + 3) & 3][0] + wave * kCpw * 1024 + c * 1024);
        if constexpr (RUNG >= 4)
            __builtin_amdgcn_global_load_lds(rsrc[c] + (size_t)(it % 192) * 64, dst, 16, 0, 0);
        else
            __builtin_amdgcn_global_load_lds(cs + (size_t)(it & 31) * kStage + c * 1024, dst, 16, 0, 0);
#endif
    };
    // k step s of K tile it on buffer b, reading step s + 1 into buffer b ^ 1
    auto step = [&](int it, int s, auto bt) {
        constexpr int b = decltype(bt)::value;
        const int ns = s ^ 1;
        const uint8_t* nbase = &lds[(ns == 0 ? it + 1 : it) & 3][0];
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int i = q / FN, j = q % FN;
            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[b][i], fb[b][j], acc[i][j], 0, 0, 0);
            if constexpr (RUNG >= 1)
                if (q < FM + FN) {
                    if (q < FM) fa[b ^ 1][q] = *reinterpret_cast<const v4i*>(nbase + offA[q] + ns * 32);
                    else fb[b ^ 1][q - FM] = *reinterpret_cast<const v4i*>(nbase + offB[q - FM] + ns * 32);
                }
            if constexpr (RUNG >= 3)
                if (s == 1 && q < kCpw) copy(it, q);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (RUNG >= 2)
            if (s == 0) {
                if constexpr (RUNG >= 3)
                    __builtin_amdgcn_s_waitcnt((kCpw & 15) | (7 << 4) | (0 << 8) | ((kCpw >> 4) << 14));
                else
                    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
                asm volatile("s_barrier" ::: "memory");
            }
    };
    const unsigned long long t0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
        step(it, 0, std::integral_constant<int, 0>{});
        step(it, 1, std::integral_constant<int, 1>{});
    }
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned long long t1 = __builtin_readcyclecounter(), r1 = __builtin_amdgcn_s_memrealtime();
    int res = 0;
    for (int i = 0; i < FM; ++i)
        for (int j = 0; j < FN; ++j)
            for (int e = 0; e < 16; ++e) res ^= acc[i][j][e];
    out[blockIdx.x * 256 + tid] = res;
    if (tid == 0) {
        clk[blockIdx.x * 2] = t1 - t0;
        clk[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

// The fp16 ring kernel's K loop (int8 weights, 128 x 128 per wave, 64-element
// K tiles of two 32-k pairs): per pair 32 v_mfma_f32_32x32x16_f16, 8 x and 4 W
// fragment reads for the next pair (double-buffered), per K tile one barrier
// and 12 one-KiB copies per wave from an L2-resident window.
// RUNG 1: MFMAs + reads; 2: + barrier; 3: + copies; 4: + the int8 -> f16
// conversion of the next pair's W fragments, one word per MFMA slot.
__device__ __forceinline__ v2h bits_half2(uint32_t u) {
    v2h h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}
template <int RUNG>
__global__ __launch_bounds__(256, 1) void ladder16(const uint8_t* __restrict__ src, int iters, float* out,
                                                   unsigned long long* clk) {
    constexpr int kStage = 256 * 128 + 256 * 64;
    constexpr int NB = 4, PER = 2 * NB * NB, NRA = 2 * NB, NR = 3 * NB;
    __shared__ __attribute__((aligned(1024))) uint8_t lds[3][kStage];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    for (int i = tid * 16; i < 3 * kStage; i += 256 * 16) {
        const uint32_t h = (uint32_t)(i + blockIdx.x * 7919) * 2654435761u;
        const v4i v = {(int)(h & 0x3bff3bff), (int)((h * 2246822519u) & 0x3bff3bff),
                       (int)((h * 3266489917u) & 0x3bff3bff), (int)((h ^ 0x9e3779b9u) & 0x3bff3bff)};
        *reinterpret_cast<v4i*>(&lds[0][0] + i) = v;
    }
    __syncthreads();
    const int wm = wave >> 1, wn = wave & 1;
    const int fr = lane & 31, fk = lane >> 5;
    int offA[NB], offB[NB];
    for (int i = 0; i < NB; ++i) {
        offA[i] = (wm * 128 + i * 32 + fr) * 128 + fk * 16;
        offB[i] = 256 * 128 + (wn * 128 + i * 32 + fr) * 64 + fk * 16;
    }
    v8h xa[2][NB][2], bh[2][NB][2];
    v4i xb[2][NB];
    for (int b = 0; b < 2; ++b)
        for (int i = 0; i < NB; ++i) {
            xa[b][i][0] = xa[b][i][1] = *reinterpret_cast<const v8h*>(&lds[0][0] + offA[i]);
            xb[b][i] = *reinterpret_cast<const v4i*>(&lds[0][0] + offB[i]);
            __builtin_memcpy(&bh[b][i][0], &xb[b][i], 16);
            bh[b][i][1] = bh[b][i][0];
        }
    v16f acc[NB][NB];
    for (int i = 0; i < NB; ++i)
        for (int j = 0; j < NB; ++j) acc[i][j] = v16f{};
    const int cp_row = lane >> 2, cp_chunk = lane & 3;
    const uint8_t* cs = src + ((size_t)(blockIdx.x % 64) * 768 + wave * 192 + cp_row) * 64 + cp_chunk * 16;
    (void)cs;
    auto copy = [&](int it, int c) {
#if defined(__HIP_DEVICE_COMPILE__)
        __builtin_amdgcn_global_load_lds(cs + (size_t)(it & 31) * kStage + c * 1024,
                                         (LDS_AS void*)(&lds[(it + 2) % 3][0] + wave * 12288 + c * 1024), 16, 0, 0);
#endif
    };
    auto pair = [&](int it, int s, auto bt) {
        constexpr int b = decltype(bt)::value;
        const int ns = s ^ 1;
        const uint8_t* nbase = &lds[(ns == 0 ? it + 1 : it) % 3][0];
#pragma unroll
        for (int q = 0; q < PER; ++q) {
            const int half = q / (NB * NB), r = q % (NB * NB), i = r / NB, j = r % NB;
            acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(xa[b][i][half], bh[b][j][half], acc[i][j], 0, 0, 0);
            if (q < NR) {
                if (q < NRA) {
                    const int bi = q >> 1, hh = q & 1;
                    xa[b ^ 1][bi][hh] =
                        *reinterpret_cast<const v8h*>(nbase + ((offA[bi] + ns * 64 + hh * 32) & (256 * 128 - 16)));
                } else {
                    xb[b ^ 1][q - NRA] = *reinterpret_cast<const v4i*>(nbase + offB[q - NRA] + ns * 32);
                }
            }
            if constexpr (RUNG >= 4) {
                const int cq = q - (NR + 2);
                if (cq >= 0 && cq < 4 * NB) {
                    const int cj = cq >> 2, w = cq & 3;
                    const uint32_t biased = (uint32_t)xb[b ^ 1][cj][w] ^ 0x80808080u;
                    const v2h k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
                    const v2h lo = bits_half2(__builtin_amdgcn_perm(0x64646464u, biased, 0x04010400u)) - k1152;
                    const v2h hi = bits_half2(__builtin_amdgcn_perm(0x64646464u, biased, 0x04030402u)) - k1152;
                    v8h& dst = bh[b ^ 1][cj][w >> 1];
                    const int e = (w & 1) * 4;
                    dst[e] = lo[0];
                    dst[e + 1] = lo[1];
                    dst[e + 2] = hi[0];
                    dst[e + 3] = hi[1];
                }
            }
            if constexpr (RUNG >= 3)
                if (s == 1 && q < 12) copy(it, q);
            __builtin_amdgcn_sched_barrier(0);
        }
        if constexpr (RUNG >= 2)
            if (s == 0) {
                if constexpr (RUNG >= 3)
                    __builtin_amdgcn_s_waitcnt((12 & 15) | (7 << 4) | (0 << 8));
                else
                    __builtin_amdgcn_s_waitcnt((15) | (7 << 4) | (0 << 8) | (3 << 14));
                asm volatile("s_barrier" ::: "memory");
            }
    };
    const unsigned long long t0 = __builtin_readcyclecounter(), r0 = __builtin_amdgcn_s_memrealtime();
    for (int it = 0; it < iters; ++it) {
        pair(it, 0, std::integral_constant<int, 0>{});
        pair(it, 1, std::integral_constant<int, 1>{});
    }
    __builtin_amdgcn_s_waitcnt(0);
    const unsigned long long t1 = __builtin_readcyclecounter(), r1 = __builtin_amdgcn_s_memrealtime();
    float res = 0;
    for (int i = 0; i < NB; ++i)
        for (int j = 0; j < NB; ++j)
            for (int e = 0; e < 16; ++e) res += acc[i][j][e];
    out[blockIdx.x * 256 + tid] = res;
    if (tid == 0) {
        clk[blockIdx.x * 2] = t1 - t0;
        clk[blockIdx.x * 2 + 1] = r1 - r0;
    }
}

template <typename F>
float time_launches(F launch) {
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
    return ms / 5;
}

double mean_cycles(const std::vector<unsigned long long>& c, int n) {
    double cyc = 0;
    for (int i = 0; i < n; ++i) cyc += (double)c[2 * i];
    return cyc / n;
}

template <int WN, int RUNG>
void run_ladder8_case(const uint8_t* src, const uint8_t* big, int* out, unsigned long long* clk, int cus) {
    const int iters = 1920;
    const float ms = time_launches(
        [&] { hipLaunchKernelGGL((ladder8<WN, RUNG>), dim3(cus), dim3(256), 0, 0, src, big, iters, out, clk); });
    std::vector<unsigned long long> c((size_t)cus * 2);
    CK(hipMemcpy(c.data(), clk, c.size() * 8, hipMemcpyDeviceToHost));
    const double ops = (double)cus * 4 * iters * 2.0 * 128 * WN * 64;
    const double mfma_cycles = (double)iters * 128 * WN * 64 * 2 / 2048.0;  // 2048 int8 ops / clk / SIMD
    const char* names[] = {"MFMAs only", "+ fragment reads", "+ barrier per K tile", "+ copies (L2-resident)",
                           "copies stream A/W from HBM"};
    printf("ladder8 wave 128x%d rung %d %-28s: %6.0f TOPS  clock %5.0f MHz  MFMA busy %5.1f%%\n", WN, RUNG,
           names[RUNG], ops / (ms * 1e-3) / 1e12, mean_mhz(c, cus), 100.0 * mfma_cycles / mean_cycles(c, cus));
    fflush(stdout);
}

template <int RUNG>
void run_ladder16_case(const uint8_t* src, float* out, unsigned long long* clk, int cus) {
    const int iters = 1000;
    const float ms =
        time_launches([&] { hipLaunchKernelGGL((ladder16<RUNG>), dim3(cus), dim3(256), 0, 0, src, iters, out, clk); });
    std::vector<unsigned long long> c((size_t)cus * 2);
    CK(hipMemcpy(c.data(), clk, c.size() * 8, hipMemcpyDeviceToHost));
    const double flops = (double)cus * 4 * iters * 2.0 * 128 * 128 * 64;
    const double mfma_cycles = (double)iters * 2.0 * 128 * 128 * 64 / 1024.0;  // 1024 f16 flops / clk / SIMD
    const char* names[] = {"", "MFMAs + fragment reads", "+ barrier per K tile", "+ copies (L2-resident)",
                           "+ int8->f16 conversion"};
    printf("ladder16 wave 128x128 rung %d %-24s: %6.0f TFLOP/s  clock %5.0f MHz  MFMA busy %5.1f%%\n", RUNG,
           names[RUNG], flops / (ms * 1e-3) / 1e12, mean_mhz(c, cus), 100.0 * mfma_cycles / mean_cycles(c, cus));
    fflush(stdout);
}

void run_ladder(int cus) {
    const size_t bytes = (size_t)64 * 768 * 64 + (size_t)32 * (256 * 128 + 256 * 64) + 4096;
    const size_t big_bytes = (size_t)(4096 + 16 * 256) * 12288;
    std::vector<uint8_t> h(big_bytes);
    uint32_t s = 1;
    for (auto& b : h) {
        s = s * 1664525u + 1013904223u;
        b = (uint8_t)(s >> 24);
    }
    uint8_t *src, *big;
    int* out;
    unsigned long long* clk;
    CK(hipMalloc(&src, bytes));
    CK(hipMalloc(&big, big_bytes));
    CK(hipMalloc(&out, (size_t)cus * 256 * 4));
    CK(hipMalloc(&clk, (size_t)cus * 16));
    CK(hipMemcpy(src, h.data(), bytes, hipMemcpyHostToDevice));
    CK(hipMemcpy(big, h.data(), big_bytes, hipMemcpyHostToDevice));
    for (int rep = 0; rep < 2; ++rep) {
        run_ladder8_case<96, 0>(src, big, out, clk, cus);
        run_ladder8_case<96, 1>(src, big, out, clk, cus);
        run_ladder8_case<96, 2>(src, big, out, clk, cus);
        run_ladder8_case<96, 3>(src, big, out, clk, cus);
        run_ladder8_case<96, 4>(src, big, out, clk, cus);
        run_ladder8_case<128, 3>(src, big, out, clk, cus);
        run_ladder8_case<128, 4>(src, big, out, clk, cus);
    }
    // fp16 operands: bytes with the f16 exponent field kept finite
    CK(hipMemset(src, 0x3b, bytes));
    for (int rep = 0; rep < 2; ++rep) {
        run_ladder16_case<1>(src, reinterpret_cast<float*>(out), clk, cus);
        run_ladder16_case<2>(src, reinterpret_cast<float*>(out), clk, cus);
        run_ladder16_case<3>(src, reinterpret_cast<float*>(out), clk, cus);
        run_ladder16_case<4>(src, reinterpret_cast<float*>(out), clk, cus);
    }
    CK(hipFree(src));
    CK(hipFree(big));
    CK(hipFree(out));
    CK(hipFree(clk));
}

// ---------------------------------------------------------------- read --
// Each thread issues U nontemporal 16-byte loads before using any; a block of
// T threads covers T * U consecutive chunks (load u of thread t: chunk
// block * T * U + u * T + t), the access pattern of the GEMV's weight loads.
typedef unsigned v4u __attribute__((ext_vector_type(4)));
template <int U>
__global__ __launch_bounds__(1024) void stream_read(const v4u* __restrict__ p, int64_t n16, unsigned* out) {
    const int64_t base = (int64_t)blockIdx.x * blockDim.x * U + threadIdx.x;
    v4u v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        int64_t i = base + (int64_t)u * blockDim.x;
        i = i < n16 ? i : n16 - 1;
        v[u] = __builtin_nontemporal_load(p + i);
    }
    unsigned x = 0;
#pragma unroll
    for (int u = 0; u < U; ++u) x ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (x == 0x12345678u) out[0] = x;  // keeps the loads
}

template <int U>
void run_read_case(const v4u* buf, int64_t n16, int copies, unsigned* out, hipStream_t s, int T) {
    const int64_t grid = (n16 + (int64_t)T * U - 1) / ((int64_t)T * U);
    const int iters = copies * 10;
    hipGraph_t g;
    hipGraphExec_t ge;
    CK(hipStreamBeginCapture(s, hipStreamCaptureModeGlobal));
    for (int i = 0; i < iters; ++i)
        hipLaunchKernelGGL((stream_read<U>), dim3((unsigned)grid), dim3(T), 0, s, buf + (int64_t)(i % copies) * n16,
                           n16, out);
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
    printf("read 58.7 MB per launch, %2d loads per thread, block %4d, grid %6lld: %6.2f us  %5.0f GB/s\n", U, T,
           (long long)grid, us, n16 * 16 / us / 1e3);
    fflush(stdout);
    CK(hipGraphExecDestroy(ge));
    CK(hipGraphDestroy(g));
}

void run_read() {
    const int64_t bytes = 4096LL * 14336, n16 = bytes / 16;
    const int copies = 19;
    v4u* buf;
    unsigned* out;
    CK(hipMalloc(&buf, bytes * copies));
    CK(hipMalloc(&out, 64));
    CK(hipMemset(buf, 1, bytes * copies));
    hipStream_t s;
    CK(hipStreamCreate(&s));
    for (int T : {256, 512, 1024}) {
        run_read_case<1>(buf, n16, copies, out, s, T);
        run_read_case<2>(buf, n16, copies, out, s, T);
        run_read_case<4>(buf, n16, copies, out, s, T);
        run_read_case<8>(buf, n16, copies, out, s, T);
        run_read_case<16>(buf, n16, copies, out, s, T);
    }
    CK(hipStreamDestroy(s));
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
