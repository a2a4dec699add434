// Per-row dynamic symmetric int8 quantisation for gfx950.
//
// Semantics: crates/omni-kernel/src/int8_matmul.rs:23-118 (quantize_rows,
// quantize_i8) and the host twin crates/omni-kernel/src/int8_host.rs:31-39.
//   row_scale = max(max|x| / 127, 1e-30)   (f32, IEEE division)
//   code      = clamp(sign(x) * floor(|x / row_scale| + 0.5), -128, 127)
//   sum       = sum of the row's codes
//
// Design: rows of up to 2048 elements take one wavefront each, rows of up to
// 16384 one 256-lane workgroup each; either way the row is read once into
// registers (16-element chunks, 128-bit loads), the peak is reduced across
// the wave (and across the 4 waves through LDS), and the codes are written as
// packed little-endian int8 words: HBM traffic is one read of x and one write
// of the codes. Longer or misaligned rows take a two-pass variant whose
// second pass re-reads the row from L2.
//
// The division x / row_scale must be IEEE (correctly rounded): a code flips
// when a quotient near k + 0.5 rounds the other way. It is computed as
// q0 = x * y, r = fma(-q0, s, x), q = fma(r, y, q0) with y = RN(1 / s)
// (Markstein's correction step), which returns RN(x / s) whenever the
// residual r is exact; rows with s < 2^-90 (where r can leave the normal
// range) use the hardware-expanded IEEE division instead.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace omni {

namespace {

template <typename T>
__device__ __forceinline__ float to_f32(T v) { return (float)v; }

// Loads VEC consecutive elements starting at p into f32 registers.
template <typename T, int VEC, bool ALIGNED>
__device__ __forceinline__ void load_row_chunk(const T* __restrict__ p, float (&v)[VEC]) {
    if constexpr (ALIGNED) {
        constexpr int kBytes = VEC * (int)sizeof(T);
        static_assert(kBytes % 16 == 0 || kBytes == 8, "vector width");
        if constexpr (kBytes == 8) {
            uint2 raw = *reinterpret_cast<const uint2*>(p);
            T tmp[VEC];
            __builtin_memcpy(tmp, &raw, 8);
#pragma unroll
            for (int i = 0; i < VEC; ++i) v[i] = to_f32(tmp[i]);
        } else {
            constexpr int kLoads = kBytes / 16;
            uint4 raw[kLoads];
#pragma unroll
            for (int i = 0; i < kLoads; ++i) raw[i] = reinterpret_cast<const uint4*>(p)[i];
            T tmp[VEC];
            __builtin_memcpy(tmp, raw, kBytes);
#pragma unroll
            for (int i = 0; i < VEC; ++i) v[i] = to_f32(tmp[i]);
        }
    } else {
#pragma unroll
        for (int i = 0; i < VEC; ++i) v[i] = to_f32(p[i]);
    }
}


// Block-wide max of one value per thread (256 threads, 4 waves).
__device__ __forceinline__ float block_max(float v, float* s_red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    return fmaxf(fmaxf(s_red[0], s_red[1]), fmaxf(s_red[2], s_red[3]));
}

// The same over NW waves of one workgroup.
template <int NW>
__device__ __forceinline__ float block_max_n(float v, float* s_red) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    v = wave_max(v);
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    float m = s_red[0];
#pragma unroll
    for (int w = 1; w < NW; ++w) m = fmaxf(m, s_red[w]);
    return m;
}

// Single-read variant: each of the TPB threads owns chunks tid + TPB*j
// (j < CPT) of 16 elements, held in registers between the peak and the code
// pass. KF > 0 builds it for width == KF == 16 * TPB * CPT: every chunk
// index is in range, with no predicate.
template <typename T, int CPT, int KF = 0, int TPB = 256>
__global__ __launch_bounds__(256) void quantize_rows_reg_kernel(
    const T* __restrict__ x, int64_t width, int64_t ld, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out, int32_t* __restrict__ sum_out) {
    static_assert(TPB % 64 == 0 && TPB <= 256, "whole waves, at most four");
    static_assert(KF == 0 || KF == 16 * TPB * CPT, "KF covers the lanes exactly");
    constexpr int NW = TPB / 64;
    __shared__ float s_peak[NW];
    __shared__ int s_sum[NW];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const T* src = x + row * ld;
    const int chunks = KF > 0 ? KF / 16 : (int)(width / 16);
    float v[CPT][16];
    float peak = 0.0f;
#pragma unroll
    for (int j = 0; j < CPT; ++j) {
        const int c = tid + TPB * j;
        if (KF > 0 || c < chunks) {
            load_row_chunk<T, 16, true>(src + (int64_t)c * 16, v[j]);
#pragma unroll
            for (int i = 0; i < 16; ++i) peak = fmaxf(peak, __builtin_fabsf(v[j][i]));
        }
    }
    peak = block_max_n<NW>(peak, s_peak);
    const float s = row_scale_of(peak);
    const float y = 1.0f / s;
    const bool tiny = s < 0x1p-90f;
    int local = 0;
    uint8_t* dst = codes + row * width;
    auto emit = [&](auto tiny_tag) {
        constexpr bool kTiny = decltype(tiny_tag)::value;
#pragma unroll
        for (int j = 0; j < CPT; ++j) {
            const int c = tid + TPB * j;
            if (KF > 0 || c < chunks) {
                uint4 w;
                w.x = pack4<kTiny>(&v[j][0], s, y, local);
                w.y = pack4<kTiny>(&v[j][4], s, y, local);
                w.z = pack4<kTiny>(&v[j][8], s, y, local);
                w.w = pack4<kTiny>(&v[j][12], s, y, local);
                *reinterpret_cast<uint4*>(dst + (int64_t)c * 16) = w;
            }
        }
    };
    if (tiny) emit(std::true_type{}); else emit(std::false_type{});
    if (sum_out) {
        local = wave_sum_i32(local);
        if ((tid & 63) == 0) s_sum[tid >> 6] = local;
        __syncthreads();
        if (tid == 0) {
            int total = 0;
#pragma unroll
            for (int w = 0; w < NW; ++w) total += s_sum[w];
            sum_out[row] = total;
        }
    }
    if (tid == 0) scale_out[row] = s;
}

// Wave-per-row variant: each wave quantises one row on its own (no LDS, no
// barrier), lane l owning chunks l + 64*j (j < CPW) of 16 elements, kept in
// registers in the input type between the peak and the code pass.
template <typename T, int CPW>
__global__ __launch_bounds__(256) void quantize_rows_wave_kernel(
    const T* __restrict__ x, int64_t rows, int64_t width, int64_t ld, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out, int32_t* __restrict__ sum_out) {
    constexpr int kWords = 16 * (int)sizeof(T) / 16;  // uint4 per 16-element chunk
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // whole wave exits together
    const T* src = x + row * ld;
    const int chunks = (int)(width / 16);
    uint4 raw[CPW][kWords];
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        const int c = lane + 64 * j;
        if (c < chunks) {
#pragma unroll
            for (int w = 0; w < kWords; ++w)
                raw[j][w] = reinterpret_cast<const uint4*>(src + (int64_t)c * 16)[w];
        }
    }
    auto unpack = [&](int j, float (&v)[16]) {
        T tmp[16];
        __builtin_memcpy(tmp, raw[j], sizeof(tmp));
#pragma unroll
        for (int i = 0; i < 16; ++i) v[i] = to_f32(tmp[i]);
    };
    float peak = 0.0f;
#pragma unroll
    for (int j = 0; j < CPW; ++j) {
        if (lane + 64 * j < chunks) {
            float v[16];
            unpack(j, v);
#pragma unroll
            for (int i = 0; i < 16; ++i) peak = fmaxf(peak, __builtin_fabsf(v[i]));
        }
    }
    peak = wave_max(peak);
    const float s = row_scale_of(peak);
    const float y = 1.0f / s;
    const bool tiny = s < 0x1p-90f;
    int local = 0;
    uint8_t* dst = codes + row * width;
    auto emit = [&](auto tiny_tag) {
        constexpr bool kTiny = decltype(tiny_tag)::value;
#pragma unroll
        for (int j = 0; j < CPW; ++j) {
            const int c = lane + 64 * j;
            if (c < chunks) {
                float v[16];
                unpack(j, v);
                uint4 w;
                w.x = pack4<kTiny>(&v[0], s, y, local);
                w.y = pack4<kTiny>(&v[4], s, y, local);
                w.z = pack4<kTiny>(&v[8], s, y, local);
                w.w = pack4<kTiny>(&v[12], s, y, local);
                *reinterpret_cast<uint4*>(dst + (int64_t)c * 16) = w;
            }
        }
    };
    if (tiny) emit(std::true_type{}); else emit(std::false_type{});
    if (sum_out) {
        local = wave_sum_i32(local);
        if (lane == 0) sum_out[row] = local;
    }
    if (lane == 0) scale_out[row] = s;
}

template <typename T, int VEC, bool ALIGNED>
__global__ __launch_bounds__(256) void quantize_rows_kernel(
    const T* __restrict__ x, int64_t width, int64_t ld, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out, int32_t* __restrict__ sum_out) {
    __shared__ float s_peak[4];
    __shared__ int s_sum[4];
    const int64_t row = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const T* src = x + row * ld;
    const int64_t chunks = width / VEC;

    float peak = 0.0f;
    for (int64_t c = tid; c < chunks; c += 256) {
        float v[VEC];
        load_row_chunk<T, VEC, ALIGNED>(src + c * VEC, v);
#pragma unroll
        for (int i = 0; i < VEC; ++i) peak = fmaxf(peak, __builtin_fabsf(v[i]));
    }
    peak = block_max(peak, s_peak);
    const float row_scale = row_scale_of(peak);
    const float y = 1.0f / row_scale;
    const bool tiny = row_scale < 0x1p-90f;

    int local = 0;
    uint8_t* dst = codes + row * width;
    for (int64_t c = tid; c < chunks; c += 256) {
        float v[VEC];
        load_row_chunk<T, VEC, ALIGNED>(src + c * VEC, v);
        u32 words[VEC / 4];
        if (tiny) {
#pragma unroll
            for (int w = 0; w < VEC / 4; ++w) words[w] = pack4<true>(&v[4 * w], row_scale, y, local);
        } else {
#pragma unroll
            for (int w = 0; w < VEC / 4; ++w) words[w] = pack4<false>(&v[4 * w], row_scale, y, local);
        }
        if constexpr (ALIGNED && VEC == 16) {
            *reinterpret_cast<uint4*>(dst + c * VEC) = make_uint4(words[0], words[1], words[2], words[3]);
        } else if constexpr (ALIGNED && VEC == 8) {
            *reinterpret_cast<uint2*>(dst + c * VEC) = make_uint2(words[0], words[1]);
        } else {
            // codes is an int32 buffer and width % 4 == 0: word stores are aligned.
#pragma unroll
            for (int w = 0; w < VEC / 4; ++w) reinterpret_cast<u32*>(dst + c * VEC)[w] = words[w];
        }
    }
    if (sum_out) {
        local = wave_sum_i32(local);
        if (lane == 0) s_sum[wave] = local;
        __syncthreads();
        if (tid == 0) sum_out[row] = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
    }
    if (tid == 0) scale_out[row] = row_scale;
}

template <typename T, int VEC>
hipError_t launch_vec(const T* x, int64_t rows, int64_t width, int64_t ld, uint8_t* codes,
                      float* scale, int32_t* sum, bool aligned, hipStream_t stream) {
    if (aligned)
        hipLaunchKernelGGL((quantize_rows_kernel<T, VEC, true>), dim3((unsigned)rows), dim3(256), 0,
                           stream, x, width, ld, codes, scale, sum);
    else
        hipLaunchKernelGGL((quantize_rows_kernel<T, VEC, false>), dim3((unsigned)rows), dim3(256), 0,
                           stream, x, width, ld, codes, scale, sum);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_typed(const T* x, int64_t rows, int64_t width, int64_t ld, uint8_t* codes,
                        float* scale, int32_t* sum, hipStream_t stream) {
    const uintptr_t base = reinterpret_cast<uintptr_t>(x);
    const uintptr_t cbase = reinterpret_cast<uintptr_t>(codes);
    // Vector loads need the row starts aligned to the load width; vector
    // stores need the code rows aligned to VEC bytes.
    auto aligned_for = [&](int vec) {
        const int64_t in_bytes = vec * (int64_t)sizeof(T);
        const int64_t align = in_bytes >= 16 ? 16 : in_bytes;
        return base % align == 0 && (ld * (int64_t)sizeof(T)) % align == 0 && cbase % vec == 0;
    };
    // One wave per row up to 2 chunks per lane (2048 elements); wider rows
    // (up to 16384) take a workgroup per row, 4 waves holding the row, which
    // measured faster on MI355X than one wave per row from 3072 f16 on (4096
    // rows: 10.2 / 11.7 us against 10.6 / 14.1 at 3072 / 4096; 15 % at 12288)
    // and slower at 1536 (8.5 against 7.4 us).
    if (width % 16 == 0 && width <= 2048 && aligned_for(16)) {
        const int cpw = (int)((width / 16 + 63) / 64);
        dim3 grid((unsigned)((rows + 3) / 4)), block(256);
#define OMNI_QWAVE(n) hipLaunchKernelGGL((quantize_rows_wave_kernel<T, n>), grid, block, 0, stream, x, rows, width, ld, codes, scale, sum)
        if (cpw <= 1) OMNI_QWAVE(1);
        else OMNI_QWAVE(2);
#undef OMNI_QWAVE
        return hipGetLastError();
    }
    if (width % 16 == 0 && width <= 16384 && aligned_for(16)) {
        const int cpt = (int)((width / 16 + 255) / 256);
        dim3 grid((unsigned)rows), block(256);
        // The bench model's widths, built with every lane owning whole
        // chunks (3072: three waves of one chunk, not four with one idle).
        if (width == 3072) {
            hipLaunchKernelGGL((quantize_rows_reg_kernel<T, 1, 3072, 192>), grid, dim3(192), 0, stream, x, width, ld,
                               codes, scale, sum);
            return hipGetLastError();
        }
        if (width == 12288) {
            hipLaunchKernelGGL((quantize_rows_reg_kernel<T, 3, 12288, 256>), grid, block, 0, stream, x, width, ld,
                               codes, scale, sum);
            return hipGetLastError();
        }
        switch (cpt) {
            case 1: hipLaunchKernelGGL((quantize_rows_reg_kernel<T, 1>), grid, block, 0, stream, x, width, ld, codes, scale, sum); break;
            case 2: hipLaunchKernelGGL((quantize_rows_reg_kernel<T, 2>), grid, block, 0, stream, x, width, ld, codes, scale, sum); break;
            case 3: hipLaunchKernelGGL((quantize_rows_reg_kernel<T, 3>), grid, block, 0, stream, x, width, ld, codes, scale, sum); break;
            default: hipLaunchKernelGGL((quantize_rows_reg_kernel<T, 4>), grid, block, 0, stream, x, width, ld, codes, scale, sum); break;
        }
        return hipGetLastError();
    }
    if (width % 16 == 0)
        return launch_vec<T, 16>(x, rows, width, ld, codes, scale, sum, aligned_for(16), stream);
    if (width % 8 == 0)
        return launch_vec<T, 8>(x, rows, width, ld, codes, scale, sum, aligned_for(8), stream);
    return launch_vec<T, 4>(x, rows, width, ld, codes, scale, sum, aligned_for(4), stream);
}

}  // namespace

hipError_t launch_quantize_rows(const void* x, bool x_is_f16, int64_t rows, int64_t width,
                                int64_t ld, uint8_t* codes, float* scale, int32_t* sum,
                                hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (x_is_f16)
        return launch_typed<_Float16>(static_cast<const _Float16*>(x), rows, width, ld, codes,
                                      scale, sum, stream);
    return launch_typed<float>(static_cast<const float*>(x), rows, width, ld, codes, scale, sum,
                               stream);
}

}  // namespace omni
