// Per-row dynamic symmetric int8 quantisation for gfx950.
//
// Semantics: crates/omni-kernel/src/int8_matmul.rs:23-118 (quantize_rows,
// quantize_i8) and the host twin crates/omni-kernel/src/int8_host.rs:31-39.
//   row_scale = max(max|x| / 127, 1e-30)   (f32, IEEE division)
//   code      = clamp(sign(x) * floor(|x / row_scale| + 0.5), -128, 127)
//   sum       = sum of the row's codes
//
// Design: one 256-lane workgroup per row. Pass 1 streams the row once for the
// peak (wave max over DPP/shuffles, then 4 partials through LDS). Pass 2
// streams it again — the row was just read, so this pass hits L2 — divides,
// rounds and writes the codes as packed little-endian int8 words. HBM traffic
// is one read of x and one write of the codes: the kernel is HBM-bound.
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
    peak = wave_max(peak);
    if (lane == 0) s_peak[wave] = peak;
    __syncthreads();
    peak = fmaxf(fmaxf(s_peak[0], s_peak[1]), fmaxf(s_peak[2], s_peak[3]));
    float row_scale = peak / 127.0f;
    // `!(a > b)` also catches a NaN peak, like Rust's f32::max with 1e-30.
    if (!(row_scale > 1.0e-30f)) row_scale = 1.0e-30f;

    int local = 0;
    uint8_t* dst = codes + row * width;
    for (int64_t c = tid; c < chunks; c += 256) {
        float v[VEC];
        load_row_chunk<T, VEC, ALIGNED>(src + c * VEC, v);
        u32 words[VEC / 4];
#pragma unroll
        for (int w = 0; w < VEC / 4; ++w) {
            u32 word = 0;
#pragma unroll
            for (int b = 0; b < 4; ++b) {
                int q = quantize_code(v[4 * w + b] / row_scale);
                local += q;
                word |= (u32)(q & 255) << (8 * b);
            }
            words[w] = word;
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
