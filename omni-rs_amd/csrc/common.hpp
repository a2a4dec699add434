// Shared device helpers for the gfx950 int8 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace omni {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef _Float16 v2h __attribute__((ext_vector_type(2)));
typedef unsigned int u32;

constexpr int kWave = 64;

// Round half away from zero, clamp to [-128, 127]; a NaN gives 0.
// crates/omni-kernel/src/int8_matmul.rs:102-118 (quantize_i8) and
// crates/omni-kernel/src/int8_host.rs:3-10 (round_half_away).
__device__ __forceinline__ int quantize_code(float value) {
    float magnitude = __builtin_fabsf(value);
    float rounded = __builtin_floorf(magnitude + 0.5f);
    float signed_v = value >= 0.0f ? rounded : -rounded;
    // NaN compares false everywhere and falls to 0.
    if (!(signed_v == signed_v)) return 0;
    signed_v = signed_v > 127.0f ? 127.0f : signed_v;
    signed_v = signed_v < -128.0f ? -128.0f : signed_v;
    return (int)signed_v;
}

// Sum of the four sign-extended bytes of a word.
__device__ __forceinline__ int sum4(u32 word) {
    return (int)(int8_t)(word) + (int)(int8_t)(word >> 8) + (int)(int8_t)(word >> 16) +
           (int)(int8_t)(word >> 24);
}

// Wave-wide reductions over 64 lanes.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
    return v;
}
__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}
__device__ __forceinline__ float wave_sum_f32(float v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

}  // namespace omni
