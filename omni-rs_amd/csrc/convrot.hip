// ConvRot activation rotation fused into per-row int8 quantisation, gfx950.
//
// Semantics (crates/qwen-image/src/convrot.rs:81-92, 113-149, then
// crates/omni-kernel/src/int8_matmul.rs:23-118):
//   r[row][256 g + c] = sum_j x[row][256 g + j] * H[j][c]          (f32)
//   H = 2^-4 * (H4 (x) H4 (x) H4 (x) H4),  H4[a][b] = -1 iff a ^ b == 3
// followed by the per-row quantisation of r exactly as quantize.hip does it
// (peak, row_scale = max(peak / 127, 1e-30), IEEE quotient, round half away).
// The reference multiplies by the 256 x 256 matrix (an f32 matmul of
// [rows * K / 256, 256] by H); here the same linear map is applied as four
// radix-4 stages, one per base-4 digit of the index within the group: the
// Kronecker factors act on distinct digits. Each stage is the 4-point
// transform y_a = s - 2 x_(3-a), s = x0 + x1 + x2 + x3 (H4 is all ones except
// -1 where a ^ b == 3). The f32 rounding differs from a 256-term dot in any
// summation order by a few units in the last place, as the reference's own
// lowerings (CPU and GPU matmul) differ from each other.
//
// Layout: one wavefront per row; a 256-element group spreads over 8 lanes
// (sub = lane & 7) and lane `sub` holds v[k][e] = element 64 k + 8 sub + e,
// k, e in [0, 4) x [0, 8): four 16-byte (f16) loads of 8 consecutive
// elements. Element-index bits 0-1 (digit 0) and 6-7 (digit 3) are in
// registers, bit 2 in registers and bit 3 across lane pairs (digit 1), bits
// 4-5 across lanes 2 and 4 apart (digit 2): every shuffle stays inside an
// aligned group of 8 lanes. A wave rotates 8 groups at a time; rows of up to
// 16 groups keep the rotated values in registers between the peak and the
// code pass, longer rows rotate twice (the second read hits the caches).
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"

namespace omni {

namespace {

constexpr int kGroup = 256;

// y = H4 x in place.
__device__ __forceinline__ void h4(float& x0, float& x1, float& x2, float& x3) {
    const float s = (x0 + x1) + (x2 + x3);
    const float y0 = __builtin_fmaf(-2.0f, x3, s);  // 2 x is exact: one rounding
    const float y1 = __builtin_fmaf(-2.0f, x2, s);
    const float y2 = __builtin_fmaf(-2.0f, x1, s);
    const float y3 = __builtin_fmaf(-2.0f, x0, s);
    x0 = y0;
    x1 = y1;
    x2 = y2;
    x3 = y3;
}

// Eight consecutive elements at p (16-byte aligned) as f32.
template <typename T>
__device__ __forceinline__ void load8(const T* p, float (&v)[8]) {
    constexpr int kLoads = 8 * (int)sizeof(T) / 16;
    uint4 raw[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) raw[i] = reinterpret_cast<const uint4*>(p)[i];
    T tmp[8];
    __builtin_memcpy(tmp, raw, sizeof(tmp));
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = (float)tmp[i];
}

// The group starting at g (nullptr: an idle slot, zeros) rotated into v. All
// 64 lanes must call it together (it shuffles).
template <typename T>
__device__ __forceinline__ void rotate_group(const T* g, int sub, float (&v)[4][8]) {
    if (g) {
#pragma unroll
        for (int k = 0; k < 4; ++k) load8<T>(g + 64 * k + 8 * sub, v[k]);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) v[k][e] = 0.0f;
    }
    // Digit 0: element bits 0-1.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        h4(v[k][0], v[k][1], v[k][2], v[k][3]);
        h4(v[k][4], v[k][5], v[k][6], v[k][7]);
    }
    // Digit 3: element bits 6-7 (k).
#pragma unroll
    for (int e = 0; e < 8; ++e) h4(v[0][e], v[1][e], v[2][e], v[3][e]);
    // Digit 1: bit 2 is e's bit 2, bit 3 is the lane's bit 0. The partner of
    // digit value a is 3 - a: both bits flip, so it is the other lane's
    // other half.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float a0 = v[k][e], a1 = v[k][e + 4];
            const float t = a0 + a1;
            const float s = t + __shfl_xor(t, 1, kWave);
            const float p0 = __shfl_xor(a1, 1, kWave);
            const float p1 = __shfl_xor(a0, 1, kWave);
            v[k][e] = __builtin_fmaf(-2.0f, p0, s);
            v[k][e + 4] = __builtin_fmaf(-2.0f, p1, s);
        }
    }
    // Digit 2: element bits 4-5 are the lane's bits 1-2.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const float x = v[k][e];
            float s = x + __shfl_xor(x, 2, kWave);
            s = s + __shfl_xor(s, 4, kWave);
            v[k][e] = __builtin_fmaf(-2.0f, __shfl_xor(x, 6, kWave), s);
        }
    }
    // 2^-4 (log4 of 256 stages of an unnormalised H4): exact.
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 8; ++e) v[k][e] *= 0.0625f;
}

// HOLD > 0: the row's groups (at most 8 * HOLD) stay in registers; HOLD == 0:
// any number of groups, rotated once for the peak and again for the codes.
template <typename T, int HOLD>
__global__ __launch_bounds__(256) void convrot_quantize_kernel(
    const T* __restrict__ x, int64_t rows, int64_t width, int64_t ld, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out, int32_t* __restrict__ sum_out) {
    const int lane = threadIdx.x & 63;
    const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (row >= rows) return;  // the row is wave-uniform: whole waves exit
    const int sub = lane & 7, slot = lane >> 3;
    const int groups = (int)(width / kGroup);
    const int passes = (groups + 7) / 8;
    const T* src = x + row * ld;
    uint8_t* dst = codes + row * width;
    auto group_ptr = [&](int p) -> const T* {
        const int g = p * 8 + slot;
        return g < groups ? src + (int64_t)g * kGroup : nullptr;
    };
    auto peak_of = [&](const float (&v)[4][8], float peak) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 8; ++e) peak = fmaxf(peak, __builtin_fabsf(v[k][e]));
        return peak;
    };
    int local = 0;
    auto emit = [&](int p, const float (&v)[4][8], float s, float y, bool tiny) {
        const int g = p * 8 + slot;
        if (g >= groups) return;
        uint8_t* out = dst + (int64_t)g * kGroup + 8 * sub;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint2 w;
            if (tiny) {
                w.x = pack4<true>(&v[k][0], s, y, local);
                w.y = pack4<true>(&v[k][4], s, y, local);
            } else {
                w.x = pack4<false>(&v[k][0], s, y, local);
                w.y = pack4<false>(&v[k][4], s, y, local);
            }
            *reinterpret_cast<uint2*>(out + 64 * k) = w;
        }
    };

    float peak = 0.0f;
    float s, y;
    bool tiny;
    if constexpr (HOLD > 0) {
        float v[HOLD][4][8];
#pragma unroll
        for (int p = 0; p < HOLD; ++p) {
            if (p < passes) {
                rotate_group<T>(group_ptr(p), sub, v[p]);
                peak = peak_of(v[p], peak);
            }
        }
        peak = wave_max(peak);
        s = row_scale_of(peak);
        y = 1.0f / s;
        tiny = s < 0x1p-90f;
#pragma unroll
        for (int p = 0; p < HOLD; ++p)
            if (p < passes) emit(p, v[p], s, y, tiny);
    } else {
        float v[4][8];
        for (int p = 0; p < passes; ++p) {
            rotate_group<T>(group_ptr(p), sub, v);
            peak = peak_of(v, peak);
        }
        peak = wave_max(peak);
        s = row_scale_of(peak);
        y = 1.0f / s;
        tiny = s < 0x1p-90f;
        for (int p = 0; p < passes; ++p) {
            rotate_group<T>(group_ptr(p), sub, v);
            emit(p, v, s, y, tiny);
        }
    }
    if (sum_out) {
        local = wave_sum_i32(local);
        if (lane == 0) sum_out[row] = local;
    }
    if (lane == 0) scale_out[row] = s;
}

template <typename T>
hipError_t launch_convrot_typed(const T* x, int64_t rows, int64_t width, int64_t ld,
                                uint8_t* codes, float* scale, int32_t* sum, hipStream_t stream) {
    const int64_t passes = (width / kGroup + 7) / 8;
    dim3 grid((unsigned)((rows + 3) / 4)), block(256);
    if (passes <= 1)
        hipLaunchKernelGGL((convrot_quantize_kernel<T, 1>), grid, block, 0, stream, x, rows, width,
                           ld, codes, scale, sum);
    else if (passes <= 2)
        hipLaunchKernelGGL((convrot_quantize_kernel<T, 2>), grid, block, 0, stream, x, rows, width,
                           ld, codes, scale, sum);
    else
        hipLaunchKernelGGL((convrot_quantize_kernel<T, 0>), grid, block, 0, stream, x, rows, width,
                           ld, codes, scale, sum);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_convrot_quantize(const void* x, bool x_is_f16, int64_t rows, int64_t width,
                                   int64_t ld, uint8_t* codes, float* scale, int32_t* sum,
                                   hipStream_t stream) {
    if (rows == 0) return hipSuccess;
    if (x_is_f16)
        return launch_convrot_typed<_Float16>(static_cast<const _Float16*>(x), rows, width, ld,
                                              codes, scale, sum, stream);
    return launch_convrot_typed<float>(static_cast<const float*>(x), rows, width, ld, codes, scale,
                                       sum, stream);
}

}  // namespace omni
