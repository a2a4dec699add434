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
// Layout: a 256-element group spreads over 4 lanes (sub = lane & 3) and
// lane `sub` holds v[k][e] = element 64 k + 16 sub + e, k in [0, 4), e in
// [0, 16): element-index bits 0-3 and 6-7 (digits 0, 1 and 3) are in
// registers, bits 4-5 (digit 2) are the lane's bits 0-1, so the one
// cross-lane stage is three quad permutes (DPP, no LDS) per value. A wave
// rotates 16 groups at once; a row of up to 16 groups takes one wave, up to
// 32 two waves, up to 64 four waves (the peak is then reduced through LDS),
// and holds its rotated values in registers between the peak and the code
// pass. Wider rows rotate each group twice (the second read hits the caches).
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

// The value of lane (lane ^ X) within its quad, X in 1..3 (DPP quad_perm).
template <int X>
__device__ __forceinline__ float quad_xor(float v) {
    constexpr int kCtrl = X == 1 ? 0xB1 : X == 2 ? 0x4E : 0x1B;  // [1,0,3,2] [2,3,0,1] [3,2,1,0]
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), kCtrl, 0xF, 0xF, true));
}

// Sixteen consecutive elements at p (16-byte aligned) as f32.
template <typename T>
__device__ __forceinline__ void load16(const T* p, float (&v)[16]) {
    constexpr int kLoads = 16 * (int)sizeof(T) / 16;
    uint4 raw[kLoads];
#pragma unroll
    for (int i = 0; i < kLoads; ++i) raw[i] = reinterpret_cast<const uint4*>(p)[i];
    T tmp[16];
    __builtin_memcpy(tmp, raw, sizeof(tmp));
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = (float)tmp[i];
}

// The group starting at g (nullptr: an idle slot, zeros) rotated into v. All
// lanes of a quad must call it together (digit 2 permutes within quads).
template <typename T>
__device__ __forceinline__ void rotate_group(const T* g, int sub, float (&v)[4][16]) {
    if (g) {
#pragma unroll
        for (int k = 0; k < 4; ++k) load16<T>(g + 64 * k + 16 * sub, v[k]);
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 16; ++e) v[k][e] = 0.0f;
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        // Digit 0: element bits 0-1.
#pragma unroll
        for (int q = 0; q < 4; ++q) h4(v[k][4 * q], v[k][4 * q + 1], v[k][4 * q + 2], v[k][4 * q + 3]);
        // Digit 1: element bits 2-3.
#pragma unroll
        for (int r = 0; r < 4; ++r) h4(v[k][r], v[k][r + 4], v[k][r + 8], v[k][r + 12]);
    }
    // Digit 3: element bits 6-7 (k).
#pragma unroll
    for (int e = 0; e < 16; ++e) h4(v[0][e], v[1][e], v[2][e], v[3][e]);
    // Digit 2: element bits 4-5 are the lane's bits 0-1; the partner of digit
    // value a is 3 - a, the lane three apart within the quad.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float x = v[k][e];
            float s = x + quad_xor<1>(x);
            s = s + quad_xor<2>(s);
            v[k][e] = __builtin_fmaf(-2.0f, quad_xor<3>(x), s);
        }
    }
    // 2^-4 (four stages of the unnormalised H4): exact.
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 16; ++e) v[k][e] *= 0.0625f;
}

// WPR waves per row (1, 2 or 4; 4 / WPR rows per 256-thread workgroup).
// Every wave rotates 16 groups per pass; HOLD: the row fits in one pass and
// stays in registers, else each group is rotated for the peak and again for
// the codes.
template <typename T, int WPR, bool HOLD>
__global__ __launch_bounds__(256) void convrot_quantize_kernel(
    const T* __restrict__ x, int64_t rows, int64_t width, int64_t ld, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out, int32_t* __restrict__ sum_out) {
    __shared__ float s_peak[4];
    __shared__ int s_sum[4];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t row_raw = (int64_t)blockIdx.x * (4 / WPR) + wave / WPR;
    // With one wave per row a wave past the last row exits; otherwise every
    // wave stays for the barriers and only a valid row is stored.
    if (WPR == 1 && row_raw >= rows) return;
    const bool valid = row_raw < rows;
    const int64_t row = valid ? row_raw : rows - 1;
    const int part = wave % WPR;
    const int sub = lane & 3, slot = lane >> 2;
    const int groups = (int)(width / kGroup);
    const int passes = (groups + 16 * WPR - 1) / (16 * WPR);
    const T* src = x + row * ld;
    uint8_t* dst = codes + row * width;
    auto group_ptr = [&](int p) -> const T* {
        const int g = (p * WPR + part) * 16 + slot;
        return g < groups ? src + (int64_t)g * kGroup : nullptr;
    };
    auto peak_of = [&](const float (&v)[4][16], float peak) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int e = 0; e < 16; ++e) peak = fmaxf(peak, __builtin_fabsf(v[k][e]));
        return peak;
    };
    int local = 0;
    auto emit = [&](int p, const float (&v)[4][16], float s, float y, bool tiny) {
        const int g = (p * WPR + part) * 16 + slot;
        if (!valid || g >= groups) return;
        uint8_t* out = dst + (int64_t)g * kGroup + 16 * sub;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            uint4 w;
            if (tiny) {
                w.x = pack4<true>(&v[k][0], s, y, local);
                w.y = pack4<true>(&v[k][4], s, y, local);
                w.z = pack4<true>(&v[k][8], s, y, local);
                w.w = pack4<true>(&v[k][12], s, y, local);
            } else {
                w.x = pack4<false>(&v[k][0], s, y, local);
                w.y = pack4<false>(&v[k][4], s, y, local);
                w.z = pack4<false>(&v[k][8], s, y, local);
                w.w = pack4<false>(&v[k][12], s, y, local);
            }
            *reinterpret_cast<uint4*>(out + 64 * k) = w;
        }
    };
    auto row_peak = [&](float peak) {
        peak = wave_max(peak);
        if constexpr (WPR > 1) {
            if (lane == 0) s_peak[wave] = peak;
            __syncthreads();
            const int first = wave - part;
#pragma unroll
            for (int w = 0; w < WPR; ++w) peak = fmaxf(peak, s_peak[first + w]);
        }
        return peak;
    };

    float peak = 0.0f;
    float v[4][16];
    float s, y;
    bool tiny;
    if constexpr (HOLD) {
        rotate_group<T>(group_ptr(0), sub, v);
        peak = row_peak(peak_of(v, peak));
        s = row_scale_of(peak);
        y = 1.0f / s;
        tiny = s < 0x1p-90f;
        emit(0, v, s, y, tiny);
    } else {
        for (int p = 0; p < passes; ++p) {
            rotate_group<T>(group_ptr(p), sub, v);
            peak = peak_of(v, peak);
        }
        peak = row_peak(peak);
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
        if constexpr (WPR > 1) {
            if (lane == 0) s_sum[wave] = local;
            __syncthreads();
            if (part == 0 && lane == 0) {
                int total = 0;
#pragma unroll
                for (int w = 0; w < WPR; ++w) total += s_sum[wave + w];
                if (valid) sum_out[row] = total;
            }
        } else if (lane == 0) {
            sum_out[row] = local;
        }
    }
    if (valid && part == 0 && lane == 0) scale_out[row] = s;
}

template <typename T>
hipError_t launch_convrot_typed(const T* x, int64_t rows, int64_t width, int64_t ld,
                                uint8_t* codes, float* scale, int32_t* sum, hipStream_t stream) {
    const int64_t groups = width / kGroup;
    dim3 block(256);
#define OMNI_CONVROT(WPR, HOLD)                                                                   \
    hipLaunchKernelGGL((convrot_quantize_kernel<T, WPR, HOLD>), dim3((unsigned)((rows + 4 / WPR - 1) / (4 / WPR))), \
                       block, 0, stream, x, rows, width, ld, codes, scale, sum)
    if (groups <= 16)
        OMNI_CONVROT(1, true);
    else if (groups <= 32)
        OMNI_CONVROT(2, true);
    else if (groups <= 64)
        OMNI_CONVROT(4, true);
    else
        OMNI_CONVROT(4, false);
#undef OMNI_CONVROT
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
