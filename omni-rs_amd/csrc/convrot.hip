// ConvRot activation rotation fused into per-row int8 quantisation, gfx950.
//
// Semantics (crates/qwen-image/src/convrot.rs:81-92, 113-149, then
// crates/omni-kernel/src/int8_matmul.rs:23-118):
//   r[row][256 g + c] = sum_j x[row][256 g + j] * H[j][c]          (f32)
//   H = 2^-4 * (H4 (x) H4 (x) H4 (x) H4),  H4[a][b] = -1 iff a ^ b == 3
// followed by the per-row quantisation of r as quantize.hip does it (peak,
// row_scale = max(peak / 127, 1e-30), the correctly rounded quotient, round
// half away; row_quot below).
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
// cross-lane stage is three adds whose permuted operand comes through DPP
// (no LDS). A wave rotates 16 groups at once. Rows of up to 64 groups are
// packed whole into workgroups of 1-4 waves and keep their rotated values in
// registers between the peak and the code pass; wider rows rotate each group
// twice (the second read hits the caches).
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

// Sixteen consecutive f32 elements at p (16-byte aligned).
__device__ __forceinline__ void load16(const float* p, float (&v)[16]) {
    uint4 raw[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) raw[i] = reinterpret_cast<const uint4*>(p)[i];
    __builtin_memcpy(v, raw, sizeof(v));
}

// f16 inputs enter the first stage without separate conversions:
// v_fma_mix_f32 reads a 16-bit half of a register as f16 (op_sel picks the
// half), widened exactly, so lo + hi and s - 2 h round exactly as the same
// f32 operations on converted values do.
__device__ __forceinline__ float f16_pair_sum(unsigned w) {
    float r;
    asm("v_fma_mix_f32 %0, %1, 1.0, %1 op_sel:[0,0,1] op_sel_hi:[1,0,1]" : "=v"(r) : "v"(w));
    return r;
}
template <bool HI>
__device__ __forceinline__ float f16_fma_m2(unsigned w, float s) {
    float r;
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, -2.0, %1, %2 op_sel:[0,1,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(w), "v"(s));
    else
        asm("v_fma_mix_f32 %0, -2.0, %1, %2 op_sel:[0,0,0] op_sel_hi:[0,1,0]" : "=v"(r) : "v"(w), "v"(s));
    return r;
}

// Sixteen consecutive f16 elements at p (16-byte aligned) through digit 0:
// h4 on each run of four, in f32.
__device__ __forceinline__ void load16_h4(const _Float16* p, float (&v)[16]) {
    uint4 raw[2];
    raw[0] = reinterpret_cast<const uint4*>(p)[0];
    raw[1] = reinterpret_cast<const uint4*>(p)[1];
    unsigned w[8];
    __builtin_memcpy(w, raw, sizeof(w));
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        // elements 4q, 4q+1 in w[2q] (lo, hi), 4q+2, 4q+3 in w[2q+1]
        const float s = f16_pair_sum(w[2 * q]) + f16_pair_sum(w[2 * q + 1]);
        v[4 * q] = f16_fma_m2<true>(w[2 * q + 1], s);
        v[4 * q + 1] = f16_fma_m2<false>(w[2 * q + 1], s);
        v[4 * q + 2] = f16_fma_m2<true>(w[2 * q], s);
        v[4 * q + 3] = f16_fma_m2<false>(w[2 * q], s);
    }
}

// The group starting at g rotated into v, unnormalised: v holds u = 16 r
// (the four H4 stages without their 2^-4). All lanes of a quad must call it
// together (digit 2 permutes within quads); an idle quad passes any valid
// group and discards the result, which costs less than a branch.
template <typename T>
__device__ __forceinline__ void rotate_group(const T* g, int sub, float (&v)[4][16]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if constexpr (std::is_same_v<T, float>) {
            load16(g + 64 * k + 16 * sub, v[k]);
#pragma unroll
            for (int q = 0; q < 4; ++q) h4(v[k][4 * q], v[k][4 * q + 1], v[k][4 * q + 2], v[k][4 * q + 3]);
        } else {
            load16_h4(g + 64 * k + 16 * sub, v[k]);
        }
        // Digit 1: element bits 2-3 (digit 0 was applied as the values loaded).
#pragma unroll
        for (int r = 0; r < 4; ++r) h4(v[k][r], v[k][r + 4], v[k][r + 8], v[k][r + 12]);
    }
    // Digit 3: element bits 6-7 (k).
#pragma unroll
    for (int e = 0; e < 16; ++e) h4(v[0][e], v[1][e], v[2][e], v[3][e]);
    // Digit 2: element bits 4-5 are the lane's bits 0-1. With a the lane's
    // digit and x' the value of lane a ^ 3, y_a = (x_a - x') + t_(a^1) where
    // t = x + x': three adds that each read their permuted operand through
    // DPP (s - 2 x' as in h4 would need a separate permute for the fma).
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        float t[16];
#pragma unroll
        for (int e = 0; e < 16; ++e) {
            const float x = v[k][e];
            t[e] = x + quad_xor<3>(x);
            v[k][e] = x - quad_xor<3>(x);
        }
#pragma unroll
        for (int e = 0; e < 16; ++e) v[k][e] += quad_xor<1>(t[e]);
    }
}

// Per-row quotient constants. The kernel holds u = 16 r; the code of r under
// row scale s is round_half_away(RN(r / s)) (int8_matmul.rs:102-118), and
// RN(u / (16 s)) is the same quotient: r / s exactly when r is normal, and a
// code of 0 either way when r is subnormal (|r| < 2^-126, s >= 1e-30).
// 16 s is exact (s >= 1e-30 is normal). The quotient is div_rn's Markstein
// step with y = RN(1 / (16 s)), exact for 16 s >= 2^-90; rows below that
// (tiny) divide with the IEEE division.
struct RowQuot {
    float s, s16, y16;
    bool tiny;
};

__device__ __forceinline__ RowQuot row_quot(float peak_u) {
    RowQuot q;
    q.s = row_scale_of(peak_u * 0.0625f);   // the peak of r; exact
    q.s16 = 16.0f * q.s;
    q.y16 = 1.0f / q.s16;
    q.tiny = q.s16 < 0x1p-90f;
    return q;
}

// Codes of u[0..3], packed little-endian, their sum accumulated, as pack4
// does. No clamp: |u| <= the row peak and 16 s >= peak / 127 (1 - 2^-23), so
// |q| + 1/2 < 127.5001 and the truncation lands in [-127, 127]; NaN gives 0
// (cvt_i32_sat). An infinite u makes the peak, hence s, infinite, and every
// code 0.
template <bool TINY>
__device__ __forceinline__ u32 pack4_rot(const float* u, const RowQuot& rq, int& sum) {
    int c[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const float q = div_rn<TINY>(u[b], rq.s16, rq.y16);
        c[b] = cvt_i32_sat(q + __builtin_copysignf(0.5f, q));
    }
    const u32 lo = __builtin_amdgcn_perm((u32)c[1], (u32)c[0], 0x0c0c0400u);  // c0.b0, c1.b0
    const u32 hi = __builtin_amdgcn_perm((u32)c[3], (u32)c[2], 0x0c0c0400u);  // c2.b0, c3.b0
    const u32 word = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    sum = __builtin_amdgcn_sdot4((int)word, 0x01010101, sum, false);
    return word;
}

// One lane's 64 codes (4 runs of 16 at out + 64 k) from its rotated values.
template <bool TINY>
__device__ __forceinline__ void emit_codes(uint8_t* out, const float (&v)[4][16], const RowQuot& rq, int& sum) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        uint4 w;
        w.x = pack4_rot<TINY>(&v[k][0], rq, sum);
        w.y = pack4_rot<TINY>(&v[k][4], rq, sum);
        w.z = pack4_rot<TINY>(&v[k][8], rq, sum);
        w.w = pack4_rot<TINY>(&v[k][12], rq, sum);
        *reinterpret_cast<uint4*>(out + 64 * k) = w;
    }
}

// The largest |v| of a lane; NaN values are skipped (fmaxf), so the result is
// a non-negative non-NaN float, whose bit pattern orders like its value.
__device__ __forceinline__ float lane_peak(const float (&v)[4][16], float peak) {
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int e = 0; e < 16; ++e) peak = fmaxf(peak, __builtin_fabsf(v[k][e]));
    return peak;
}

// Rows of up to 64 groups. A workgroup of W waves has 16 W group slots (one
// per lane quad) and takes `per_block` = floor(16 W / G) whole rows of G
// groups: slot s holds group s % G of the block's row s / G, so a 12-group
// row wastes no lanes with W = 3 and 4 rows per block. Each quad's peak and
// code sum are combined per row with LDS atomics; the rotated values stay in
// registers between the peak and the codes.
template <typename T>
__global__ __launch_bounds__(256) void convrot_rows_kernel(
    const T* __restrict__ x, int64_t rows, int64_t width, int64_t ld, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out, int32_t* __restrict__ sum_out, int per_block) {
    __shared__ unsigned s_peak[64];
    __shared__ int s_sum[64];
    const int sub = threadIdx.x & 3;
    const int slot = threadIdx.x >> 2;
    const int groups = (int)(width / kGroup);
    const int r = slot / groups;                    // < 64: slot < 64, groups >= 1
    const int g = slot - r * groups;
    const int64_t row = (int64_t)blockIdx.x * per_block + r;
    const bool active = r < per_block && row < rows;
    if ((int)threadIdx.x < per_block) {
        s_peak[threadIdx.x] = 0u;
        s_sum[threadIdx.x] = 0;
    }
    float v[4][16];
    rotate_group<T>(active ? x + row * ld + (int64_t)g * kGroup : x, sub, v);
    float peak = lane_peak(v, 0.0f);
    peak = fmaxf(peak, quad_xor<1>(peak));
    peak = fmaxf(peak, quad_xor<2>(peak));
    __syncthreads();                                // the clears above are visible
    if (active && sub == 0) atomicMax(&s_peak[r], __float_as_uint(peak));
    __syncthreads();
    const RowQuot rq = row_quot(__uint_as_float(s_peak[r]));
    int local = 0;
    // Rows of different scales share a wave; the IEEE division runs only in
    // waves that hold a tiny row (a wave-uniform branch).
    const bool any_tiny = __builtin_amdgcn_ballot_w64(active && rq.tiny) != 0;
    if (active) {
        uint8_t* dst = codes + row * width + (int64_t)g * kGroup + 16 * sub;
        if (any_tiny)
            emit_codes<true>(dst, v, rq, local);
        else
            emit_codes<false>(dst, v, rq, local);
    }
    if (sum_out) {
        local += __float_as_int(quad_xor<1>(__int_as_float(local)));
        local += __float_as_int(quad_xor<2>(__int_as_float(local)));
        if (active && sub == 0) atomicAdd(&s_sum[r], local);
    }
    __syncthreads();
    if ((int)threadIdx.x < per_block) {
        const int64_t out_row = (int64_t)blockIdx.x * per_block + threadIdx.x;
        if (out_row < rows) {
            scale_out[out_row] = row_quot(__uint_as_float(s_peak[threadIdx.x])).s;
            if (sum_out) sum_out[out_row] = s_sum[threadIdx.x];
        }
    }
}

// Rows of more than 64 groups: four waves per row, each rotating 16 groups
// per pass; every group is rotated for the peak and again for the codes (the
// second read hits the caches).
template <typename T>
__global__ __launch_bounds__(256) void convrot_wide_kernel(
    const T* __restrict__ x, int64_t rows, int64_t width, int64_t ld, uint8_t* __restrict__ codes,
    float* __restrict__ scale_out, int32_t* __restrict__ sum_out) {
    constexpr int kWaves = 4;
    __shared__ float s_peak[kWaves];
    __shared__ int s_sum[kWaves];
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t row = blockIdx.x;
    const int sub = lane & 3, slot = lane >> 2;
    const int groups = (int)(width / kGroup);
    const int passes = (groups + 16 * kWaves - 1) / (16 * kWaves);
    const T* src = x + row * ld;
    auto group_of = [&](int p) { return (p * kWaves + wave) * 16 + slot; };
    float v[4][16];
    float peak = 0.0f;
    for (int p = 0; p < passes; ++p) {
        const int g = group_of(p);
        rotate_group<T>(g < groups ? src + (int64_t)g * kGroup : src, sub, v);
        peak = lane_peak(v, peak);
    }
    peak = wave_max(peak);
    if (lane == 0) s_peak[wave] = peak;
    __syncthreads();
    peak = fmaxf(fmaxf(s_peak[0], s_peak[1]), fmaxf(s_peak[2], s_peak[3]));
    const RowQuot rq = row_quot(peak);
    int local = 0;
    for (int p = 0; p < passes; ++p) {
        const int g = group_of(p);
        rotate_group<T>(g < groups ? src + (int64_t)g * kGroup : src, sub, v);
        if (g < groups) {
            uint8_t* dst = codes + row * width + (int64_t)g * kGroup + 16 * sub;
            if (rq.tiny)  // one row per workgroup: uniform
                emit_codes<true>(dst, v, rq, local);
            else
                emit_codes<false>(dst, v, rq, local);
        }
    }
    if (sum_out) {
        local = wave_sum_i32(local);
        if (lane == 0) s_sum[wave] = local;
        __syncthreads();
        if (threadIdx.x == 0) sum_out[row] = s_sum[0] + s_sum[1] + s_sum[2] + s_sum[3];
    }
    if (threadIdx.x == 0) scale_out[row] = rq.s;
}

// Waves per workgroup for rows of G <= 64 groups: the W in 1..4 whose
// floor(16 W / G) whole rows leave the fewest idle slots (ties: fewer waves).
int rows_kernel_waves(int groups) {
    int best = 4;
    double best_use = 0.0;
    for (int w = 1; w <= 4; ++w) {
        const int per = 16 * w / groups;
        const double use = per > 0 ? (double)(per * groups) / (16 * w) : 0.0;
        if (use > best_use + 1e-9) {
            best_use = use;
            best = w;
        }
    }
    return best;
}

template <typename T>
hipError_t launch_convrot_typed(const T* x, int64_t rows, int64_t width, int64_t ld,
                                uint8_t* codes, float* scale, int32_t* sum, hipStream_t stream) {
    const int64_t groups = width / kGroup;
    if (groups < 1) return hipErrorInvalidValue;
    if (groups <= 64) {
        const int w = rows_kernel_waves((int)groups);
        const int per = 16 * w / (int)groups;
        hipLaunchKernelGGL(convrot_rows_kernel<T>, dim3((unsigned)((rows + per - 1) / per)), dim3(64 * w), 0,
                           stream, x, rows, width, ld, codes, scale, sum, per);
    } else {
        hipLaunchKernelGGL(convrot_wide_kernel<T>, dim3((unsigned)rows), dim3(256), 0, stream, x, rows,
                           width, ld, codes, scale, sum);
    }
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
