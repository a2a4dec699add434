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

// f32 -> int32 by v_cvt_i32_f32, which the ISA defines to truncate toward
// zero, saturate to the int32 range and return 0 for NaN. A C++ (int) cast
// of NaN or of an out-of-range value is undefined (LLVM's fptosi gives
// poison), so the instruction is issued directly.
__device__ __forceinline__ int cvt_i32_sat(float v) {
    int r;
    asm("v_cvt_i32_f32 %0, %1" : "=v"(r) : "v"(v));
    return r;
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

// ---- cross-lane moves in registers (no LDS round trip) ----

// DPP move of v within a wave; CTRL is a gfx9 DPP control, every source lane
// valid for the controls used here.
template <int CTRL>
__device__ __forceinline__ float dpp_mov(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, false));
}

// The value of lane (lane ^ O) for O in 1, 2, 4, 8: quad_perm for 1 and 2;
// xor 4 = row_half_mirror (xor 7) after quad_perm [3,2,1,0] (xor 3);
// xor 8 = row_mirror (xor 15) after row_half_mirror (xor 7).
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(O == 1 || O == 2 || O == 4 || O == 8, "within a row of 16 lanes");
    if constexpr (O == 1) return dpp_mov<0xB1>(v);                  // quad_perm [1,0,3,2]
    if constexpr (O == 2) return dpp_mov<0x4E>(v);                  // quad_perm [2,3,0,1]
    if constexpr (O == 4) return dpp_mov<0x141>(dpp_mov<0x1B>(v));  // half_mirror(quad_perm [3,2,1,0])
    return dpp_mov<0x140>(dpp_mov<0x141>(v));                       // row_mirror(half_mirror)
}

// One butterfly step across lanes l and l ^ O for O = 16 or 32 with the
// gfx950 permlane swaps: lanes with bit O clear return a + a(l ^ O), lanes
// with it set return b + b(l ^ O). v_permlane16_swap(a, b) returns the rows
// (16 lanes) {a0, b0, a2, b2} and {a1, b1, a3, b3}; v_permlane32_swap(a, b)
// the halves {a_lo, b_lo} and {a_hi, b_hi} (lane layout checked on MI355X),
// so the two results' sum is the step.
template <int O>
__device__ __forceinline__ float swap_add(float a, float b) {
    static_assert(O == 16 || O == 32, "across rows or halves");
    const unsigned ua = __float_as_uint(a), ub = __float_as_uint(b);
    if constexpr (O == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(ua, ub, false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(ua, ub, false, false);
        return __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
}

// RN(x / s) given y = RN(1 / s): q0 = x * y, r = fma(-q0, s, x),
// q = fma(r, y, q0) (Markstein's correction step) returns the correctly
// rounded quotient whenever the residual r is exact, which holds for
// s >= 2^-90; TINY rows (s below that) use the IEEE division itself.
template <bool TINY>
__device__ __forceinline__ float div_rn(float x, float s, float y) {
#pragma clang fp contract(off)
    if constexpr (TINY) return x / s;
    const float q0 = x * y;
    const float r = __builtin_fmaf(-q0, s, x);
    return __builtin_fmaf(r, y, q0);
}

// Codes of four consecutive values packed little-endian into one word; the
// codes' sum is accumulated with one v_dot4 against 1,1,1,1.
//
// Rounding: trunc(q + copysign(0.5, q)) equals sign(q) * floor(|q| + 0.5)
// with the same f32 addition as the reference (q - 0.5 is exactly
// -(|q| + 0.5)), and cvt_i32_sat truncates toward zero and maps NaN to 0.
// |q| <= 127 * (1 + 2^-23) always (the row scale is the peak / 127), so the
// clamp to [-128, 127] only ever matters for NaN/Inf-derived values.
template <bool TINY>
__device__ __forceinline__ u32 pack4(const float* v, float s, float y, int& sum) {
    int c[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        const float q = div_rn<TINY>(v[b], s, y);
        const int r = cvt_i32_sat(q + __builtin_copysignf(0.5f, q));
        c[b] = r < -128 ? -128 : (r > 127 ? 127 : r);
    }
    const u32 lo = __builtin_amdgcn_perm((u32)c[1], (u32)c[0], 0x0c0c0400u);  // c0.b0, c1.b0
    const u32 hi = __builtin_amdgcn_perm((u32)c[3], (u32)c[2], 0x0c0c0400u);  // c2.b0, c3.b0
    const u32 word = __builtin_amdgcn_perm(hi, lo, 0x05040100u);
    sum = __builtin_amdgcn_sdot4((int)word, 0x01010101, sum, false);
    return word;
}

// Row scale from the peak: max(peak / 127, 1e-30) (int8_matmul.rs:63-68).
__device__ __forceinline__ float row_scale_of(float peak) {
    float row_scale = peak / 127.0f;
    // `!(a > b)` also catches a NaN peak, like Rust's f32::max with 1e-30.
    if (!(row_scale > 1.0e-30f)) row_scale = 1.0e-30f;
    return row_scale;
}

// ---- LDS-DMA pipeline helpers shared by the MFMA GEMM kernels ----

// Hardware workgroup id -> logical tile id, so that the workgroups one XCD
// runs (hardware ids congruent mod 8) get a contiguous range of logical tiles.
__device__ __forceinline__ int xcd_remap(int b, int total) {
    constexpr int kXcds = 8;
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = b % kXcds, local = b / kXcds;
    return xcd * per + (xcd < rem ? xcd : rem) + local;
}


#define OMNI_LDS __attribute__((address_space(3)))

// One 16-byte-per-lane global -> LDS copy (global_load_lds_dwordx4). The
// builtin needs a gfx950 target feature that the host compilation pass lacks,
// so it is emitted in the device pass only.
__device__ __forceinline__ void lds_copy16(const uint8_t* src, uint8_t* lds_dst) {
#if defined(__HIP_DEVICE_COMPILE__)
    __builtin_amdgcn_global_load_lds(src, (OMNI_LDS void*)lds_dst, 16, 0, 0);
#endif
}

// The same copy as inline assembly: the compiler then sees no LDS write in
// flight, so it inserts no vmcnt wait of its own before a later LDS read
// (where it cannot tell which ring stage a copy targets it waits for every
// outstanding operation, a full pipeline drain per K tile). The caller's
// explicit waits order the copies. The source is a wave-uniform 64-bit base
// (SGPRs) plus a 32-bit per-lane byte offset (no per-lane 64-bit pointer is
// held or added); the LDS byte address is a wave-uniform integer (see
// lds_addr). m0 is listed as clobbered, which the compiler reports as a
// reserved register it will not preserve: a kernel that uses this copy must
// not also use the builtin lds_copy16 (whose m0 setup the compiler may hoist);
// the only other m0 users on gfx950 are absent from these kernels.
__device__ __forceinline__ void lds_copy16_saddr(unsigned voff, const void* base, unsigned lds_byte) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "s"(lds_byte)
                 : "memory", "m0");
#endif
}

// The same for 4 bytes per lane: lane l's dword lands at lds_byte + 4 l.
__device__ __forceinline__ void lds_copy4_saddr(unsigned voff, const void* base, unsigned lds_byte) {
#if defined(__HIP_DEVICE_COMPILE__)
    asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "s"(lds_byte)
                 : "memory", "m0");
#endif
}

// LDS byte address of a __shared__ object, as a wave-uniform integer.
__device__ __forceinline__ unsigned lds_addr(const void* p) {
#if defined(__HIP_DEVICE_COMPILE__)
    return __builtin_amdgcn_readfirstlane((unsigned)(uintptr_t)(const OMNI_LDS void*)p);
#else
    (void)p;
    return 0;
#endif
}


// s_waitcnt vmcnt(N) (and lgkmcnt(0) when LGKM0) for a compile-time N.
template <int N, bool LGKM0 = false>
__device__ __forceinline__ void s_waitcnt_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    // gfx9 encoding: vmcnt[3:0] | expcnt << 4 | lgkmcnt << 8 | vmcnt[5:4] << 14
    __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | ((LGKM0 ? 0 : 15) << 8) | ((N >> 4) << 14));
}

// Workgroup barrier for the LDS-DMA pipeline. __syncthreads() would wait for
// every outstanding vector-memory operation (its release fence counts the
// in-flight global->LDS copies as LDS writes); here the caller has already
// waited for the copies that matter, and lgkmcnt(0) retires this wave's LDS
// reads, so a plain s_barrier suffices. The memory clobber keeps the compiler
// from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_barrier" ::: "memory"); }

}  // namespace omni
