/*
 * CPU oracle for the int8 quantised-matmul hot path.
 *
 * TEST INFRASTRUCTURE ONLY. This file is a plain-C restatement of the
 * reference's CPU arithmetic. It is linked by the tests, by
 * __graft_entry__.smoke() (as the checker) and by bench.py's cpu_baseline leg.
 * The product library (omni-rs_amd/csrc) never links or calls it, and there
 * is no CPU fallback in the product path.
 *
 * Build with -ffp-contract=off and without -ffast-math (oracle/Makefile):
 * the reference is Rust, which never fuses a multiply and an add, and its
 * f32 division is IEEE.
 *
 * Reference: GoooIce/omni-rs (Rust). Each function cites the file:line it
 * restates. Parity pins for every function are listed in the header
 * oracle_int8.h; none is "parity unpinned" except where that header says so.
 */
#include "oracle_int8.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* ---------------------------------------------------------------------------
 * IEEE binary16 <-> binary32, round-to-nearest-even. gcc 11 on x86-64 has no
 * _Float16, so the conversion is written out from the IEEE 754 encoding.
 * Pinned exhaustively against numpy.float16 in tests/test_oracle.py.
 * ------------------------------------------------------------------------- */
static uint32_t f32_bits(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
static float bits_f32(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }

float oracle_f16_to_f32(uint16_t h)
{
    uint32_t sign = (uint32_t)(h >> 15) << 31;
    uint32_t exp = (h >> 10) & 0x1f;
    uint32_t man = h & 0x3ff;
    if (exp == 0x1f) /* inf / nan: keep payload */
        return bits_f32(sign | 0x7f800000u | (man << 13));
    if (exp == 0) {
        /* zero or subnormal: value = man * 2^-24, exact in f32 */
        float v = (float)man * (1.0f / 16777216.0f);
        return sign ? -v : v;
    }
    return bits_f32(sign | ((exp + 112u) << 23) | (man << 13));
}

uint16_t oracle_f32_to_f16(float f)
{
    uint32_t u = f32_bits(f);
    uint16_t sign = (uint16_t)((u >> 16) & 0x8000u);
    uint32_t exp = (u >> 23) & 0xff;
    uint32_t man = u & 0x7fffffu;
    if (exp == 0xff) /* inf / nan (quiet the nan) */
        return (uint16_t)(sign | 0x7c00u | (man ? 0x200u | (man >> 13) : 0u));
    int e = (int)exp - 127; /* unbiased */
    if (e > 15)
        return (uint16_t)(sign | 0x7c00u); /* overflow to inf */
    if (e >= -14) {
        /* normal f16 range: 10 mantissa bits kept, 13 dropped */
        uint32_t m = man;
        uint32_t half = (uint32_t)(e + 15) << 10 | (m >> 13);
        uint32_t rest = m & 0x1fffu;
        if (rest > 0x1000u || (rest == 0x1000u && (half & 1u)))
            half += 1u; /* carry may roll into the exponent, and to inf: correct */
        return (uint16_t)(sign | half);
    }
    if (e < -25)
        return sign; /* below half the smallest subnormal: rounds to zero */
    /* subnormal result: value / 2^-24 rounded to an integer, RNE */
    {
        uint32_t m = man | 0x800000u; /* 24-bit significand, value = m * 2^(e-23) */
        int shift = -e - 1;           /* bits to drop so the unit is 2^-24: 13 + (-14 - e) */
        uint32_t q = m >> shift;
        uint32_t rest = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rest > halfway || (rest == halfway && (q & 1u)))
            q += 1u;
        return (uint16_t)(sign | q);
    }
}

/* ---------------------------------------------------------------------------
 * W8A8 core.
 * ------------------------------------------------------------------------- */

/* crates/omni-kernel/src/int8_host.rs:3-10 (round_half_away): round half away
 * from zero in f32, then clamp to [-128, 127] and convert. Rust's `as i32` on
 * a NaN gives 0 and `clamp` keeps NaN, so a NaN code is 0. */
int32_t oracle_round_half_away(float value)
{
    float rounded = value >= 0.0f ? floorf(value + 0.5f) : ceilf(value - 0.5f);
    if (isnan(rounded))
        return 0;
    if (rounded < -128.0f)
        rounded = -128.0f;
    if (rounded > 127.0f)
        rounded = 127.0f;
    return (int32_t)rounded;
}

/* crates/omni-kernel/src/int8_host.rs:12-17 (unpack_i8): little-endian bytes of
 * each i32 word, sign-extended. */
void oracle_unpack_i8(const int32_t* words, int64_t count, int8_t* out)
{
    for (int64_t i = 0; i < count; ++i) {
        uint32_t w = (uint32_t)words[i];
        for (int lane = 0; lane < 4; ++lane)
            out[4 * i + lane] = (int8_t)(uint8_t)(w >> (8 * lane));
    }
}

/* crates/qwen-image/src/convrot.rs:151-160 (pack_i8): four codes per i32, the
 * first code in the lowest byte. */
void oracle_pack_i8(const int8_t* codes, int64_t count, int32_t* words)
{
    for (int64_t i = 0; i < count / 4; ++i) {
        uint32_t w = 0;
        for (int lane = 0; lane < 4; ++lane)
            w |= (uint32_t)(uint8_t)codes[4 * i + lane] << (8 * lane);
        words[i] = (int32_t)w;
    }
}

/* Per-row dynamic symmetric quantisation.
 * crates/omni-kernel/src/int8_host.rs:31-39 (host) and
 * crates/omni-kernel/src/int8_matmul.rs:23-118 (quantize_rows / quantize_i8):
 *   peak      = max |x| over the row, folded from 0.0 in f32 (NaN ignored,
 *               as Rust's f32::max and the kernel's `>` test both do);
 *   row_scale = max(peak / 127, 1e-30) in f32;
 *   code      = round_half_away(x / row_scale) with an IEEE f32 division;
 *   sum       = sum of the row's codes (int8_matmul.rs:86-98).
 * x is row-major with leading dimension ld (elements). */
void oracle_quantize_rows(const float* x, int64_t rows, int64_t width, int64_t ld,
                          int8_t* codes, float* row_scale, int32_t* row_sum)
{
    for (int64_t r = 0; r < rows; ++r) {
        const float* s = x + r * ld;
        float peak = 0.0f;
        for (int64_t k = 0; k < width; ++k) {
            float a = fabsf(s[k]);
            if (a > peak)
                peak = a;
        }
        float scale = peak / 127.0f;
        if (!(scale > 1.0e-30f))
            scale = 1.0e-30f;
        int32_t sum = 0;
        for (int64_t k = 0; k < width; ++k) {
            float q = s[k] / scale;
            int32_t c = oracle_round_half_away(q);
            codes[r * width + k] = (int8_t)c;
            sum += c;
        }
        if (row_scale)
            row_scale[r] = scale;
        if (row_sum)
            row_sum[r] = sum;
    }
}

/* Exact int32 accumulators acc[m][n] = sum_k codes[m][k] * w[n][k].
 * crates/omni-kernel/src/int8_host.rs:40-47 (the `acc` loop). w is [N][K]
 * row-major int8, i.e. the bytes of the reference's packed [N][K/4] words. */
void oracle_int8_acc(const int8_t* codes, const int8_t* w, int64_t rows, int64_t columns,
                     int64_t width, int32_t* acc)
{
    for (int64_t r = 0; r < rows; ++r) {
        const int8_t* a = codes + r * width;
        for (int64_t c = 0; c < columns; ++c) {
            const int8_t* b = w + c * width;
            int32_t s = 0;
            for (int64_t k = 0; k < width; ++k)
                s += (int32_t)a[k] * (int32_t)b[k];
            acc[r * columns + c] = s;
        }
    }
}

/* The reference epilogue, crates/omni-kernel/src/int8_matmul.rs:145-159 (store)
 * and int8_host.rs:48-49: out = f32(acc - sum*zero) * row_scale * w_scale,
 * evaluated left to right in f32. */
float oracle_epilogue(int32_t acc, int32_t sum, int32_t zero, float row_scale, float w_scale)
{
    int32_t centered = acc - sum * zero;
    float t = (float)centered * row_scale;
    return t * w_scale;
}

/* Whole reference CPU path: crates/omni-kernel/src/int8_host.rs:19-53 (gemm).
 * x f32 [rows][width], w int8 [columns][width], scale f32 [columns],
 * zero i32 [columns] -> out f32 [rows][columns]. Same loop order as the
 * reference (row, then column, then k), quantisation recomputed per row. */
void oracle_int8_gemm(const float* x, int64_t rows, int64_t width, const int8_t* w,
                      const float* scale, const int32_t* zero, int64_t columns, float* out)
{
    int8_t* codes = (int8_t*)malloc((size_t)width);
    for (int64_t r = 0; r < rows; ++r) {
        float rs;
        int32_t sum;
        oracle_quantize_rows(x + r * width, 1, width, width, codes, &rs, &sum);
        for (int64_t c = 0; c < columns; ++c) {
            const int8_t* b = w + c * width;
            int32_t acc = 0;
            for (int64_t k = 0; k < width; ++k)
                acc += (int32_t)codes[k] * (int32_t)b[k];
            out[r * columns + c] = oracle_epilogue(acc, sum, zero[c], rs, scale[c]);
        }
    }
    free(codes);
}

/* oracle_int8_gemm with its rows spread over `threads` OpenMP threads: each
 * row is computed exactly as oracle_int8_gemm computes it (rows are
 * independent), so the output is bit-identical. It exists to time the
 * reference's CPU path on every host core as well as on one (the reference
 * itself is single-threaded, int8_host.rs:19-53). */
void oracle_int8_gemm_threads(const float* x, int64_t rows, int64_t width, const int8_t* w,
                              const float* scale, const int32_t* zero, int64_t columns,
                              float* out, int threads)
{
    if (threads < 1)
        threads = 1;
#pragma omp parallel for num_threads(threads) schedule(dynamic, 1)
    for (int64_t r = 0; r < rows; ++r)
        oracle_int8_gemm(x + r * width, 1, width, w, scale, zero, columns, out + r * columns);
}

/* Epilogue variant with an optional bias and an fp16 output. The reference op
 * has no bias (crates/qwen-image/src/convrot.rs:30-67 loads none) and returns
 * f32 that its caller casts to the model precision (convrot.rs:89-91). This
 * variant keeps the reference f32 value bit for bit, adds bias[n] in f32 and
 * rounds once to fp16 (RNE): the cast convrot.rs:91 performs, with the bias
 * add in between. */
void oracle_w8a8_finish(const int32_t* acc, const int32_t* row_sum, const float* row_scale,
                        const float* w_scale, const int32_t* w_zero, const float* bias,
                        int64_t rows, int64_t columns, float* out_f32, uint16_t* out_f16)
{
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < columns; ++c) {
            float v = oracle_epilogue(acc[r * columns + c], row_sum[r], w_zero[c],
                                      row_scale[r], w_scale[c]);
            if (bias)
                v = v + bias[c];
            if (out_f32)
                out_f32[r * columns + c] = v;
            if (out_f16)
                out_f16[r * columns + c] = oracle_f32_to_f16(v);
        }
}

/* The reference's dequantised-weight check, crates/omni-kernel/src/int8_matmul.rs:621-655
 * (dequantized_weight_reference): activations are quantised and dequantised
 * per row, weights are dequantised through fp16 as f16((w - zero) * scale),
 * and the dot accumulates in f32 in k order. */
void oracle_dequant_reference(const float* x, int64_t rows, int64_t width, const int8_t* w,
                              const float* scale, const int32_t* zero, int64_t columns,
                              float* out)
{
    float* act = (float*)malloc((size_t)width * sizeof(float));
    for (int64_t r = 0; r < rows; ++r) {
        const float* s = x + r * width;
        float peak = 0.0f;
        for (int64_t k = 0; k < width; ++k) {
            float a = fabsf(s[k]);
            if (a > peak)
                peak = a;
        }
        float rs = peak / 127.0f;
        if (!(rs > 1.0e-30f))
            rs = 1.0e-30f;
        for (int64_t k = 0; k < width; ++k) {
            float q = s[k] / rs;
            act[k] = (float)oracle_round_half_away(q) * rs;
        }
        for (int64_t c = 0; c < columns; ++c) {
            float acc = 0.0f;
            for (int64_t k = 0; k < width; ++k) {
                float wd = oracle_f16_to_f32(oracle_f32_to_f16(
                    (float)((int32_t)w[c * width + k] - zero[c]) * scale[c]));
                acc += act[k] * wd;
            }
            out[r * columns + c] = acc;
        }
    }
    free(act);
}

/* ---------------------------------------------------------------------------
 * W8A16 weight-only path. The reference has no such op; its semantics are the
 * reference's own dequantisation conventions:
 *   crates/minicpm-v/src/quant.rs:186-200 — dequantise at load to f32
 *     (value * scale) and cast to the model precision, then x.matmul(w^T);
 *   crates/omni-kernel/src/int8_matmul.rs:644-649 — f16 dequantised weight,
 *     f32 accumulation.
 * ------------------------------------------------------------------------- */

/* Ground truth in f64: out[m][n] = sum_k x[m][k] * (w[n][k] * scale[n]) + bias[n].
 * x f16 [rows][width], w int8 [columns][width], scale f16 [columns],
 * bias f16 [columns] or NULL. */
void oracle_w8a16_f64(const uint16_t* x, int64_t rows, int64_t width, const int8_t* w,
                      const uint16_t* scale, const uint16_t* bias, int64_t columns, double* out)
{
    double* xr = (double*)malloc((size_t)width * sizeof(double));
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < width; ++k)
            xr[k] = (double)oracle_f16_to_f32(x[r * width + k]);
        for (int64_t c = 0; c < columns; ++c) {
            const int8_t* b = w + c * width;
            double s = 0.0;
            for (int64_t k = 0; k < width; ++k)
                s += xr[k] * (double)b[k];
            s *= (double)oracle_f16_to_f32(scale[c]);
            if (bias)
                s += (double)oracle_f16_to_f32(bias[c]);
            out[r * columns + c] = s;
        }
    }
    free(xr);
}

/* The reference CPU route restated (quant.rs:186-200 with int8_matmul.rs:644-649):
 * w_deq = f16(f32(w) * f32(scale)); acc = sum_k f32(x) * f32(w_deq) in f32, k
 * order; acc += bias (f32); out = f16(acc). */
void oracle_w8a16_gemm(const uint16_t* x, int64_t rows, int64_t width, const int8_t* w,
                       const uint16_t* scale, const uint16_t* bias, int64_t columns,
                       uint16_t* out)
{
    float* xr = (float*)malloc((size_t)width * sizeof(float));
    float* wd = (float*)malloc((size_t)width * sizeof(float));
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < width; ++k)
            xr[k] = oracle_f16_to_f32(x[r * width + k]);
        for (int64_t c = 0; c < columns; ++c) {
            float sc = oracle_f16_to_f32(scale[c]);
            for (int64_t k = 0; k < width; ++k)
                wd[k] = oracle_f16_to_f32(oracle_f32_to_f16((float)w[c * width + k] * sc));
            float acc = 0.0f;
            for (int64_t k = 0; k < width; ++k) {
                acc += xr[k] * wd[k];
            }
            if (bias)
                acc += oracle_f16_to_f32(bias[c]);
            out[r * columns + c] = oracle_f32_to_f16(acc);
        }
    }
    free(xr);
    free(wd);
}

/* ---------------------------------------------------------------------------
 * ConvRot Hadamard rotation (the caller of the W8A8 op).
 * ------------------------------------------------------------------------- */

/* crates/qwen-image/src/convrot.rs:139-149 (sign_negative): parity of the
 * base-4 digits of (row ^ column) that equal 3. */
int oracle_hadamard_sign_negative(uint64_t row, uint64_t column, uint64_t size)
{
    uint64_t v = row ^ column;
    uint64_t threes = v & (v >> 1) & 0x5555555555555555ull;
    int digits = 0;
    while ((1ull << (2 * digits)) < size)
        ++digits;
    int parity = 0;
    for (int i = 0; i < digits; ++i) {
        parity ^= (int)(threes & 1ull);
        threes >>= 2;
    }
    return parity;
}

/* crates/qwen-image/src/convrot.rs:121-133 (hadamard): entries +-2^(-log4 size),
 * negative where sign_negative holds. size must be a power of four. */
void oracle_hadamard(int64_t size, float* matrix)
{
    int log2 = 0;
    while ((1ll << log2) < size)
        ++log2;
    float scale = ldexpf(1.0f, -(log2 / 2));
    for (int64_t r = 0; r < size; ++r)
        for (int64_t c = 0; c < size; ++c)
            matrix[r * size + c] =
                oracle_hadamard_sign_negative((uint64_t)r, (uint64_t)c, (uint64_t)size) ? -scale
                                                                                         : scale;
}

/* crates/qwen-image/src/convrot.rs:113-119 (rotate): each group of `group`
 * consecutive elements of a row is multiplied by H (row vector times H), with
 * an f32 dot in j order. out may not alias x. */
void oracle_rotate(const float* x, int64_t rows, int64_t width, int64_t group, float* out)
{
    float* h = (float*)malloc((size_t)(group * group) * sizeof(float));
    oracle_hadamard(group, h);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g < width / group; ++g) {
            const float* src = x + r * width + g * group;
            float* dst = out + r * width + g * group;
            for (int64_t c = 0; c < group; ++c) {
                float acc = 0.0f;
                for (int64_t j = 0; j < group; ++j) {
                    acc += src[j] * h[j * group + c];
                }
                dst[c] = acc;
            }
        }
    free(h);
}

/* The same group-256 rotation as an f32 fast transform, op for op as the GPU
 * kernel evaluates it (omni-rs_amd/csrc/convrot.hip, rotate_group), so that
 * the kernel's codes can be checked bit for bit. It returns u = 16 r, the
 * rotation without its 2^-4 (r = u / 16 is exact for normal values). The
 * linear map is the reference's H (convrot.rs:121-149) times 16:
 * H4 (x) H4 (x) H4 (x) H4, H4[a][b] = -1 iff a ^ b == 3, one radix-4 stage per
 * base-4 digit of the element index within the group, in the order
 *   digit 0 (index bits 0-1) and digit 1 (bits 2-3), each as
 *     s = (x0 + x1) + (x2 + x3),  y_a = fma(-2, x_(3-a), s);
 *   digit 3 (bits 6-7), the same;
 *   digit 2 (bits 4-5) as y_a = (x_a - x_(a^3)) + (x_(a^1) + x_(a^2)).
 * Only its rounding differs from the reference's f32 matmul (whose
 * summation order is its backend's); pinned in tests/test_convrot.py against
 * the exact rotation (f64) within the transform's error bound and exactly on
 * unit vectors. */
static void oracle_h4(float* x0, float* x1, float* x2, float* x3)
{
    float s = (*x0 + *x1) + (*x2 + *x3);
    float y0 = fmaf(-2.0f, *x3, s);
    float y1 = fmaf(-2.0f, *x2, s);
    float y2 = fmaf(-2.0f, *x1, s);
    float y3 = fmaf(-2.0f, *x0, s);
    *x0 = y0;
    *x1 = y1;
    *x2 = y2;
    *x3 = y3;
}

void oracle_convrot_fwht(const float* x, int64_t rows, int64_t width, int64_t ld, float* u)
{
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t g = 0; g + 256 <= width; g += 256) {
            float v[256];
            memcpy(v, x + r * ld + g, sizeof v);
            /* digit 0: elements 4q .. 4q+3 */
            for (int q = 0; q < 64; ++q)
                oracle_h4(&v[4 * q], &v[4 * q + 1], &v[4 * q + 2], &v[4 * q + 3]);
            /* digit 1: within each run of 16, elements e, e+4, e+8, e+12 */
            for (int b = 0; b < 256; b += 16)
                for (int e = 0; e < 4; ++e)
                    oracle_h4(&v[b + e], &v[b + e + 4], &v[b + e + 8], &v[b + e + 12]);
            /* digit 3: elements i, i+64, i+128, i+192 */
            for (int i = 0; i < 64; ++i)
                oracle_h4(&v[i], &v[i + 64], &v[i + 128], &v[i + 192]);
            /* digit 2: elements i + 16 a for a = 0..3 */
            for (int k = 0; k < 256; k += 64)
                for (int e = 0; e < 16; ++e) {
                    float xa[4], y[4];
                    for (int a = 0; a < 4; ++a)
                        xa[a] = v[k + 16 * a + e];
                    for (int a = 0; a < 4; ++a) {
                        float d = xa[a] - xa[a ^ 3];
                        float t = xa[a ^ 1] + xa[a ^ 2];
                        y[a] = d + t;
                    }
                    for (int a = 0; a < 4; ++a)
                        v[k + 16 * a + e] = y[a];
                }
            memcpy(u + r * width + g, v, sizeof v);
        }
}

/* ConvRot rotation + quantisation as the GPU kernel computes it: u from
 * oracle_convrot_fwht, then the per-row quantisation of r = u / 16 of
 * int8_matmul.rs:23-118 (peak of |r| with NaN skipped, row_scale =
 * max(peak / 127, 1e-30), code = round_half_away(r / row_scale)), with the
 * quotient taken as u / (16 row_scale): the same real number whenever r is
 * normal, and a code of 0 either way when r is subnormal (|r| < 2^-126 and
 * row_scale >= 1e-30). */
void oracle_convrot_quantize_fwht(const float* x, int64_t rows, int64_t width, int64_t ld,
                                  int8_t* codes, float* row_scale, int32_t* row_sum)
{
    float* u = (float*)malloc((size_t)width * sizeof(float));
    for (int64_t r = 0; r < rows; ++r) {
        oracle_convrot_fwht(x + r * ld, 1, width, width, u);
        float peak = 0.0f;
        for (int64_t k = 0; k < width; ++k) {
            float a = fabsf(u[k]);
            if (a > peak)
                peak = a;
        }
        float scale = (peak * 0.0625f) / 127.0f;
        if (!(scale > 1.0e-30f))
            scale = 1.0e-30f;
        const float s16 = 16.0f * scale;
        int32_t sum = 0;
        for (int64_t k = 0; k < width; ++k) {
            int32_t c = oracle_round_half_away(u[k] / s16);
            codes[r * width + k] = (int8_t)c;
            sum += c;
        }
        row_scale[r] = scale;
        row_sum[r] = sum;
    }
    free(u);
}

/* ---- W4A16 (crates/minicpm-v/src/quant.rs) --------------------------------- */

/* quant.rs:22-29 (unpack_int4): two values per byte, low nibble first, each
 * stored as an unsigned nibble offset by 8 (8 means 0, 0 means -8). */
void oracle_unpack_int4(const uint8_t* packed, int64_t bytes, int8_t* out)
{
    for (int64_t i = 0; i < bytes; ++i) {
        out[2 * i] = (int8_t)((int)(packed[i] & 0xF) - 8);
        out[2 * i + 1] = (int8_t)((int)(packed[i] >> 4) - 8);
    }
}

/* quant.rs:74-81 (bf16_scale_bytes): a bf16 is the top half of an f32. */
float oracle_bf16_to_f32(uint16_t b)
{
    uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* quant.rs:186-200 (load_packed, Dequantize mode): each run of `group`
 * consecutive values of the row-major [rows][width] weight times the next
 * scale, in f32; then, for the F16 precision, rounded once to f16. */
void oracle_w4a16_dequant(const uint8_t* packed, const uint16_t* scale_bf16, int64_t rows,
                          int64_t width, int64_t group, int f16_round, float* w_deq)
{
    const int64_t n = rows * width;
    int8_t* v = (int8_t*)malloc((size_t)n);
    oracle_unpack_int4(packed, n / 2, v);
    for (int64_t i = 0; i < n; ++i) {
        float d = (float)v[i] * oracle_bf16_to_f32(scale_bf16[i / group]);
        w_deq[i] = f16_round ? oracle_f16_to_f32(oracle_f32_to_f16(d)) : d;
    }
    free(v);
}

/* Ground truth: x @ (q * s)^T (+ bias) in f64 (every product is exact). */
void oracle_w4a16_f64(const uint16_t* x, int64_t rows, int64_t width, const uint8_t* packed,
                      const uint16_t* scale_bf16, int64_t group, const uint16_t* bias,
                      int64_t columns, double* out)
{
    float* w = (float*)malloc((size_t)(columns * width) * sizeof(float));
    oracle_w4a16_dequant(packed, scale_bf16, columns, width, group, 0, w);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < columns; ++c) {
            double s = 0.0;
            for (int64_t k = 0; k < width; ++k)
                s += (double)oracle_f16_to_f32(x[r * width + k]) * (double)w[c * width + k];
            if (bias)
                s += (double)oracle_f16_to_f32(bias[c]);
            out[r * columns + c] = s;
        }
    free(w);
}

/* The reference's CPU route in F16 precision: dequantise at load to f16
 * (quant.rs:186-200), then x @ w^T (quant.rs:53-58) with f32 accumulation in
 * k order, output rounded to f16. */
void oracle_w4a16_gemm(const uint16_t* x, int64_t rows, int64_t width, const uint8_t* packed,
                       const uint16_t* scale_bf16, int64_t group, const uint16_t* bias,
                       int64_t columns, uint16_t* out)
{
    float* w = (float*)malloc((size_t)(columns * width) * sizeof(float));
    oracle_w4a16_dequant(packed, scale_bf16, columns, width, group, 1, w);
    for (int64_t r = 0; r < rows; ++r)
        for (int64_t c = 0; c < columns; ++c) {
            float acc = 0.0f;
            for (int64_t k = 0; k < width; ++k)
                acc += oracle_f16_to_f32(x[r * width + k]) * w[c * width + k];
            if (bias)
                acc += oracle_f16_to_f32(bias[c]);
            out[r * columns + c] = oracle_f32_to_f16(acc);
        }
    free(w);
}

/* fp16 linear ground truth in f64, as the reference's GEMV test computes its
 * expected value (crates/breeze-tts/src/metal_depth_tests.rs:67-73):
 * out[m][n] = sum_k f64(x[m][k]) * f64(w[n][k]); x f16 [rows][width],
 * w f16 [columns][width] (output-major). */
void oracle_f16_linear_f64(const uint16_t* x, int64_t rows, int64_t width, const uint16_t* w,
                           int64_t columns, double* out)
{
    double* xr = (double*)malloc((size_t)width * sizeof(double));
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t k = 0; k < width; ++k)
            xr[k] = (double)oracle_f16_to_f32(x[r * width + k]);
        for (int64_t c = 0; c < columns; ++c) {
            const uint16_t* b = w + c * width;
            double s = 0.0;
            for (int64_t k = 0; k < width; ++k)
                s += xr[k] * (double)oracle_f16_to_f32(b[k]);
            out[r * columns + c] = s;
        }
    }
    free(xr);
}

/* The reference GEMV restated (crates/breeze-tts/src/metal_depth.rs:13-35):
 * lane l of a 32-lane group sums f32(x[k]) * f32(w[k]) over k = 32 i + l in
 * order, in f32; the 32 partials are added (plane_sum, whose order Metal does
 * not fix: here a butterfly over lane distances 16, 8, 4, 2, 1); the f32 sum
 * is rounded to f16. width % 32 == 0. */
void oracle_f16_gemv(const uint16_t* x, int64_t rows, int64_t width, const uint16_t* w,
                     int64_t columns, uint16_t* out)
{
    for (int64_t r = 0; r < rows; ++r) {
        const uint16_t* a = x + r * width;
        for (int64_t c = 0; c < columns; ++c) {
            const uint16_t* b = w + c * width;
            float lane[32];
            for (int l = 0; l < 32; ++l) {
                float s = 0.0f;
                for (int64_t k = l; k < width; k += 32)
                    s += oracle_f16_to_f32(a[k]) * oracle_f16_to_f32(b[k]);
                lane[l] = s;
            }
            for (int d = 16; d >= 1; d /= 2)
                for (int l = 0; l < d; ++l)
                    lane[l] += lane[l + d];
            out[r * columns + c] = oracle_f32_to_f16(lane[0]);
        }
    }
}
