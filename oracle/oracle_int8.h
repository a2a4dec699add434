/*
 * CPU oracle for the int8 quantised-matmul hot path — TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg load
 * this library, and only as the checker or the timed CPU baseline. The
 * product library never links it.
 *
 * The reference (GoooIce/omni-rs) is Rust 2024 with crates.io dependencies
 * (burn 0.21, cubecl 0.10, wgpu 29); no Rust toolchain exists in this image,
 * so there is no oracle/_ref build: the restatement below is pinned instead.
 *
 * Parity pins (tests/test_oracle.py), one line per function:
 *   oracle_f16_to_f32 / oracle_f32_to_f16 — all 65536 halves and 2^20 floats
 *       (ties, subnormals, overflow) against numpy.float16.
 *   oracle_round_half_away — the ties +-0.5, +-1.5, +-2.5, +-127.5, +-128.5
 *       and the clamp, as int8_host.rs:3-10 defines them.
 *   oracle_unpack_i8 / oracle_pack_i8 — brute force on every byte value and
 *       the byte identity with row-major int8 (convrot.rs:151-160).
 *   oracle_quantize_rows — the hand codes [32,-64,16,127] for x=[1,-2,0.5,4]
 *       (int8_matmul.rs:757), exact half-way inputs, the 1e-30 floor on a zero
 *       row, |dequant - x| <= scale/2, and a numpy vectorised float32
 *       restatement on random rows.
 *   oracle_int8_acc — numpy int64 matmul (an exact integer product) and the
 *       hand accumulator -300 (int8_matmul.rs:757).
 *   oracle_epilogue / oracle_int8_gemm — the hand value -411/127
 *       (int8_matmul.rs:700-732) and the prototype check shapes (5,12,6) and
 *       (17,36,14) (prototypes/int8-gemm/src/main.rs:69-89) against
 *       oracle_dequant_reference within 1e-3, with a +1 negative control
 *       (int8_matmul.rs:768).
 *   oracle_w8a8_finish — equals oracle_int8_gemm on the f32 path; the fp16
 *       output equals numpy's float16 cast of that value plus the bias.
 *   oracle_dequant_reference — the hand value -411/127 within 1e-4
 *       (int8_matmul.rs:709) and the 64x64x64 tile fixture (:734-747).
 *   oracle_w8a16_f64 — numpy float64 matmul of the same operands.
 *   oracle_w8a16_gemm — within 1e-2 relative of oracle_w8a16_f64 (the
 *       tolerance the path is specified to) and exact on integer-valued cases.
 *   oracle_unpack_int4 — every byte value against the rule of quant.rs:22-29
 *       and its own test values (8 -> 0, 0 -> -8, 0xF -> 7).
 *   oracle_bf16_to_f32 — every bf16 bit pattern against numpy's float32 top
 *       half (the definition of bf16).
 *   oracle_w4a16_dequant / _f64 / _gemm — the synthetic weights of
 *       quant.rs:419-462 round-trip through pack/unpack exactly; the route is
 *       within the reference test's 5e-2 (quant.rs:503) of the f64 truth and
 *       equals numpy restating dequantise -> f16 -> f32 dot on small cases.
 *   oracle_f16_linear_f64 — numpy float64 matmul of the same halves, and the
 *       closed form width * a * b for constant operands.
 *   oracle_f16_gemv — within the reference test's 0.002 + 0.001 |e| of
 *       oracle_f16_linear_f64 on its shapes and values
 *       (metal_depth_tests.rs:16-80), and equal to numpy's f32 lane-strided
 *       sums cast to float16.
 *   oracle_hadamard / oracle_rotate — symmetry, H*H = I within 1e-4 and the
 *       float-matmul cancellation (convrot.rs:169-220); the 4x4 base
 *       H4[a][b] = -1 iff a^b == 3 (convrot.rs:139-140); scipy.linalg.hadamard
 *       has the same absolute values and orthogonality.
 */
#ifndef OMNI_ORACLE_INT8_H
#define OMNI_ORACLE_INT8_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float oracle_f16_to_f32(uint16_t h);
uint16_t oracle_f32_to_f16(float f);

int32_t oracle_round_half_away(float value);
void oracle_unpack_i8(const int32_t* words, int64_t count, int8_t* out);
void oracle_pack_i8(const int8_t* codes, int64_t count, int32_t* words);
void oracle_quantize_rows(const float* x, int64_t rows, int64_t width, int64_t ld,
                          int8_t* codes, float* row_scale, int32_t* row_sum);
void oracle_int8_acc(const int8_t* codes, const int8_t* w, int64_t rows, int64_t columns,
                     int64_t width, int32_t* acc);
float oracle_epilogue(int32_t acc, int32_t sum, int32_t zero, float row_scale, float w_scale);
void oracle_int8_gemm(const float* x, int64_t rows, int64_t width, const int8_t* w,
                      const float* scale, const int32_t* zero, int64_t columns, float* out);
/* The same, rows spread over `threads` OpenMP threads; bit-identical output
 * (pinned against oracle_int8_gemm in tests/test_oracle.py). */
void oracle_int8_gemm_threads(const float* x, int64_t rows, int64_t width, const int8_t* w,
                              const float* scale, const int32_t* zero, int64_t columns,
                              float* out, int threads);
void oracle_w8a8_finish(const int32_t* acc, const int32_t* row_sum, const float* row_scale,
                        const float* w_scale, const int32_t* w_zero, const float* bias,
                        int64_t rows, int64_t columns, float* out_f32, uint16_t* out_f16);
void oracle_dequant_reference(const float* x, int64_t rows, int64_t width, const int8_t* w,
                              const float* scale, const int32_t* zero, int64_t columns,
                              float* out);

void oracle_w8a16_f64(const uint16_t* x, int64_t rows, int64_t width, const int8_t* w,
                      const uint16_t* scale, const uint16_t* bias, int64_t columns, double* out);
void oracle_w8a16_gemm(const uint16_t* x, int64_t rows, int64_t width, const int8_t* w,
                       const uint16_t* scale, const uint16_t* bias, int64_t columns,
                       uint16_t* out);

int oracle_hadamard_sign_negative(uint64_t row, uint64_t column, uint64_t size);
void oracle_hadamard(int64_t size, float* matrix);
void oracle_rotate(const float* x, int64_t rows, int64_t width, int64_t group, float* out);

/* The kernel's radix-4 fast transform of each group of 256 (u = 16 r, op for
 * op as omni-rs_amd/csrc/convrot.hip), and the kernel's codes from it. Pinned
 * against the exact rotation within the transform's error bound and exactly
 * on unit vectors (tests/test_convrot.py). */
void oracle_convrot_fwht(const float* x, int64_t rows, int64_t width, int64_t ld, float* u);
void oracle_convrot_quantize_fwht(const float* x, int64_t rows, int64_t width, int64_t ld,
                                  int8_t* codes, float* row_scale, int32_t* row_sum);

void oracle_unpack_int4(const uint8_t* packed, int64_t bytes, int8_t* out);
float oracle_bf16_to_f32(uint16_t b);
void oracle_w4a16_dequant(const uint8_t* packed, const uint16_t* scale_bf16, int64_t rows,
                          int64_t width, int64_t group, int f16_round, float* w_deq);
void oracle_w4a16_f64(const uint16_t* x, int64_t rows, int64_t width, const uint8_t* packed,
                      const uint16_t* scale_bf16, int64_t group, const uint16_t* bias,
                      int64_t columns, double* out);
void oracle_w4a16_gemm(const uint16_t* x, int64_t rows, int64_t width, const uint8_t* packed,
                       const uint16_t* scale_bf16, int64_t group, const uint16_t* bias,
                       int64_t columns, uint16_t* out);
void oracle_f16_linear_f64(const uint16_t* x, int64_t rows, int64_t width, const uint16_t* w,
                           int64_t columns, double* out);
void oracle_f16_gemv(const uint16_t* x, int64_t rows, int64_t width, const uint16_t* w,
                     int64_t columns, uint16_t* out);

#ifdef __cplusplus
}
#endif

#endif
