/*
 * omni_int8 — MI355X (gfx950) int8 quantised-matmul hot path, C ABI.
 *
 * This is the drop-in boundary for omni-rs's int8 matmul operator. Every
 * entry point takes plain device pointers, sizes and a HIP stream handle
 * (hipStream_t passed as void*, NULL = the null stream). The library
 * allocates nothing: the caller owns every buffer, including the workspace
 * omni_try_int8_gemm needs. Calls are asynchronous on `stream`; calls on
 * distinct streams may run concurrently.
 *
 * Return status (mirrors the reference's Option convention):
 *   OMNI_OK (0)            the work was enqueued;
 *   OMNI_NOT_HANDLED (1)   shapes disagree — the reference returns None here
 *                          and its caller panics or falls back;
 *   OMNI_NO_DEVICE (2)     the current device is not gfx950;
 *   OMNI_BAD_ARGUMENT (3)  a null pointer, a negative size, an unknown dtype
 *                          or a misaligned buffer;
 *   OMNI_HIP_ERROR (-1)    a HIP launch failed; omni_int8_last_error() says why.
 *
 * Data layouts (all row-major, no padding):
 *   x            [rows][width] f32 or f16 activations, row stride ld_x elements;
 *   x_packed     [rows][width] int8 codes == [rows][width/4] int32 words, the
 *                first code in the lowest byte;
 *   w_packed     [columns][width] int8 == [columns][width/4] int32 words
 *                (byte-identical to the checkpoint's row-major int8 [out][in]);
 *   w_scale      [columns] f32, w_zero [columns] int32;
 *   out          [rows][columns].
 */
#ifndef OMNI_INT8_H
#define OMNI_INT8_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum omni_status {
    OMNI_OK = 0,
    OMNI_NOT_HANDLED = 1,
    OMNI_NO_DEVICE = 2,
    OMNI_BAD_ARGUMENT = 3,
    OMNI_HIP_ERROR = -1,
};

enum omni_dtype {
    OMNI_F32 = 0,
    OMNI_F16 = 1,
};

/* W8A8 GEMM lowering selection for omni_w8a8_gemm / omni_try_int8_gemm.
 * Replaces crates/omni-kernel/src/int8_tensorops.rs:15-24 (matmul2d_lowered /
 * enabled). The reference's switch OMNI_CONVROT_TENSOROPS=0 forces the
 * scalar kernel here too, as does OMNI_INT8_FORCE_SCALAR=1; both are read on
 * every call, as the reference reads its variable. Otherwise the int8-MFMA
 * kernel runs whenever width % 16 == 0 and the scalar v_dot4 kernel
 * otherwise. */
enum omni_w8a8_lowering {
    OMNI_LOWERING_AUTO = 0,
    OMNI_LOWERING_MFMA = 1,
    OMNI_LOWERING_SCALAR = 2,
};

/* 1 when `device` is a gfx950 GPU, else 0; the answer is cached per device.
 * Replaces crates/omni-kernel/src/int8_tensorops.rs:26-43 (apple10: the
 * cached per-device family probe) and the backend check of
 * crates/omni-kernel/src/lib.rs:32-47 (device). */
int omni_int8_arch_supported(int device);

/* Lowering that omni_w8a8_gemm would pick for this width (after the
 * OMNI_CONVROT_TENSOROPS=0 / OMNI_INT8_FORCE_SCALAR=1 overrides). Mirrors
 * int8_tensorops.rs:15-20. */
int omni_w8a8_lowering(int64_t width);

/* Message for the last non-OK status returned on this thread. */
const char* omni_int8_last_error(void);

/* Tuning and test knobs: the OMNI_W8A8_TILE / _SPLITS, OMNI_W8A16_* ,
 * OMNI_W4A16_* and OMNI_F16_* variables that pin a kernel variant or a
 * split count. The library reads them from the environment once per
 * process, not on every launch; this call overrides one for the rest of the
 * process (thread-safe): mode 2 = `value`, mode 1 = unset (the shape rules
 * decide), mode 0 = back to the environment's value. No counterpart in the
 * reference (its one switch, OMNI_CONVROT_TENSOROPS, int8_tensorops.rs:15-20,
 * is still read on every call, as there). OMNI_BAD_ARGUMENT for an unknown
 * name. */
int omni_int8_set_tuning(const char* name, int mode, int value);

/* Per-row dynamic symmetric int8 quantisation.
 * Replaces quantize_rows + quantize_i8, crates/omni-kernel/src/int8_matmul.rs:23-118
 * (host twin: crates/omni-kernel/src/int8_host.rs:31-39):
 *   row_scale = max(max|x| / 127, 1e-30); code = round-half-away(x / row_scale)
 *   clamped to [-128, 127]; x_sum[row] = sum of the row's codes.
 * x_dtype is OMNI_F32 or OMNI_F16 (the reference casts f16 to f32 first,
 * int8_matmul.rs:525; an f16 value is exact in f32). width % 4 == 0.
 * x_sum may be NULL. */
int omni_int8_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t width,
                            int64_t ld_x, int32_t* x_packed, float* x_scale, int32_t* x_sum,
                            void* stream);

/* W8A8 int8 x int8 -> int32 GEMM with the fused reference epilogue.
 * Replaces int8_dot / int8_dot_tile64 / store, crates/omni-kernel/src/int8_matmul.rs:145-373:
 *   acc[m][n] = sum_k x_packed[m][k] * w_packed[n][k]           (exact int32)
 *   out[m][n] = f32(acc - x_sum[m] * w_zero[n]) * x_scale[m] * w_scale[n]
 *               (+ bias[n] in f32 when bias != NULL)
 * then stored as out_dtype (OMNI_F32: the reference's output; OMNI_F16: one
 * round-to-nearest-even cast, what convrot.rs:91 does after the op).
 * acc_dump, when not NULL, receives the raw int32 accumulators [rows][columns]
 * (for bit-exact checks). width % 4 == 0; |acc| must fit in int32, which holds
 * for width <= 131072. x_sum may be NULL only when w_zero is NULL (zero
 * points all 0). `lowering` is an omni_w8a8_lowering value. */
int omni_w8a8_gemm(const int32_t* x_packed, const float* x_scale, const int32_t* x_sum,
                   const int32_t* w_packed, const float* w_scale, const int32_t* w_zero,
                   const float* bias, int64_t rows, int64_t columns, int64_t width, void* out,
                   int out_dtype, int32_t* acc_dump, int lowering, void* stream);

/* Bytes of workspace omni_w8a8_gemm_ws uses for this shape on the current
 * device: split-K partial sums (int32 [splits][rows][columns]) for shapes
 * whose 256 x 128 output tiles alone would leave most CUs idle (the
 * reference's own 256-row benchmark shapes); 0 when the shape does not
 * split. */
size_t omni_w8a8_gemm_workspace_size(int64_t rows, int64_t columns, int64_t width);

/* omni_w8a8_gemm with a caller-owned workspace (256-byte aligned, or NULL
 * with workspace_bytes 0), which lets the MFMA GEMM split K across
 * workgroups (a second launch adds the partial sums and applies the
 * epilogue); with less than omni_w8a8_gemm_workspace_size bytes it splits
 * less, with none it runs as omni_w8a8_gemm. The workspace needs no
 * initialisation; calls that overlap in time must not share one. The int32
 * partial sums add exactly, so outputs (and acc_dump) are bit-identical to
 * omni_w8a8_gemm's. */
int omni_w8a8_gemm_ws(const int32_t* x_packed, const float* x_scale, const int32_t* x_sum,
                      const int32_t* w_packed, const float* w_scale, const int32_t* w_zero,
                      const float* bias, int64_t rows, int64_t columns, int64_t width, void* out,
                      int out_dtype, int32_t* acc_dump, int lowering, void* workspace,
                      size_t workspace_bytes, void* stream);

/* Workspace bytes omni_try_int8_gemm needs for `rows` x `width` activations
 * (codes, row scales and row sums, each 256-byte aligned). */
size_t omni_try_int8_gemm_workspace_size(int64_t rows, int64_t width);

/* Workspace bytes with which omni_try_int8_gemm and omni_convrot_linear also
 * split K for this shape (omni_try_int8_gemm_workspace_size(rows, width)
 * plus omni_w8a8_gemm_workspace_size(rows, columns, width)): the reference's
 * own 256-row shapes run in a fraction of the unsplit time. No counterpart
 * in the reference, whose try_int8_gemm allocates per call
 * (int8_matmul.rs:386-471). The workspace needs no initialisation; outputs
 * are bit-identical to the unsplit call. */
size_t omni_try_int8_gemm_split_workspace_size(int64_t rows, int64_t columns, int64_t width);

/* The whole reference operator, x @ W^T after per-row int8 quantisation of x.
 * Replaces try_int8_gemm, crates/omni-kernel/src/int8_matmul.rs:505-560
 * (and its launch :386-471). Shape guard as :517-521: columns = scale_len;
 * returns OMNI_NOT_HANDLED (the reference's None) unless width % 4 == 0,
 * w_packed_len == columns * width / 4 and zero_len == columns.
 * x [rows][width] (x_dtype f32 or f16, contiguous) -> out f32 [rows][columns].
 * workspace: at least omni_try_int8_gemm_workspace_size(rows, width) bytes,
 * 256-byte aligned; with omni_try_int8_gemm_split_workspace_size(rows,
 * columns, width) bytes the GEMM may split K (same results; one more
 * launch, the reduction of the partial sums). */
int omni_try_int8_gemm(const void* x, int x_dtype, int64_t rows, int64_t width,
                       const int32_t* w_packed, int64_t w_packed_len, const float* w_scale,
                       int64_t scale_len, const int32_t* w_zero, int64_t zero_len, float* out,
                       void* workspace, size_t workspace_bytes, void* stream);

/* Bytes of the static device scratch behind omni_try_int8_gemm_noalloc. */
#define OMNI_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* omni_try_int8_gemm without its workspace argument, for callers that cannot
 * allocate device memory: code under HIP graph capture that must not call
 * hipMalloc, tight serving loops, harnesses that forbid allocation. It has
 * no counterpart in the reference. The codes, row scales and row sums live
 * in a static device array of OMNI_NOALLOC_SCRATCH_BYTES that each GPU the
 * library runs on holds until the process ends; shapes whose
 * omni_try_int8_gemm_workspace_size(rows, width) exceeds it are rejected
 * with OMNI_BAD_ARGUMENT (64 MiB covers 4352 x 12288 activations); where
 * omni_try_int8_gemm_split_workspace_size fits, the GEMM splits K as
 * omni_try_int8_gemm does with that workspace. The call
 * allocates nothing. Every call on one GPU shares that GPU's array: calls
 * that overlap in time on one GPU (other streams, other host threads) race
 * on it and must be serialised by the caller. Arguments, guard, result and
 * NOT_HANDLED convention are omni_try_int8_gemm's. */
int omni_try_int8_gemm_noalloc(const void* x, int x_dtype, int64_t rows, int64_t width,
                               const int32_t* w_packed, int64_t w_packed_len, const float* w_scale,
                               int64_t scale_len, const int32_t* w_zero, int64_t zero_len,
                               float* out, void* stream);

/* ConvRot activation rotation fused into per-row quantisation.
 * Replaces the rotate step of Int8Linear::forward followed by
 * try_int8_gemm's quantize_rows: crates/qwen-image/src/convrot.rs:86-88 and
 * :113-119 (rotate), the matrix of :121-149 (hadamard, sign_negative), then
 * crates/omni-kernel/src/int8_matmul.rs:23-118.
 *   r = each group of 256 consecutive elements of a row times H,
 *   H = 2^-4 * H4 (x) H4 (x) H4 (x) H4 with H4[a][b] = -1 iff a ^ b == 3;
 *   then codes, row scales and row sums of r as omni_int8_quantize_rows.
 * r is computed in f32 by a radix-4 fast transform, not by a 256-term dot:
 * only its rounding differs from the reference's f32 matmul (the error is
 * at most 12 * 2^-24 * sum|x| over the group, in units of 16 r), so a code can
 * differ by one where r / row_scale lies within that of k + 0.5. From r on,
 * the quantisation is omni_int8_quantize_rows' own: the correctly rounded
 * quotient r / row_scale, then round half away from zero.
 * group must be 256 (convrot.rs:12), width % 256 == 0 (convrot.rs:39-43),
 * else OMNI_NOT_HANDLED; x and every row start (ld_x) 16-byte aligned,
 * x_packed 16-byte aligned. x_sum may be NULL. */
int omni_convrot_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t width,
                               int64_t ld_x, int64_t group, int32_t* x_packed, float* x_scale,
                               int32_t* x_sum, void* stream);

/* The whole ConvRot linear layer: rotation + quantisation + W8A8 GEMM, output
 * in the model precision. Replaces Int8Linear::forward with project,
 * crates/qwen-image/src/convrot.rs:81-102. Shape guard as omni_try_int8_gemm
 * (columns = scale_len) plus width % 256 == 0; OMNI_NOT_HANDLED where the
 * reference panics. out_dtype OMNI_F16 (the model's Precision::F16: the f32
 * result rounded once to nearest even, convrot.rs:91) or OMNI_F32.
 * x contiguous [rows][width]; workspace as omni_try_int8_gemm (at least
 * omni_try_int8_gemm_workspace_size(rows, width) bytes, 256-byte aligned;
 * with omni_try_int8_gemm_split_workspace_size bytes the GEMM may split K). */
int omni_convrot_linear(const void* x, int x_dtype, int64_t rows, int64_t width,
                        const int32_t* w_packed, int64_t w_packed_len, const float* w_scale,
                        int64_t scale_len, const int32_t* w_zero, int64_t zero_len, void* out,
                        int out_dtype, void* workspace, size_t workspace_bytes, void* stream);

/* Weight-only int8 linear with fp16 per-output-channel scales (W8A16).
 * No single counterpart in the reference: it follows the reference's
 * dequantisation convention, w_deq = w * scale, f32 accumulation
 * (crates/omni-kernel/src/int8_matmul.rs:644-649; the weight-only CPU route
 * crates/minicpm-v/src/quant.rs:186-200) and the decode GEMV guard style of
 * crates/breeze-tts/src/metal_depth.rs:84-123.
 *   out[m][n] = f16(scale[n] * sum_k x[m][k] * w[n][k] + bias[n])
 * x f16 [rows][width], w int8 [columns][width], scale f16 [columns],
 * bias f16 [columns] or NULL, out f16 [rows][columns]. width % 16 == 0.
 * rows <= 4 with width <= 16384 runs the HBM-bound GEMV, up to 16 rows (up
 * to 64 on smaller matrices) the skinny MFMA kernel, more rows the
 * fp16-MFMA GEMM. */
int omni_w8a16_gemm(const uint16_t* x, const int8_t* w, const uint16_t* scale,
                    const uint16_t* bias, int64_t rows, int64_t columns, int64_t width,
                    uint16_t* out, void* stream);

/* Bytes of workspace omni_w8a16_gemm_ws uses for this shape on the current
 * device: split-K partial sums (f32 [splits][rows][columns]) for GEMM shapes
 * whose output tiles alone would leave CUs idle; 0 when the shape does not
 * split. */
size_t omni_w8a16_gemm_workspace_size(int64_t rows, int64_t columns, int64_t width);

/* omni_w8a16_gemm with a caller-owned workspace (256-byte aligned, or NULL
 * with workspace_bytes 0), which lets the GEMM split K across workgroups;
 * with less than omni_w8a16_gemm_workspace_size bytes it splits less, with
 * none it runs as omni_w8a16_gemm. Same contract otherwise (the split sums
 * K in a different order: f32 rounding differs, not the operation). */
int omni_w8a16_gemm_ws(const uint16_t* x, const int8_t* w, const uint16_t* scale,
                       const uint16_t* bias, int64_t rows, int64_t columns, int64_t width,
                       uint16_t* out, void* workspace, size_t workspace_bytes, void* stream);

/* Weight-only int4 linear (W4A16), the MiniCPM-V pack-quantized format.
 * Replaces the packed-int4 matmul of crates/minicpm-v/src/quant.rs:43-58
 * (PackedWeight::matmul_transpose, x @ W^T) with the weight layout that
 * load_packed reads (:145-201): w_packed [columns][width / 2] bytes, two
 * values per byte, low nibble first, each stored plus 8 (unpack_int4,
 * :22-29); scale_bf16 [columns][width / group] bf16, one per group of
 * consecutive values along the row (:74-81, :186-200, GROUP_SIZE = 128).
 *   out[m][n] = f16(sum_k x[m][k] * (q[n][k] * scale[n][k / group]) + bias[n])
 * x f16 [rows][width], bias f16 [columns] or NULL, out f16 [rows][columns].
 * width % group == 0 and group % 32 == 0, else OMNI_NOT_HANDLED; x and
 * w_packed 16-byte aligned. rows <= 4 (width <= 32768) runs the HBM-bound
 * GEMV, up to 16 rows (up to 64 on smaller matrices) the skinny MFMA kernel,
 * more rows the fp16-MFMA GEMM. */
int omni_w4a16_gemm(const uint16_t* x, const uint8_t* w_packed, const uint16_t* scale_bf16,
                    int64_t group, const uint16_t* bias, int64_t rows, int64_t columns,
                    int64_t width, uint16_t* out, void* stream);

/* Bytes of workspace omni_w4a16_gemm_ws uses for this shape on the current
 * device: split-K partial sums (f32 [splits][rows][columns]) for the shapes
 * that split (GEMM shapes, and 5..16 rows over long K and many columns); 0
 * when the shape does not split. No counterpart in the reference: it
 * serves omni_w4a16_gemm_ws. */
size_t omni_w4a16_gemm_workspace_size(int64_t rows, int64_t columns, int64_t width, int64_t group);

/* omni_w4a16_gemm with a caller-owned workspace (256-byte aligned, or NULL
 * with workspace_bytes 0), which lets the GEMM split K across workgroups;
 * with less than omni_w4a16_gemm_workspace_size bytes it splits less, with
 * none it runs as omni_w4a16_gemm. Same contract otherwise (the split sums
 * K in a different order: f32 rounding differs, not the operation). No
 * counterpart in the reference: the extension of omni_w4a16_gemm that
 * split K needs, as omni_w8a16_gemm_ws is for omni_w8a16_gemm. */
int omni_w4a16_gemm_ws(const uint16_t* x, const uint8_t* w_packed, const uint16_t* scale_bf16,
                       int64_t group, const uint16_t* bias, int64_t rows, int64_t columns,
                       int64_t width, uint16_t* out, void* workspace, size_t workspace_bytes,
                       void* stream);

/* fp16 decode GEMV, the Breeze TTS depth decoder's linear. Replaces
 * crates/breeze-tts/src/metal_depth.rs:84-123 (try_linear) and the kernel it
 * launches (gemv_kernel :13-35 via raw_gemv :36-83):
 *   out[m][n] = f16(sum_k f32(x[m][k]) * f32(w[n][k]))
 * x f16 [rows][width], w f16 [columns][width] (output-major: the transposed
 * view of the Linear's [width][columns] weight that the reference's custom
 * path takes, :42-44), out f16 [rows][columns]. f32 accumulation; the
 * summation order is not the reference's. The reference's guard (:94-104):
 * 1 <= rows <= 64, width > 0, width % 32 == 0, 1 <= columns <= 4096, else
 * OMNI_NOT_HANDLED (its None). x and w 16-byte aligned. */
int omni_f16_gemv(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t columns,
                  int64_t width, uint16_t* out, void* stream);

/* fp16 GEMM for the Qwen-Image DiT linears. Replaces
 * crates/qwen-image/src/metal_tensorops.rs:161-203 (try_linear) and its
 * 64 x 64 matmul2d shader (tensorops.metal:18-39): out = f16(x @ w^T) with
 * f32 accumulation, x f16 [rows][width], w f16 [columns][width], out f16
 * [rows][columns]. The reference's guard (:174-187): 256 <= rows <= 65535,
 * width and columns multiples of 64 in 4096..=12288, else OMNI_NOT_HANDLED;
 * OMNI_QWEN_TENSOROPS=0 in the environment (read once) turns it off, as
 * :165-169 does. x and w 16-byte aligned. */
int omni_f16_gemm(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t columns,
                  int64_t width, uint16_t* out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* OMNI_INT8_H */
