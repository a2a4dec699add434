// Host-side launchers of the gfx950 kernels (internal to libomni_int8).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace omni {

// Tuning and test knobs (kernel pins, split overrides). Each one's value is a
// test's override when one is set (omni_int8_set_tuning), else the
// environment variable of the knob's name as read once per process, else
// `unset`; reading one on a launch is two atomic loads, no getenv.
enum class Knob : int {
    W8A8Tile,          // OMNI_W8A8_TILE
    W8A8Splits,        // OMNI_W8A8_SPLITS
    W8A16Gemv,         // OMNI_W8A16_GEMV
    F16Gemv,           // OMNI_F16_GEMV
    W8A16Skinny,       // OMNI_W8A16_SKINNY
    W8A16SkinnySplit,  // OMNI_W8A16_SKINNY_SPLIT
    W8A16Tile,         // OMNI_W8A16_TILE
    W8A16Splits,       // OMNI_W8A16_SPLITS
    W8A16Route,        // OMNI_W8A16_ROUTE
    W4A16Gemv,         // OMNI_W4A16_GEMV
    W4A16SkinnySplit,  // OMNI_W4A16_SKINNY_SPLIT
    W4A16Splits,       // OMNI_W4A16_SPLITS
    W4A16Tile,         // OMNI_W4A16_TILE
    F16Tile,           // OMNI_F16_TILE
    Count
};
int knob(Knob k, int unset);

// Compute units of the current device (cached per device, thread-safe).
int num_cus();

hipError_t launch_quantize_rows(const void* x, bool x_is_f16, int64_t rows, int64_t width,
                                int64_t ld, uint8_t* codes, float* scale, int32_t* sum,
                                hipStream_t stream);

// ConvRot group-256 Hadamard rotation fused into quantize_rows (convrot.hip);
// width % 256 == 0, x and every row start 16-byte aligned.
hipError_t launch_convrot_quantize(const void* x, bool x_is_f16, int64_t rows, int64_t width,
                                   int64_t ld, uint8_t* codes, float* scale, int32_t* sum,
                                   hipStream_t stream);

struct W8A8Args {
    const uint8_t* x;      // [rows][width] int8 codes
    const float* x_scale;  // [rows]
    const int32_t* x_sum;  // [rows] or null when w_zero is null
    const uint8_t* w;      // [columns][width] int8
    const float* w_scale;  // [columns]
    const int32_t* w_zero; // [columns] or null (all zero)
    const float* bias;     // [columns] or null
    void* out;             // [rows][columns] f32 or f16
    int32_t* acc_dump;     // [rows][columns] or null
    int64_t rows, columns, width;
    bool out_f16;
    int32_t* partial = nullptr;  // split-K: int32 [splits][rows][columns]
    int64_t partial_elems = 0;   // int32s available at `partial`
};

hipError_t launch_w8a8_mfma(const W8A8Args& a, hipStream_t stream);
// int32s of split-K partial sums launch_w8a8_mfma uses for this shape on the
// current device (0: no split); with fewer in W8A8Args it splits less.
int64_t w8a8_partial_elems(int64_t rows, int64_t columns, int64_t width);
hipError_t launch_w8a8_scalar(const W8A8Args& a, hipStream_t stream);

struct W8A16Args {
    const _Float16* x;      // [rows][width]
    const int8_t* w;        // [columns][width] int8, [columns][width / 2] packed int4, or f16
    const _Float16* scale;  // [columns] (int8 weights)
    const _Float16* bias;   // [columns] or null
    _Float16* out;          // [rows][columns]
    int64_t rows, columns, width;
    const uint16_t* gscale = nullptr;  // int4 weights: bf16 [columns][width / group]
    int64_t group = 0;                  // int4 weights: values per scale along K
    float* partial = nullptr;           // split-K: f32 [splits][rows][columns]
    int64_t partial_elems = 0;          // floats available at `partial`
};

// Whether an LDS-DMA ring GEMM can run this shape (int8, int4: also the
// group and scale layout); without one launch_w8a16_mfma and
// launch_w4a16_mfma take the register-staged tiled kernels.
bool w8a16_ring_usable(const W8A16Args& a);
bool w4a16_ring_usable(const W8A16Args& a);

hipError_t launch_w8a16_gemv(const W8A16Args& a, hipStream_t stream);
hipError_t launch_w8a16_skinny(const W8A16Args& a, hipStream_t stream);
hipError_t launch_w8a16_mfma(const W8A16Args& a, hipStream_t stream);
// Floats of split-K partial sums launch_w8a16_mfma uses for this shape on the
// current device (0: no split); with fewer in W8A16Args it splits less.
int64_t w8a16_partial_elems(int64_t rows, int64_t columns, int64_t width);
// The same for launch_w8a16_skinny (up to 16 rows: split-K skinny kernel).
int64_t w8a16_skinny_partial_elems(int64_t rows, int64_t columns, int64_t width);

// W4A16 (w8a16.hip): packed int4 weights (two per byte, low nibble first,
// offset by 8) with bf16 scales per group of K values.
hipError_t launch_w4a16_gemv(const W8A16Args& a, hipStream_t stream);
hipError_t launch_w4a16_skinny(const W8A16Args& a, hipStream_t stream);
hipError_t launch_w4a16_mfma(const W8A16Args& a, hipStream_t stream);
// Floats of split-K partial sums launch_w4a16_mfma uses for this shape on the
// current device (0: no split); with fewer in W8A16Args it splits less.
int64_t w4a16_partial_elems(int64_t rows, int64_t columns, int64_t width, int64_t group);
// The same for launch_w4a16_skinny (up to 16 rows: split-K skinny kernel).
int64_t w4a16_skinny_partial_elems(int64_t rows, int64_t columns, int64_t width);

// fp16 linear (w8a16.hip): w is f16 [columns][width] (cast to int8_t*), no
// scale; out[m][n] = f16(sum_k x[m][k] * w[n][k] + bias[n]).
hipError_t launch_f16_gemv(const W8A16Args& a, hipStream_t stream);
hipError_t launch_f16_skinny(const W8A16Args& a, hipStream_t stream);
hipError_t launch_f16_mfma(const W8A16Args& a, hipStream_t stream);

}  // namespace omni
