// omni_kernel — C++ host mirror of omni-rs's int8 matmul operator API, over
// the C ABI in omni_int8.h. Header-only, C++17.
//
// The reference is Rust (crates/omni-kernel); its operator is
//   pub fn try_int8_gemm<B: Backend>(x: Tensor<B,2>, w_packed: Tensor<B,1,Int>,
//       w_scale: Tensor<B,1>, w_zero: Tensor<B,1,Int>) -> Option<Tensor<B,2>>
// (crates/omni-kernel/src/int8_matmul.rs:511-516). This header keeps its name,
// argument meaning and None-on-shape-mismatch behaviour with a minimal device
// tensor type in place of Burn's Tensor. Tensors are device buffers (HIP);
// the operator allocates its output and workspace through an Allocator, as
// Burn allocates them inside the reference op (int8_matmul.rs:403-406).
#ifndef OMNI_KERNEL_HPP
#define OMNI_KERNEL_HPP

#include <hip/hip_runtime.h>

#include <cstdint>
#include <optional>
#include <stdexcept>
#include <string>
#include <vector>

#include "omni_int8.h"

namespace omni_kernel {

enum class DType { F32, F16, I32, I8 };

inline size_t dtype_size(DType d) {
    switch (d) {
        case DType::F32: return 4;
        case DType::F16: return 2;
        case DType::I32: return 4;
        case DType::I8: return 1;
    }
    return 0;
}

// A contiguous row-major device tensor (non-owning view).
struct DeviceTensor {
    void* data = nullptr;
    std::vector<int64_t> shape;
    DType dtype = DType::F32;

    int64_t dim(size_t i) const { return shape.at(i); }
    int64_t numel() const {
        int64_t n = 1;
        for (int64_t s : shape) n *= s;
        return n;
    }
    size_t bytes() const { return (size_t)numel() * dtype_size(dtype); }
};

// Device memory for op outputs and scratch. The default uses the stream-ordered
// hipMallocAsync / hipFreeAsync.
struct Allocator {
    virtual ~Allocator() = default;
    virtual void* allocate(size_t bytes, hipStream_t stream) = 0;
    virtual void release(void* p, hipStream_t stream) = 0;
};

struct HipAllocator final : Allocator {
    void* allocate(size_t bytes, hipStream_t stream) override {
        void* p = nullptr;
        if (hipMallocAsync(&p, bytes ? bytes : 1, stream) != hipSuccess)
            throw std::runtime_error("hipMallocAsync failed");
        return p;
    }
    void release(void* p, hipStream_t stream) override { (void)hipFreeAsync(p, stream); }
};

// A non-OK status from the library other than "not handled" (the reference's
// None). Device-side failures are raised here; the reference only logs them
// (prototypes/int8-gemm/src/main.rs:38-44).
struct Int8Error : std::runtime_error {
    int status;
    Int8Error(int s, const std::string& what) : std::runtime_error(what), status(s) {}
};

inline void check(int status) {
    if (status != OMNI_OK && status != OMNI_NOT_HANDLED)
        throw Int8Error(status, omni_int8_last_error());
}

// gfx950 gate of the current device (int8_tensorops.rs:26-43 analog).
inline bool device_supported() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    return omni_int8_arch_supported(dev) != 0;
}

namespace int8_matmul {

// x @ W^T after per-row symmetric int8 quantisation of x.
// crates/omni-kernel/src/int8_matmul.rs:505-560. w_packed holds n * (k / 4)
// little-endian int8 groups (int32 words); w_scale (f32) and w_zero (int32)
// are per output row. Returns an f32 [rows, n] tensor allocated from
// `alloc`, or std::nullopt when the shapes disagree (:517-521) or the current
// device is not gfx950. x may be f32
// or f16 (f16 is exact in f32; the reference casts to f32 first, :525).
inline std::optional<DeviceTensor> try_int8_gemm(const DeviceTensor& x, const DeviceTensor& w_packed,
                                                 const DeviceTensor& w_scale,
                                                 const DeviceTensor& w_zero, Allocator& alloc,
                                                 hipStream_t stream = nullptr) {
    if (x.shape.size() != 2 || w_packed.shape.size() != 1 || w_scale.shape.size() != 1 ||
        w_zero.shape.size() != 1)
        return std::nullopt;
    const int64_t rows = x.dim(0), width = x.dim(1), columns = w_scale.dim(0);
    if (width % 4 != 0 || w_packed.dim(0) != columns * width / 4 || w_zero.dim(0) != columns)
        return std::nullopt;
    if ((x.dtype != DType::F32 && x.dtype != DType::F16) || w_packed.dtype != DType::I32 ||
        w_scale.dtype != DType::F32 || w_zero.dtype != DType::I32)
        throw Int8Error(OMNI_BAD_ARGUMENT, "try_int8_gemm: x f32/f16, w_packed i32, w_scale f32, w_zero i32");
    DeviceTensor out{alloc.allocate((size_t)(rows * columns) * 4, stream), {rows, columns}, DType::F32};
    // Room for the split-K partial sums too: the reference's 256-row shapes
    // split K.
    const size_t ws_bytes = omni_try_int8_gemm_split_workspace_size(rows, columns, width);
    void* ws = alloc.allocate(ws_bytes, stream);
    const int st = omni_try_int8_gemm(x.data, x.dtype == DType::F16 ? OMNI_F16 : OMNI_F32, rows,
                                      width, static_cast<const int32_t*>(w_packed.data),
                                      w_packed.dim(0), static_cast<const float*>(w_scale.data),
                                      columns, static_cast<const int32_t*>(w_zero.data),
                                      w_zero.dim(0), static_cast<float*>(out.data), ws, ws_bytes,
                                      stream);
    alloc.release(ws, stream);
    // Shape disagreement, or a device this library does not serve: the
    // reference's None (int8_matmul.rs:517-521, :494-503).
    if (st == OMNI_NOT_HANDLED || st == OMNI_NO_DEVICE) {
        alloc.release(out.data, stream);
        return std::nullopt;
    }
    if (st != OMNI_OK) {
        alloc.release(out.data, stream);
        check(st);
    }
    return out;
}

}  // namespace int8_matmul

// Weight-only int8 linear with fp16 per-channel scales (no reference
// counterpart; semantics of int8_matmul.rs:644-649 and quant.rs:186-200):
// out f16 [rows, n] = f16(scale[n] * sum_k x[m,k] * w[n,k] + bias[n]).
inline DeviceTensor w8a16_linear(const DeviceTensor& x, const DeviceTensor& w,
                                 const DeviceTensor& scale, const DeviceTensor* bias,
                                 Allocator& alloc, hipStream_t stream = nullptr) {
    if (x.shape.size() != 2 || w.shape.size() != 2 || x.dtype != DType::F16 || w.dtype != DType::I8 ||
        scale.dtype != DType::F16 || w.dim(1) != x.dim(1) || scale.numel() != w.dim(0) ||
        (bias && (bias->dtype != DType::F16 || bias->numel() != w.dim(0))))
        throw Int8Error(OMNI_BAD_ARGUMENT, "w8a16_linear: shapes/dtypes disagree");
    DeviceTensor out{alloc.allocate((size_t)(x.dim(0) * w.dim(0)) * 2, stream), {x.dim(0), w.dim(0)}, DType::F16};
    // Split-K partial sums when the shape asks for them (0 bytes: none).
    const size_t ws_bytes = omni_w8a16_gemm_workspace_size(x.dim(0), w.dim(0), x.dim(1));
    void* ws = ws_bytes ? alloc.allocate(ws_bytes, stream) : nullptr;
    const int st = omni_w8a16_gemm_ws(static_cast<const uint16_t*>(x.data), static_cast<const int8_t*>(w.data),
                                      static_cast<const uint16_t*>(scale.data),
                                      bias ? static_cast<const uint16_t*>(bias->data) : nullptr, x.dim(0),
                                      w.dim(0), x.dim(1), static_cast<uint16_t*>(out.data), ws, ws_bytes, stream);
    if (ws) alloc.release(ws, stream);
    if (st != OMNI_OK) {
        alloc.release(out.data, stream);
        if (st == OMNI_NOT_HANDLED) throw Int8Error(st, omni_int8_last_error());
        check(st);
    }
    return out;
}

}  // namespace omni_kernel

#endif  // OMNI_KERNEL_HPP
