// W8A8 int8 x int8 -> int32 GEMM with the reference's fused f32 epilogue, gfx950.
//
// Semantics (crates/omni-kernel/src/int8_matmul.rs:145-373):
//   acc[m][n] = sum_k x[m][k] * w[n][k]                       exact int32
//   out[m][n] = f32(acc - x_sum[m] * w_zero[n]) * x_scale[m] * w_scale[n]
// left to right in f32 (store, :145-159), optionally + bias[n], stored as f32
// (the reference's output) or rounded once to f16.
//
// Two lowerings, as the reference has two (int8_dot and int8_dot_tile64):
//  * w8a8_mfma_kernel — the int8 MFMA path. Both operands are K-contiguous
//    ("NT"), which is the layout v_mfma_i32_32x32x32_i8 wants for A and B
//    alike: each lane feeds 16 consecutive k bytes of one row of A and one
//    row of W. K tiles are staged through LDS (double-buffered, one barrier
//    per K tile) with an XOR swizzle of the 16-byte chunk index so both the
//    row-wise global->LDS writes and the column-of-rows fragment reads are
//    bank-conflict free. The epilogue runs on the accumulators in registers,
//    so no int32 accumulator array ever reaches HBM (the reference's tile64
//    lowering round-trips one, int8_matmul.rs:423-439).
//  * w8a8_scalar_kernel — v_dot4_i32_i8 per thread, the analog of the
//    reference's scalar int8_dot; it serves widths that are not a multiple of
//    16 and the OMNI_INT8_FORCE_SCALAR override.
#include <atomic>
#include <cstdlib>

#include "common.hpp"
#include "kernels.hpp"

namespace omni {

namespace {

// crates/omni-kernel/src/int8_matmul.rs:156-158. Contraction is off so that
// (centered * row_scale) * w_scale and the bias add round as separate f32 ops.
__device__ __forceinline__ float w8a8_epilogue(int acc, int sum, int zero, float row_scale,
                                               float w_scale, float bias, bool has_bias) {
#pragma clang fp contract(off)
    int centered = acc - sum * zero;
    float t = (float)centered * row_scale;
    float v = t * w_scale;
    if (has_bias) v = v + bias;
    return v;
}

__device__ __forceinline__ void store_out(void* out, int64_t idx, float v, bool out_f16) {
    if (out_f16)
        static_cast<_Float16*>(out)[idx] = (_Float16)v;  // v_cvt_f16_f32: round to nearest even
    else
        static_cast<float*>(out)[idx] = v;
}

// ---------------------------------------------------------------------------
// Scalar lowering: one thread = one row x 4 consecutive columns, v_dot4 over K.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void w8a8_scalar_kernel(W8A8Args a) {
    const int64_t col0 = ((int64_t)blockIdx.x * 64 + threadIdx.x) * 4;
    const int64_t row = (int64_t)blockIdx.y * 4 + threadIdx.y;
    if (row >= a.rows || col0 >= a.columns) return;
    const int64_t words = a.width / 4;
    const u32* xr = reinterpret_cast<const u32*>(a.x + row * a.width);
    int acc[4] = {0, 0, 0, 0};
    const u32* wr[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t c = col0 + j < a.columns ? col0 + j : a.columns - 1;
        wr[j] = reinterpret_cast<const u32*>(a.w + c * a.width);
    }
    for (int64_t k = 0; k < words; ++k) {
        const int xw = (int)xr[k];
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_sdot4(xw, (int)wr[j][k], acc[j], false);
    }
    const float rs = a.x_scale[row];
    const int sum = a.x_sum ? a.x_sum[row] : 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t c = col0 + j;
        if (c >= a.columns) break;
        const int64_t idx = row * a.columns + c;
        if (a.acc_dump) a.acc_dump[idx] = acc[j];
        const int zero = a.w_zero ? a.w_zero[c] : 0;
        const float b = a.bias ? a.bias[c] : 0.0f;
        store_out(a.out, idx, w8a8_epilogue(acc[j], sum, zero, rs, a.w_scale[c], b, a.bias != nullptr),
                  a.out_f16);
    }
}

// ---------------------------------------------------------------------------
// MFMA lowering.
// ---------------------------------------------------------------------------

// Hardware workgroup id -> logical tile id, so that the workgroups one XCD
// runs (hardware ids congruent mod 8) get a contiguous range of logical tiles.
__device__ __forceinline__ int xcd_remap(int b, int total) {
    constexpr int kXcds = 8;
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = b % kXcds, local = b / kXcds;
    return xcd * per + (xcd < rem ? xcd : rem) + local;
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GROUP_M>
struct MfmaCfg {
    static constexpr int kThreads = 64 * WAVES_M * WAVES_N;
    static constexpr int WM = BM / WAVES_M;
    static constexpr int WN = BN / WAVES_N;
    static constexpr int FM = WM / 32;
    static constexpr int FN = WN / 32;
    static constexpr int kChunks = BK / 16;                 // 16-byte chunks per tile row
    static constexpr int kALoads = (BM * kChunks + kThreads - 1) / kThreads;
    static constexpr int kBLoads = (BN * kChunks + kThreads - 1) / kThreads;
    static constexpr int kStageBytes = (BM + BN) * BK;
    static_assert(WM % 32 == 0 && WN % 32 == 0, "wave tile is a multiple of 32x32");
    static_assert(BK % 32 == 0 && kChunks <= 8, "K tile of 32..128 bytes");
    static_assert((BM * kChunks) % kThreads == 0 && (BN * kChunks) % kThreads == 0,
                  "loads divide evenly among threads");
};

// Physical 16-byte chunk slot of logical chunk c in tile row r.
template <int kChunks>
__device__ __forceinline__ int swz(int r, int c) {
    return c ^ (r & (kChunks - 1));
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GROUP_M>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void w8a8_mfma_kernel(W8A8Args a) {
    using C = MfmaCfg<BM, BN, BK, WAVES_M, WAVES_N, GROUP_M>;
    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* sA = smem;                    // [2][BM][BK]
    uint8_t* sB = smem + 2 * BM * BK;      // [2][BN][BK]

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N;
    const int wn = wave % WAVES_N;

    // Tile coordinates: XCD-contiguous logical ids, then GROUP_M tile rows
    // walked column by column so that concurrent tiles share A rows and W rows.
    const int tiles_m = (int)((a.rows + BM - 1) / BM);
    const int tiles_n = (int)((a.columns + BN - 1) / BN);
    const int t = xcd_remap(blockIdx.x, tiles_m * tiles_n);
    const int group_size = GROUP_M * tiles_n;
    const int first_m = (t / group_size) * GROUP_M;
    const int gm = min(tiles_m - first_m, GROUP_M);
    const int tm = first_m + (t % group_size) % gm;
    const int tn = (t % group_size) / gm;
    const int64_t m0 = (int64_t)tm * BM;
    const int64_t n0 = (int64_t)tn * BN;

    const int64_t K = a.width;
    const int ktiles = (int)((K + BK - 1) / BK);

    // Global -> register staging for one K tile.
    uint4 ra[C::kALoads];
    uint4 rb[C::kBLoads];
    auto load_tile = [&](int kt) {
        const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
        for (int i = 0; i < C::kALoads; ++i) {
            const int id = tid + i * C::kThreads;
            const int r = id / C::kChunks, c = id % C::kChunks;
            const int64_t gr = m0 + r, gk = k0 + c * 16;
            ra[i] = (gr < a.rows && gk < K)
                        ? *reinterpret_cast<const uint4*>(a.x + gr * K + gk)
                        : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < C::kBLoads; ++i) {
            const int id = tid + i * C::kThreads;
            const int r = id / C::kChunks, c = id % C::kChunks;
            const int64_t gr = n0 + r, gk = k0 + c * 16;
            rb[i] = (gr < a.columns && gk < K)
                        ? *reinterpret_cast<const uint4*>(a.w + gr * K + gk)
                        : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_tile = [&](int buf) {
        uint8_t* dA = sA + buf * BM * BK;
        uint8_t* dB = sB + buf * BN * BK;
#pragma unroll
        for (int i = 0; i < C::kALoads; ++i) {
            const int id = tid + i * C::kThreads;
            const int r = id / C::kChunks, c = id % C::kChunks;
            *reinterpret_cast<uint4*>(dA + r * BK + swz<C::kChunks>(r, c) * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < C::kBLoads; ++i) {
            const int id = tid + i * C::kThreads;
            const int r = id / C::kChunks, c = id % C::kChunks;
            *reinterpret_cast<uint4*>(dB + r * BK + swz<C::kChunks>(r, c) * 16) = rb[i];
        }
    };

    v16i acc[C::FM][C::FN];
#pragma unroll
    for (int i = 0; i < C::FM; ++i)
#pragma unroll
        for (int j = 0; j < C::FN; ++j) acc[i][j] = v16i{};

    load_tile(0);
    store_tile(0);
    __syncthreads();

    const int frag_row = lane & 31;  // row of A (or of W) this lane feeds
    const int frag_kc = lane >> 5;   // which 16-byte half of a 32-byte k step
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) load_tile(kt + 1);
        const uint8_t* tA = sA + buf * BM * BK;
        const uint8_t* tB = sB + buf * BN * BK;
#pragma unroll
        for (int ks = 0; ks < BK / 32; ++ks) {
            const int c = ks * 2 + frag_kc;
            v4i fa[C::FM], fb[C::FN];
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const int r = wm * C::WM + i * 32 + frag_row;
                fa[i] = *reinterpret_cast<const v4i*>(tA + r * BK + swz<C::kChunks>(r, c) * 16);
            }
#pragma unroll
            for (int j = 0; j < C::FN; ++j) {
                const int r = wn * C::WN + j * 32 + frag_row;
                fb[j] = *reinterpret_cast<const v4i*>(tB + r * BK + swz<C::kChunks>(r, c) * 16);
            }
#pragma unroll
            for (int i = 0; i < C::FM; ++i)
#pragma unroll
                for (int j = 0; j < C::FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < ktiles) store_tile(buf ^ 1);
        __syncthreads();
    }

    // Epilogue straight from the accumulators. 32x32 accumulator layout:
    // lane holds column (lane & 31) and rows 8*(r/4) + 4*(lane/32) + (r%4).
    const bool has_bias = a.bias != nullptr;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
        const int64_t col = n0 + wn * C::WN + j * 32 + (lane & 31);
        if (col >= a.columns) continue;
        const float ws = a.w_scale[col];
        const int zero = a.w_zero ? a.w_zero[col] : 0;
        const float bias = has_bias ? a.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < C::FM; ++i) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * C::WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= a.rows) continue;
                const int64_t idx = row * a.columns + col;
                const int v = acc[i][j][r];
                if (a.acc_dump) a.acc_dump[idx] = v;
                const int sum = a.w_zero ? a.x_sum[row] : 0;
                store_out(a.out, idx, w8a8_epilogue(v, sum, zero, a.x_scale[row], ws, bias, has_bias),
                          a.out_f16);
            }
        }
    }
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GROUP_M>
hipError_t launch_cfg(const W8A8Args& a, hipStream_t stream) {
    using C = MfmaCfg<BM, BN, BK, WAVES_M, WAVES_N, GROUP_M>;
    auto kernel = w8a8_mfma_kernel<BM, BN, BK, WAVES_M, WAVES_N, GROUP_M>;
    const size_t smem = 2 * (size_t)C::kStageBytes;
    // Dynamic LDS above 64 KiB needs an opt-in; setting it is idempotent.
    static std::atomic<bool> configured{false};
    if (!configured.load(std::memory_order_acquire)) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
        configured.store(true, std::memory_order_release);
    }
    const int64_t tiles = ((a.rows + BM - 1) / BM) * ((a.columns + BN - 1) / BN);
    hipLaunchKernelGGL(kernel, dim3((unsigned)tiles), dim3(C::kThreads), smem, stream, a);
    return hipGetLastError();
}

// OMNI_W8A8_TILE=<n> pins one tile configuration (tuning aid; 0 = heuristic).
int w8a8_tile_override() {
    static const int value = [] {
        const char* v = std::getenv("OMNI_W8A8_TILE");
        return v ? std::atoi(v) : 0;
    }();
    return value;
}

}  // namespace

hipError_t launch_w8a8_scalar(const W8A8Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    dim3 block(64, 4);
    dim3 grid((unsigned)((a.columns + 255) / 256), (unsigned)((a.rows + 3) / 4));
    hipLaunchKernelGGL(w8a8_scalar_kernel, grid, block, 0, stream, a);
    return hipGetLastError();
}

hipError_t launch_w8a8_mfma(const W8A8Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    switch (w8a8_tile_override()) {
        case 1: return launch_cfg<256, 256, 64, 2, 2, 4>(a, stream);
        case 2: return launch_cfg<256, 256, 128, 2, 4, 4>(a, stream);
        case 3: return launch_cfg<256, 256, 64, 2, 4, 4>(a, stream);
        case 4: return launch_cfg<256, 128, 128, 2, 2, 4>(a, stream);
        case 5: return launch_cfg<128, 128, 128, 2, 2, 4>(a, stream);
        case 6: return launch_cfg<256, 128, 64, 2, 2, 4>(a, stream);
        default: break;
    }
    return launch_cfg<256, 256, 64, 2, 4, 4>(a, stream);
}

}  // namespace omni
