// Weight-only int8 linear (W8A16) for gfx950:
//   out[m][n] = f16(scale[n] * sum_k x[m][k] * w[n][k] + bias[n])
// x f16 [rows][width], w int8 [columns][width], scale/bias f16 [columns].
//
// The reference has no such op. It follows the reference's dequantisation
// convention — w_deq = w * scale per output channel, f32 accumulation
// (crates/omni-kernel/src/int8_matmul.rs:644-649, crates/minicpm-v/src/quant.rs:186-200).
// The per-channel scale is constant along k, so it factors out of the k sum
// and is applied once per output in the epilogue.
//
// int8 -> f16 is exact: v_perm_b32 builds the f16 bit patterns 0x6400|(w+128)
// = 1024 + (w + 128) for two codes at once, and one packed f16 subtract of
// 1152 leaves w exactly (all values are integers below 2048).
//
//  * w8a16_gemv_kernel (rows <= 4, the decode shape) is HBM-bound: each
//    workgroup keeps its slice of x resident in registers ("x-stationary":
//    256 lanes own fixed 16-element k chunks) and streams R weight rows at a
//    time with 128-bit loads, v_dot2_f32_f16 into f32 partial sums, then one
//    wave reduction plus an LDS step across the 4 waves.
//  * w8a16_mfma_kernel (prefill) converts each weight tile to f16 once while
//    staging it into LDS, then runs v_mfma_f32_32x32x16_f16 on LDS fragments
//    with the same swizzled, double-buffered layout as the W8A8 kernel.
#include <cstdlib>

#include "common.hpp"
#include "kernels.hpp"

namespace omni {

namespace {

__device__ __forceinline__ u32 half2_bits(v2h h) {
    u32 u;
    __builtin_memcpy(&u, &h, 4);
    return u;
}
__device__ __forceinline__ v2h bits_half2(u32 u) {
    v2h h;
    __builtin_memcpy(&h, &u, 4);
    return h;
}

// Four int8 codes in `word` -> two f16 pairs (codes 0,1) and (codes 2,3), exact.
__device__ __forceinline__ void i8x4_to_f16x4(u32 word, v2h& lo, v2h& hi) {
    const u32 biased = word ^ 0x80808080u;  // w + 128 as unsigned bytes
    const u32 p0 = __builtin_amdgcn_perm(0x64646464u, biased, 0x04010400u);
    const u32 p1 = __builtin_amdgcn_perm(0x64646464u, biased, 0x04030402u);
    const v2h k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
    lo = bits_half2(p0) - k1152;
    hi = bits_half2(p1) - k1152;
}

// ---------------------------------------------------------------------------
// Decode GEMV.
// ---------------------------------------------------------------------------

// Butterfly fold of N partial sums per lane across the 64 lanes of a wave:
// at each offset O the lanes exchange half of their values, so N values cost
// about N shuffles instead of 6N. Afterwards every lane holds one complete
// sum, of index fold_index<N>(lane).
template <int N, int O>
struct Fold {
    static __device__ __forceinline__ void run(float* v, int lane) {
        if constexpr (O == 0) {
            return;
        } else if constexpr (N > 1) {
            constexpr int H = N / 2;
            const bool upper = (lane & O) != 0;
#pragma unroll
            for (int i = 0; i < H; ++i) {
                const float send = upper ? v[i] : v[i + H];
                const float keep = upper ? v[i + H] : v[i];
                v[i] = keep + __shfl_xor(send, O, kWave);
            }
            Fold<H, O / 2>::run(v, lane);
        } else {
            v[0] += __shfl_xor(v[0], O, kWave);
            Fold<1, O / 2>::run(v, lane);
        }
    }
};

template <int N>
__device__ __forceinline__ int fold_index(int lane) {
    int idx = 0;
#pragma unroll
    for (int l = 0, h = N / 2; h >= 1; ++l, h /= 2) idx += ((lane >> (5 - l)) & 1) * h;
    return idx;
}

// MR activation rows (1, 2 or 4; unused rows are zero), CPL 16-element k
// chunks per lane (the workgroup's 256 lanes own chunks tid + 256*j), R weight
// rows per group. Weights of the next group are loaded while the current
// group is reduced (PIPE).
template <int MR, int CPL, int R, bool PIPE>
__global__ __launch_bounds__(256) void w8a16_gemv_kernel(W8A16Args a) {
    constexpr int V = R * MR;
    static_assert((V & (V - 1)) == 0 && V <= 64, "power-of-two partial count");
    __shared__ float s_part[4][V];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t K = a.width;
    const int64_t chunks = K / 16;
    const int64_t groups = (a.columns + R - 1) / R;

    // Resident x: for each owned chunk j and row m, 16 halves as 8 f16 pairs.
    v2h xr[CPL][MR][8];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + 256 * j;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if (c < chunks && m < a.rows) {
                const uint4* p = reinterpret_cast<const uint4*>(a.x + m * K + c * 16);
                const uint4 q0 = p[0], q1 = p[1];
                xr[j][m][0] = bits_half2(q0.x); xr[j][m][1] = bits_half2(q0.y);
                xr[j][m][2] = bits_half2(q0.z); xr[j][m][3] = bits_half2(q0.w);
                xr[j][m][4] = bits_half2(q1.x); xr[j][m][5] = bits_half2(q1.y);
                xr[j][m][6] = bits_half2(q1.z); xr[j][m][7] = bits_half2(q1.w);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) xr[j][m][e] = v2h{};
            }
        }
    }

    auto load = [&](uint4 (&wv)[R][CPL], int64_t g) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t n0 = g * R + r;
            const int64_t n = n0 < a.columns ? n0 : a.columns - 1;
            const int8_t* wrow = a.w + n * K;
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                // Clamped, not predicated: a predicated load lets the compiler
                // pull its consumers next to it, which waits for it at once.
                // Chunks past K meet zero activations, so their value is moot.
                const int64_t c = tid + 256 * j < chunks ? tid + 256 * j : chunks - 1;
                wv[r][j] = *reinterpret_cast<const uint4*>(wrow + c * 16);
            }
        }
    };

    // Row groups blockIdx.x, blockIdx.x + gridDim.x, ... (measured faster on
    // MI355X than giving each workgroup a contiguous range).
    const int64_t g_begin = blockIdx.x, g_end = groups, g_step = gridDim.x;
    // One row group: wait for its weights (cur), issue the next group's
    // (nxt, unconditional: the last group re-reads itself from L2, so every
    // path issues the same loads and the wait for cur leaves nxt in flight),
    // then dot, reduce and store. The loop below alternates two register sets.
    auto group = [&](uint4 (&cur)[R][CPL], uint4 (&nxt)[R][CPL], int64_t g) {
        // This group's scale and bias, loaded by every thread (row tid % R)
        // ahead of the next group's weights.
        const int64_t n_ep = min(g * R + (tid / MR) % R, a.columns - 1);
        const _Float16 sc_h = a.scale[n_ep];
        const _Float16 bi_h = (a.bias ? a.bias : a.scale)[n_ep];  // unconditional load
        if constexpr (PIPE) load(nxt, g + g_step < g_end ? g + g_step : g);
        float part[V];
#pragma unroll
        for (int i = 0; i < V; ++i) part[i] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
#pragma unroll
            for (int j = 0; j < CPL; ++j) {
                const u32 words[4] = {cur[r][j].x, cur[r][j].y, cur[r][j].z, cur[r][j].w};
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    v2h w01, w23;
                    i8x4_to_f16x4(words[q], w01, w23);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        float& p = part[r * MR + m];
                        p = __builtin_amdgcn_fdot2(w01, xr[j][m][2 * q], p, false);
                        p = __builtin_amdgcn_fdot2(w23, xr[j][m][2 * q + 1], p, false);
                    }
                }
            }
        }
        Fold<V, 32>::run(part, lane);
        if ((lane & (64 / V - 1)) == 0) s_part[wave][fold_index<V>(lane)] = part[0];
        __syncthreads();
        if (tid < V) {
            const int r = tid / MR, m = tid % MR;
            const int64_t n = g * R + r;
            if (n < a.columns && m < a.rows) {
                const float acc = s_part[0][tid] + s_part[1][tid] + s_part[2][tid] + s_part[3][tid];
                const float bi = a.bias ? (float)bi_h : 0.0f;
                a.out[(int64_t)m * a.columns + n] = (_Float16)(acc * (float)sc_h + bi);
            }
        }
        __syncthreads();
        if constexpr (!PIPE) {
            if (g + g_step < g_end) load(cur, g + g_step);
        }
    };

    uint4 wa[R][CPL], wb[R][CPL];
    load(wa, g_begin);
    for (int64_t g = g_begin; g < g_end; g += 2 * g_step) {
        if constexpr (PIPE) {
            group(wa, wb, g);
            if (g + g_step < g_end) group(wb, wa, g + g_step);
        } else {
            group(wa, wa, g);
            if (g + g_step < g_end) group(wa, wa, g + g_step);
        }
    }
}

// OMNI_W8A16_GRID=<n> pins the GEMV grid size (tuning aid; 0 = heuristic).
int gemv_grid_override() {
    static const int value = [] {
        const char* v = std::getenv("OMNI_W8A16_GRID");
        return v ? std::atoi(v) : 0;
    }();
    return value;
}

template <int MR, int CPL, int R, bool PIPE>
hipError_t launch_gemv_cfg(const W8A16Args& a, hipStream_t stream) {
    const int64_t groups = (a.columns + R - 1) / R;
    // Up to 1024 workgroups (4 per CU), but at least two row groups per
    // workgroup where there are enough, so that the next group's weights
    // stream in while the current one is reduced (256-1024, measured).
    int64_t grid = (groups + 1) / 2;
    grid = grid < 256 ? 256 : (grid > 1024 ? 1024 : grid);
    if (gemv_grid_override() > 0) grid = gemv_grid_override();
    if (grid > groups) grid = groups;
    hipLaunchKernelGGL((w8a16_gemv_kernel<MR, CPL, R, PIPE>), dim3((unsigned)grid), dim3(256), 0,
                       stream, a);
    return hipGetLastError();
}

template <int MR>
hipError_t launch_gemv_m(const W8A16Args& a, hipStream_t stream) {
    const int64_t cpl = (a.width / 16 + 255) / 256;
    switch (cpl) {
        case 1: return launch_gemv_cfg<MR, 1, 8, true>(a, stream);
        case 2: return launch_gemv_cfg<MR, 2, 4, true>(a, stream);
        case 3: return launch_gemv_cfg<MR, 3, 4, MR < 4>(a, stream);
        default: return launch_gemv_cfg<MR, 4, 4, MR < 4>(a, stream);
    }
}

// ---------------------------------------------------------------------------
// Prefill GEMM on fp16 MFMA.
// ---------------------------------------------------------------------------
__device__ __forceinline__ int xcd_remap16(int b, int total) {
    constexpr int kXcds = 8;
    const int per = total / kXcds, rem = total % kXcds;
    const int xcd = b % kXcds, local = b / kXcds;
    return xcd * per + (xcd < rem ? xcd : rem) + local;
}

// Tile rows hold BK f16 = 2*BK bytes; 16-byte chunks swizzled by row.
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GROUP_M>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void w8a16_mfma_kernel(W8A16Args a) {
    constexpr int kThreads = 64 * WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int kRowBytes = BK * 2;
    constexpr int kChunks = kRowBytes / 16;  // 16-byte chunks (8 halves) per row
    static_assert(kChunks == 8, "BK = 64 halves");
    constexpr int kALoads = BM * kChunks / kThreads;        // x: 8 halves per load
    constexpr int kBLoads = BN * (BK / 16) / kThreads;      // w: 16 codes per load
    static_assert(kALoads * kThreads == BM * kChunks, "even A loads");
    static_assert(kBLoads * kThreads == BN * (BK / 16), "even B loads");

    extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
    uint8_t* sA = smem;
    uint8_t* sB = smem + 2 * BM * kRowBytes;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int tiles_m = (int)((a.rows + BM - 1) / BM);
    const int tiles_n = (int)((a.columns + BN - 1) / BN);
    const int t = xcd_remap16(blockIdx.x, tiles_m * tiles_n);
    const int group_size = GROUP_M * tiles_n;
    const int first_m = (t / group_size) * GROUP_M;
    const int gm = min(tiles_m - first_m, GROUP_M);
    const int tm = first_m + (t % group_size) % gm;
    const int tn = (t % group_size) / gm;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
    const int64_t K = a.width;
    const int ktiles = (int)((K + BK - 1) / BK);
    // 128-byte rows: two rows per 256-byte LDS window (see the W8A8 kernel).
    auto swz = [](int r, int c) { return c ^ ((r >> 1) & 7); };

    uint4 ra[kALoads];
    uint4 rb[kBLoads];
    auto load_tile = [&](int kt) {
        const int64_t k0 = (int64_t)kt * BK;
#pragma unroll
        for (int i = 0; i < kALoads; ++i) {
            const int id = tid + i * kThreads;
            const int r = id / kChunks, c = id % kChunks;
            const int64_t gr = m0 + r, gk = k0 + c * 8;
            ra[i] = (gr < a.rows && gk < K) ? *reinterpret_cast<const uint4*>(a.x + gr * K + gk)
                                            : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < kBLoads; ++i) {
            const int id = tid + i * kThreads;
            const int r = id / (BK / 16), c = id % (BK / 16);
            const int64_t gr = n0 + r, gk = k0 + c * 16;
            rb[i] = (gr < a.columns && gk < K) ? *reinterpret_cast<const uint4*>(a.w + gr * K + gk)
                                               : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_tile = [&](int buf) {
        uint8_t* dA = sA + buf * BM * kRowBytes;
        uint8_t* dB = sB + buf * BN * kRowBytes;
#pragma unroll
        for (int i = 0; i < kALoads; ++i) {
            const int id = tid + i * kThreads;
            const int r = id / kChunks, c = id % kChunks;
            *reinterpret_cast<uint4*>(dA + r * kRowBytes + swz(r, c) * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < kBLoads; ++i) {
            const int id = tid + i * kThreads;
            const int r = id / (BK / 16), c = id % (BK / 16);
            // 16 codes -> 16 halves = two 16-byte chunks 2c and 2c+1.
            const u32 words[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
            v2h h[8];
#pragma unroll
            for (int q = 0; q < 4; ++q) i8x4_to_f16x4(words[q], h[2 * q], h[2 * q + 1]);
            uint4 lo = make_uint4(half2_bits(h[0]), half2_bits(h[1]), half2_bits(h[2]), half2_bits(h[3]));
            uint4 hi = make_uint4(half2_bits(h[4]), half2_bits(h[5]), half2_bits(h[6]), half2_bits(h[7]));
            *reinterpret_cast<uint4*>(dB + r * kRowBytes + swz(r, 2 * c) * 16) = lo;
            *reinterpret_cast<uint4*>(dB + r * kRowBytes + swz(r, 2 * c + 1) * 16) = hi;
        }
    };

    v16f acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

    load_tile(0);
    store_tile(0);
    __syncthreads();
    const int frag_row = lane & 31, frag_kc = lane >> 5;
    for (int kt = 0; kt < ktiles; ++kt) {
        const int buf = kt & 1;
        if (kt + 1 < ktiles) load_tile(kt + 1);
        const uint8_t* tA = sA + buf * BM * kRowBytes;
        const uint8_t* tB = sB + buf * BN * kRowBytes;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int c = ks * 2 + frag_kc;
            v8h fa[FM], fb[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int r = wm * WM + i * 32 + frag_row;
                fa[i] = *reinterpret_cast<const v8h*>(tA + r * kRowBytes + swz(r, c) * 16);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int r = wn * WN + j * 32 + frag_row;
                fb[j] = *reinterpret_cast<const v8h*>(tB + r * kRowBytes + swz(r, c) * 16);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_f16(fa[i], fb[j], acc[i][j], 0, 0, 0);
        }
        if (kt + 1 < ktiles) store_tile(buf ^ 1);
        __syncthreads();
    }

#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int64_t col = n0 + wn * WN + j * 32 + (lane & 31);
        if (col >= a.columns) continue;
        const float sc = (float)a.scale[col];
        const float bias = a.bias ? (float)a.bias[col] : 0.0f;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t row = m0 + wm * WM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row >= a.rows) continue;
                a.out[row * a.columns + col] = (_Float16)(acc[i][j][r] * sc + bias);
            }
    }
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GROUP_M>
hipError_t launch_mfma16_cfg(const W8A16Args& a, hipStream_t stream) {
    auto kernel = w8a16_mfma_kernel<BM, BN, BK, WAVES_M, WAVES_N, GROUP_M>;
    const size_t smem = 2 * (size_t)(BM + BN) * BK * 2;
    if (smem > 65536) {
        hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                           hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
        if (e != hipSuccess) return e;
    }
    const int64_t tiles = ((a.rows + BM - 1) / BM) * ((a.columns + BN - 1) / BN);
    hipLaunchKernelGGL(kernel, dim3((unsigned)tiles), dim3(64 * WAVES_M * WAVES_N), smem, stream, a);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_w8a16_gemv(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    switch (a.rows) {
        case 1: return launch_gemv_m<1>(a, stream);
        case 2: return launch_gemv_m<2>(a, stream);
        default: return launch_gemv_m<4>(a, stream);  // 3 rows run with one zero row
    }
}

hipError_t launch_w8a16_mfma(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    const int64_t big_tiles = ((a.rows + 127) / 128) * ((a.columns + 127) / 128);
    if (big_tiles >= 512) return launch_mfma16_cfg<128, 128, 64, 2, 2, 4>(a, stream);
    return launch_mfma16_cfg<64, 64, 64, 2, 2, 4>(a, stream);
}

}  // namespace omni
