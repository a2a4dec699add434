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
#include <type_traits>

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

// The same four codes as the f16 values 1152 + w (exact): three VALU per
// four codes. A dot product against them exceeds the true one by 1152 * (the
// sum of the activations), which the caller subtracts once per row.
__device__ __forceinline__ void i8x4_to_f16x4_biased(u32 word, v2h& lo, v2h& hi) {
    const u32 biased = word ^ 0x80808080u;
    lo = bits_half2(__builtin_amdgcn_perm(0x64646464u, biased, 0x04010400u));
    hi = bits_half2(__builtin_amdgcn_perm(0x64646464u, biased, 0x04030402u));
}

// Eight int4 codes of `word` (low nibble first, each stored plus 8, as
// crates/minicpm-v/src/quant.rs:22-29 unpacks them) -> four f16 pairs in k
// order (n0,n1) (n2,n3) (n4,n5) (n6,n7), exact: bytes [n, 0x64] are the f16
// 1024 + n, and one packed subtract of 1032 leaves n - 8.
// Byte t of word >> 4 holds code 2t + 1 in its low nibble: two v_perm_b32
// and two masks give the codes in k order one per byte, and one v_perm_b32
// per pair spreads two of them under 0x64 bytes (nine integer ops per word).
__device__ __forceinline__ void i4x8_to_f16x8(u32 word, v2h (&h)[4]) {
    const u32 sh = word >> 4;
    const u32 c0 = __builtin_amdgcn_perm(sh, word, 0x05010400u) & 0x0F0F0F0Fu;  // n0 n1 n2 n3
    const u32 c1 = __builtin_amdgcn_perm(sh, word, 0x07030602u) & 0x0F0F0F0Fu;  // n4 n5 n6 n7
    const u32 k64 = 0x64646464u;
    const v2h k1032 = {(_Float16)1032.0f, (_Float16)1032.0f};
    h[0] = bits_half2(__builtin_amdgcn_perm(k64, c0, 0x04010400u)) - k1032;
    h[1] = bits_half2(__builtin_amdgcn_perm(k64, c0, 0x04030402u)) - k1032;
    h[2] = bits_half2(__builtin_amdgcn_perm(k64, c1, 0x04010400u)) - k1032;
    h[3] = bits_half2(__builtin_amdgcn_perm(k64, c1, 0x04030402u)) - k1032;
}

// Eight int4 codes of `word` as the f16 values 1024 + nibble (exact), one
// v_perm_b32 per pair placing a nibble byte under the high byte 0x64 taken
// from k64 = 0x64646464, in the pairs (n0, n2), (n1, n3), (n4, n6), (n5, n7).
// The codes are nibble - 8, so a dot product against these values exceeds
// the true one by 1032 * (the sum of the activations), which the caller
// subtracts once per row of partial sums instead of once per pair.
__device__ __forceinline__ void i4x8_to_f16x8_biased(u32 word, u32 k64, v2h (&h)[4]) {
    const u32 lo = word & 0x0F0F0F0Fu;         // n0 n2 n4 n6
    const u32 hi = (word >> 4) & 0x0F0F0F0Fu;  // n1 n3 n5 n7
    h[0] = bits_half2(__builtin_amdgcn_perm(k64, lo, 0x04010400u));
    h[1] = bits_half2(__builtin_amdgcn_perm(k64, hi, 0x04010400u));
    h[2] = bits_half2(__builtin_amdgcn_perm(k64, lo, 0x04030402u));
    h[3] = bits_half2(__builtin_amdgcn_perm(k64, hi, 0x04030402u));
}

// A bf16 scale (quant.rs:74-81) as f32 (exact) and as f16 (exact for scales
// in f16's normal range, 2^-14 .. 65504).
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((u32)b << 16); }

// 16 int4 codes (two words) times one scale -> 16 halves in k order:
// f16(q * s), the dequantised value the reference's F16 route rounds to
// (quant.rs:186-200): q * s is exact in f32 and the packed f16 multiply
// rounds it once, like the f32 -> f16 cast.
__device__ __forceinline__ void i4x16_dequant(u32 w0, u32 w1, _Float16 s, v2h (&h)[8]) {
    v2h a[4], b[4];
    i4x8_to_f16x8(w0, a);
    i4x8_to_f16x8(w1, b);
    const v2h s2 = {s, s};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        h[i] = a[i] * s2;
        h[4 + i] = b[i] * s2;
    }
}

// ---------------------------------------------------------------------------
// Decode GEMV.
// ---------------------------------------------------------------------------

// Butterfly fold of N partial sums per lane across the 64 lanes of a wave:
// at each offset O the lanes exchange half of their values, so N values cost
// about N exchanges instead of 6N. Afterwards every lane holds one complete
// sum, of index fold_index<N>(lane). Every move stays in registers: offsets
// 32 and 16 are one permlane swap per pair of values (swap_add), 8 .. 1 are
// DPP moves (lane_xor), so the fold adds no LDS round trips to the end of
// the kernel.
template <int N, int O>
struct Fold {
    static __device__ __forceinline__ void run(float* v, int lane) {
        if constexpr (O == 0) {
            return;
        } else if constexpr (N > 1) {
            constexpr int H = N / 2;
            if constexpr (O >= 16) {
#pragma unroll
                for (int i = 0; i < H; ++i) v[i] = swap_add<O>(v[i], v[i + H]);
            } else {
                const bool upper = (lane & O) != 0;
#pragma unroll
                for (int i = 0; i < H; ++i) {
                    const float send = upper ? v[i] : v[i + H];
                    const float keep = upper ? v[i + H] : v[i];
                    v[i] = keep + lane_xor<O>(send);
                }
            }
            Fold<H, O / 2>::run(v, lane);
        } else {
            if constexpr (O >= 16)
                v[0] = swap_add<O>(v[0], v[0]);
            else
                v[0] += lane_xor<O>(v[0]);
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

// MR activation rows (1, 2 or 4; unused rows are zero). A workgroup of T
// lanes (T = blockDim.x, a multiple of 64, at most 1024) owns R consecutive
// weight rows; lane t owns the 16-byte weight chunks t + T*j, j < CPL (16
// int8 codes, or 8 halves with WB = 16), so one row of W is T*CPL*16 bytes
// wide at most. Every weight load of the workgroup is issued before any
// arithmetic (after x's chunks, which hit in L2), as nontemporal loads (the
// weights are read once; keeping them out of the caches keeps x and the
// scales there), so the whole workgroup's share of W is in flight at once.
// One workgroup per row group, many of them resident per CU, keeps the HBM
// queues full: measured on MI355X this streams within a few percent of a
// bare read kernel of the same size, and a 525 MB weight (a 128256 x 4096
// vocabulary head) at 7.2 TB/s.
// B batches of R rows (R * B rows per workgroup): all R * B rows' loads are
// issued up front, the partial sums of one batch at a time are kept and
// folded, so each x chunk held in registers serves R * B weight rows (x is
// read from L2 once per workgroup: 2 * MR bytes per weight byte / (R * B)).
// WB = 16: f16 weights, no scale (the fp16 linear).
// KF > 0 builds the kernel for K == KF with the workgroup size the launcher
// derives from it: where the lanes' chunks cover the row exactly, no chunk
// index is clamped or checked.
template <int MR, int CPL, int R, int WB = 8, int B = 1, int KF = 0>
__global__ __launch_bounds__(1024) void w8a16_gemv_kernel(W8A16Args a) {
    constexpr int V = R * MR;
    constexpr int RB = R * B;
    static_assert((V & (V - 1)) == 0 && V <= 64, "power-of-two partial count");
    static_assert(WB == 8 || WB == 16, "int8 or f16 weights");
    constexpr int kE = WB == 8 ? 16 : 8;  // weights per 16-byte chunk
    constexpr int kP = kE / 2;            // f16 pairs of x per chunk
    constexpr int kChunks = KF / kE;
    constexpr int kT = ((kChunks + CPL - 1) / CPL + 63) / 64 * 64;  // the launcher's workgroup size for KF
    constexpr bool kExact = KF > 0 && kT * CPL == kChunks;          // every chunk index in range
    __shared__ float s_part[16][B * V];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int T = KF > 0 ? kT : (int)blockDim.x;
    const int64_t K = KF > 0 ? KF : a.width;
    const int64_t chunks = K / kE;
    const int64_t n0 = (int64_t)blockIdx.x * RB;

    // x chunks: kE halves of each owned chunk and row as kP f16 pairs.
    v2h xr[CPL][MR][kP];
#pragma unroll
    for (int j = 0; j < CPL; ++j) {
        const int64_t c = tid + (int64_t)T * j;
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            if ((kExact || c < chunks) && (MR == 1 || m < a.rows)) {  // rows >= 1
                const uint4* p = reinterpret_cast<const uint4*>(a.x + m * K + c * kE);
#pragma unroll
                for (int u = 0; u < kE / 8; ++u) {
                    const uint4 q = p[u];
                    xr[j][m][4 * u] = bits_half2(q.x);
                    xr[j][m][4 * u + 1] = bits_half2(q.y);
                    xr[j][m][4 * u + 2] = bits_half2(q.z);
                    xr[j][m][4 * u + 3] = bits_half2(q.w);
                }
            } else {
#pragma unroll
                for (int e = 0; e < kP; ++e) xr[j][m][e] = v2h{};
            }
        }
    }

    // With more weight rows than activation rows per lane, codes enter the
    // dot products as 1152 + w (three VALU per four codes, not five) and
    // each row's partial sum drops xc = 1152 * sum(x), accumulated in the
    // same order. Products are exact and the f32 sums stay below
    // 2^11 * sum|x|: ~1e-5 of the result relative, nothing on integer data.
    constexpr bool kBiased = WB == 8 && RB > MR;
    float xc[MR];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        xc[m] = 0.0f;
        if constexpr (kBiased) {
            const v2h k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
            for (int j = 0; j < CPL; ++j)
#pragma unroll
                for (int e = 0; e < kP; ++e) xc[m] = __builtin_amdgcn_fdot2(k1152, xr[j][m][e], xc[m], false);
        }
    }

    // Then every weight load. Rows past the matrix and chunks past K are
    // clamped, not predicated (a predicated load lets the compiler pull its
    // consumers next to it); clamped chunks meet zero activations.
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u wv[RB][CPL];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int64_t n = n0 + r < a.columns ? n0 + r : a.columns - 1;
        const uint8_t* wrow = reinterpret_cast<const uint8_t*>(a.w) + n * K * (WB / 8);
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const int64_t c = kExact || tid + (int64_t)T * j < chunks ? tid + (int64_t)T * j : chunks - 1;
            wv[r][j] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wrow + c * 16));
        }
    }
    // This thread's epilogue row (tid / MR) % RB: scale and bias.
    const int64_t n_ep = min(n0 + (tid / MR) % RB, a.columns - 1);
    _Float16 sc_h = (_Float16)1.0f, bi_h = (_Float16)0.0f;
    if constexpr (WB == 8) {
        sc_h = a.scale[n_ep];
        bi_h = (a.bias ? a.bias : a.scale)[n_ep];  // unconditional load
    } else {
        if (a.bias) bi_h = a.bias[n_ep];
    }

#pragma unroll
    for (int b = 0; b < B; ++b) {
    float part[V];
#pragma unroll
    for (int i = 0; i < V; ++i) part[i] = 0.0f;
#pragma unroll
    for (int r = 0; r < R; ++r) {
#pragma unroll
        for (int j = 0; j < CPL; ++j) {
            const v4u wq = wv[b * R + r][j];
            const u32 words[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if constexpr (WB == 8) {
                    v2h w01, w23;
                    if constexpr (kBiased)
                        i8x4_to_f16x4_biased(words[q], w01, w23);
                    else
                        i8x4_to_f16x4(words[q], w01, w23);
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        float& p = part[r * MR + m];
                        p = __builtin_amdgcn_fdot2(w01, xr[j][m][2 * q], p, false);
                        p = __builtin_amdgcn_fdot2(w23, xr[j][m][2 * q + 1], p, false);
                    }
                } else {
#pragma unroll
                    for (int m = 0; m < MR; ++m) {
                        float& p = part[r * MR + m];
                        p = __builtin_amdgcn_fdot2(bits_half2(words[q]), xr[j][m][q], p, false);
                    }
                }
            }
        }
    }
    if constexpr (kBiased) {
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int m = 0; m < MR; ++m) part[r * MR + m] -= xc[m];
    }
    Fold<V, 32>::run(part, lane);
    if ((lane & (64 / V - 1)) == 0) s_part[wave][b * V + fold_index<V>(lane)] = part[0];
    }
    __syncthreads();
    if (tid < B * V) {
        const int r = tid / MR, m = tid % MR;
        const int64_t n = n0 + r;
        if (n < a.columns && m < a.rows) {
            float acc = 0.0f;
            for (int w = 0; w < T / 64; ++w) acc += s_part[w][tid];
            const float bi = a.bias ? (float)bi_h : 0.0f;
            a.out[(int64_t)m * a.columns + n] = (_Float16)(acc * (float)sc_h + bi);
        }
    }
}

// Streamed decode GEMV for 2 to 4 activation rows, int8 weights, K == KF
// (one 16-element chunk per lane, KF / 16 lanes rounded up to whole waves).
// The weight rows come in batches of R; workgroup g takes batches g, g +
// grid, ..., holding its lanes' x chunks of every row in registers for all
// of them (x is read from L2 once per workgroup, not once per batch), with
// the next batch's weights (and its output rows' scale and bias) in flight
// while the current batch is summed: two register buffers, the loop
// unrolled by two. Per batch: the same code conversion (1152 + w),
// dot products, fold and cross-wave sum as w8a16_gemv_kernel, through a
// parity-double-buffered LDS block, so one barrier per batch.
template <int MR, int R, int KF>
__global__ __launch_bounds__((KF / 16 + 63) / 64 * 64) void w8a16_gemv_stream_kernel(W8A16Args a) {
    constexpr int kP = 8;                      // f16 pairs of x per chunk
    constexpr int kChunks = KF / 16;
    constexpr int kT = (kChunks + 63) / 64 * 64;
    constexpr bool kExact = kT == kChunks;
    constexpr int V = R * MR;
    static_assert((V & (V - 1)) == 0 && V <= 64, "power-of-two partial count");
    constexpr bool kBiased = R > MR;  // as in w8a16_gemv_kernel: more weight rows than x rows
    static_assert(kT <= 1024, "one chunk per lane");
    __shared__ float s_part[2][kT / 64][V];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t K = KF;
    const int64_t nb = (a.columns + R - 1) / R;
    int64_t b = blockIdx.x;
    if (b >= nb) return;  // the whole workgroup
    const int64_t c = kExact || tid < kChunks ? tid : kChunks - 1;  // clamped chunks meet zero x
    const bool live = kExact || tid < kChunks;

    v2h xr[MR][kP];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        if (live && m < a.rows) {
            const uint4* px = reinterpret_cast<const uint4*>(a.x + m * K + c * 16);
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const uint4 q = px[u];
                xr[m][4 * u] = bits_half2(q.x);
                xr[m][4 * u + 1] = bits_half2(q.y);
                xr[m][4 * u + 2] = bits_half2(q.z);
                xr[m][4 * u + 3] = bits_half2(q.w);
            }
        } else {
#pragma unroll
            for (int e = 0; e < kP; ++e) xr[m][e] = v2h{};
        }
    }
    float xc[MR];
    {
        const v2h k1152 = {(_Float16)1152.0f, (_Float16)1152.0f};
#pragma unroll
        for (int m = 0; m < MR; ++m) {
            xc[m] = 0.0f;
            if constexpr (kBiased) {
#pragma unroll
                for (int e = 0; e < kP; ++e) xc[m] = __builtin_amdgcn_fdot2(k1152, xr[m][e], xc[m], false);
            }
        }
    }

    typedef unsigned v4u_t __attribute__((ext_vector_type(4)));
    // Weights of batch bb, and (threads < V) scale and bias of the output
    // row the thread writes.
    auto load_batch = [&](int64_t bb, v4u_t (&w)[R], _Float16& sc, _Float16& bi) {
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t n = bb * R + r < a.columns ? bb * R + r : a.columns - 1;
            w[r] = __builtin_nontemporal_load(reinterpret_cast<const v4u_t*>(
                reinterpret_cast<const uint8_t*>(a.w) + n * K + c * 16));
        }
        const int64_t ne = min(bb * R + (tid / MR) % R, a.columns - 1);
        sc = a.scale[ne];
        bi = (a.bias ? a.bias : a.scale)[ne];  // unconditional load
    };
    auto sum_batch = [&](int64_t bb, const v4u_t (&w)[R], _Float16 sc, _Float16 bi, int par) {
        float part[V];
#pragma unroll
        for (int i = 0; i < V; ++i) part[i] = 0.0f;
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const u32 words[4] = {w[r].x, w[r].y, w[r].z, w[r].w};
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                v2h w01, w23;
                if constexpr (kBiased)
                    i8x4_to_f16x4_biased(words[q], w01, w23);
                else
                    i8x4_to_f16x4(words[q], w01, w23);
#pragma unroll
                for (int m = 0; m < MR; ++m) {
                    float& pp = part[r * MR + m];
                    pp = __builtin_amdgcn_fdot2(w01, xr[m][2 * q], pp, false);
                    pp = __builtin_amdgcn_fdot2(w23, xr[m][2 * q + 1], pp, false);
                }
            }
        }
        if constexpr (kBiased) {
#pragma unroll
            for (int r = 0; r < R; ++r)
#pragma unroll
                for (int m = 0; m < MR; ++m) part[r * MR + m] -= xc[m];
        }
        Fold<V, 32>::run(part, lane);
        if ((lane & (64 / V - 1)) == 0) s_part[par][wave][fold_index<V>(lane)] = part[0];
        __syncthreads();
        if (tid < V) {
            const int r = tid / MR, m = tid % MR;
            const int64_t n = bb * R + r;
            if (n < a.columns && m < a.rows) {
                float acc = 0.0f;
                for (int wv = 0; wv < kT / 64; ++wv) acc += s_part[par][wv][tid];
                const float bias = a.bias ? (float)bi : 0.0f;
                a.out[(int64_t)m * a.columns + n] = (_Float16)(acc * (float)sc + bias);
            }
        }
    };

    v4u_t wA[R], wB[R];
    _Float16 scA, biA, scB, biB;
    load_batch(b, wA, scA, biA);
    while (true) {
        const int64_t b1 = b + gridDim.x;
        if (b1 < nb) load_batch(b1, wB, scB, biB);
        sum_batch(b, wA, scA, biA, 0);
        if (b1 >= nb) break;
        const int64_t b2 = b1 + gridDim.x;
        if (b2 < nb) load_batch(b2, wA, scA, biA);
        sum_batch(b1, wB, scB, biB, 1);
        if (b2 >= nb) break;
        b = b2;
    }
}

// Streamed GEMV launch: grid = min(batches, mult workgroups per CU).
template <int MR, int R, int KF>
hipError_t launch_gemv_stream(const W8A16Args& a, hipStream_t stream, int mult) {
    if (a.width != KF) return hipErrorInvalidValue;
    constexpr int kT = (KF / 16 + 63) / 64 * 64;
    const int64_t nb = (a.columns + R - 1) / R;
    const int64_t cap = (int64_t)num_cus() * mult;
    const int64_t grid = nb < cap ? nb : cap;
    hipLaunchKernelGGL((w8a16_gemv_stream_kernel<MR, R, KF>), dim3((unsigned)grid), dim3(kT), 0, stream, a);
    return hipGetLastError();
}

// OMNI_W8A16_GEMV=<cpl><r> (e.g. 14 = one chunk per lane, four rows per
// workgroup; <1><r><b> with b batches per workgroup; 9<r><m> the streamed
// GEMV, r = 4 or 8 rows a batch, m workgroups per CU, 2..4 rows at K = 4096
// or 14336) pins the int8 GEMV configuration, OMNI_F16_GEMV the f16 one
// (tuning knobs, omni::knob; unset = heuristic).
int gemv_cfg_override(int wb) { return knob(wb == 8 ? Knob::W8A16Gemv : Knob::F16Gemv, 0); }

template <int MR, int CPL, int R, int WB, int B = 1, int KF = 0>
hipError_t launch_gemv_cfg(const W8A16Args& a, hipStream_t stream) {
    if (KF > 0 && a.width != KF) return hipErrorInvalidValue;
    const int64_t chunks = a.width / (WB == 8 ? 16 : 8);
    const int64_t lanes = (chunks + CPL - 1) / CPL;
    const int64_t T = ((lanes + 63) / 64) * 64;
    if (T > 1024) return hipErrorInvalidValue;  // the caller bounds width
    const int64_t grid = (a.columns + R * B - 1) / (R * B);
    hipLaunchKernelGGL((w8a16_gemv_kernel<MR, CPL, R, WB, B, KF>), dim3((unsigned)grid), dim3((unsigned)T), 0,
                       stream, a);
    return hipGetLastError();
}

// One-row decode at the widths of the benchmarked models' linears (int8:
// 4096, 14336 and the small VLM's 1536, 8960; f16: the 8192-wide depth
// GEMV) runs the kernel built for that K.
template <int MR, int CPL, int R, int WB, int B = 1>
hipError_t launch_gemv_k(const W8A16Args& a, hipStream_t stream) {
    if constexpr (MR == 1 && WB == 8) {
        if (a.width == 4096) return launch_gemv_cfg<MR, CPL, R, WB, B, 4096>(a, stream);
        if (a.width == 14336) return launch_gemv_cfg<MR, CPL, R, WB, B, 14336>(a, stream);
        if (a.width == 1536) return launch_gemv_cfg<MR, CPL, R, WB, B, 1536>(a, stream);
        if (a.width == 8960) return launch_gemv_cfg<MR, CPL, R, WB, B, 8960>(a, stream);
    }
    if constexpr (MR == 1 && WB == 16) {
        if (a.width == 8192) return launch_gemv_cfg<MR, CPL, R, WB, B, 8192>(a, stream);
    }
    return launch_gemv_cfg<MR, CPL, R, WB, B>(a, stream);
}

template <int MR, int WB>
hipError_t launch_gemv_m(const W8A16Args& a, hipStream_t stream) {
    switch (gemv_cfg_override(WB)) {
        case 11: return launch_gemv_cfg<MR, 1, 1, WB>(a, stream);
        case 12: return launch_gemv_cfg<MR, 1, 2, WB>(a, stream);
        case 14: return launch_gemv_cfg<MR, 1, 4, WB>(a, stream);
        case 18: return launch_gemv_cfg<MR, 1, 8, WB>(a, stream);
        case 21: return launch_gemv_cfg<MR, 2, 1, WB>(a, stream);
        case 22: return launch_gemv_cfg<MR, 2, 2, WB>(a, stream);
        case 24: return launch_gemv_cfg<MR, 2, 4, WB>(a, stream);
        case 41: return launch_gemv_cfg<MR, 4, 1, WB>(a, stream);
        case 142: return launch_gemv_cfg<MR, 1, 4, WB, 2>(a, stream);
        case 144: return launch_gemv_cfg<MR, 1, 4, WB, 4>(a, stream);
        case 124: return launch_gemv_cfg<MR, 1, 2, WB, 4>(a, stream);
        case 182: return launch_gemv_cfg<MR, 1, 8, WB, 2>(a, stream);
        case 242: return launch_gemv_cfg<MR, 2, 4, WB, 2>(a, stream);
        case 222: return launch_gemv_cfg<MR, 2, 2, WB, 2>(a, stream);
        default: break;
    }
    if constexpr (WB == 8 && MR >= 2) {
        // 9RM: the streamed GEMV with R = 4 (R digit 4) or 8 (8), M workgroups per CU.
        const int ov = gemv_cfg_override(WB);
        if (ov >= 900 && ov <= 999 && (a.width == 4096 || a.width == 14336)) {
            const int rr = (ov / 10) % 10, mult = ov % 10;
            if (mult >= 1 && (rr == 4 || rr == 8)) {
                if (a.width == 4096)
                    return rr == 8 ? launch_gemv_stream<MR, 8, 4096>(a, stream, mult)
                                   : launch_gemv_stream<MR, 4, 4096>(a, stream, mult);
                return rr == 8 ? launch_gemv_stream<MR, 8, 14336>(a, stream, mult)
                               : launch_gemv_stream<MR, 4, 14336>(a, stream, mult);
            }
        }
    }
    const int64_t chunks = a.width / (WB == 8 ? 16 : 8);
    if constexpr (WB == 16) {
        // f16 weights: 2048 chunks (K = 16384) fit one chunk each of 1024
        // lanes twice over; wider rows take four chunks per lane.
        if (chunks > 2048) return launch_gemv_cfg<MR, 4, 1, WB>(a, stream);
        if (chunks > 1024) return launch_gemv_cfg<MR, 2, 2, WB>(a, stream);
        if (a.columns * a.width * 2 <= (4 << 20)) return launch_gemv_cfg<MR, 1, 2, WB>(a, stream);
        if (MR == 4) return launch_gemv_cfg<MR, 1, 8, WB>(a, stream);
        return launch_gemv_k<MR, 1, 4, WB>(a, stream);
    }
    // Measured on MI355X over the BASELINE decode shapes: 64 bytes of weights
    // in flight per lane, two chunks per lane once a row is wider than 512
    // chunks, and more, smaller workgroups when the whole matrix is a few MB.
    // Four activation rows: two batches per workgroup (x is then re-read
    // from L2 for a fraction of the weight bytes): batches of 4 rows up to
    // 512 chunks and 64 M weights (17 % faster than batches of 8 at
    // 4096 x 4096, 5 % at 4096 x 14336), batches of 8 beyond (the 128256-row
    // head, K = 14336).
    if (a.columns * a.width <= (4 << 20)) return launch_gemv_k<MR, 2, 1, WB>(a, stream);
    // Two to four rows at K = 4096 on up to 64 M weights: the streamed GEMV
    // with eight weight rows a batch and up to eight workgroups per CU, which
    // at these sizes is one batch per workgroup (MI355X, weights rotated past
    // the MALL: 4096 x 4096 5.54 against 5.90 us at M = 4, 5.02 against 5.20
    // at M = 2; 4096 x 14336 13.0-13.3 against 13.2-14.1 at M = 4, 11.1
    // against 11.6 at M = 2). On the 128256-row head it is 12 % slower.
    if constexpr (MR >= 2) {
        if (a.width == 4096 && a.columns * a.width <= (64 << 20)) return launch_gemv_stream<MR, 8, 4096>(a, stream, 8);
    }
    if (MR == 4 && chunks <= 512 && a.columns * a.width <= (64 << 20))
        return launch_gemv_cfg<MR, 1, 4, WB, 2>(a, stream);
    if (MR == 4 && chunks <= 1024) return launch_gemv_cfg<MR, 1, 8, WB, 2>(a, stream);
    if (chunks > 512) return launch_gemv_k<MR, 2, 4, WB>(a, stream);
    return launch_gemv_k<MR, 1, 4, WB>(a, stream);
}

// ---------------------------------------------------------------------------
// Skinny GEMM (5..64 activation rows): GEMV-shaped, on fp16 MFMA.
// ---------------------------------------------------------------------------

typedef float v4f_t __attribute__((ext_vector_type(4)));

// MB blocks of 16 activation rows. A 1024-lane workgroup owns 16 weight rows
// (output columns) n0..n0+15 and splits K over its 16 waves in steps of 64
// (wave w takes steps w, w + 16, ...). Per step a lane loads 16 weight codes
// (row n0 + lane % 16, k = k0 + 16 (lane / 16) .. +16) and the same 16 k of
// activation row lane % 16 of each block, and feeds two
// v_mfma_f32_16x16x32_f16: the first on codes 0..7 of every lane, the second
// on codes 8..15. Within one MFMA the hardware's k order is its own, but A and
// B use the same lane-to-k map, so each product pairs matching k and the 64
// k of the step are summed exactly once. The 16 waves' 16 x 16 partial tiles
// are reduced through LDS; scale (and bias) are applied once per output.
// WB = 16: f16 weights (32 bytes per lane per step), no scale.
template <int MB, int WB = 8>
__global__ __launch_bounds__(1024) void w8a16_skinny_kernel(W8A16Args a) {
    __shared__ float s_part[16][MB][256];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t K = a.width;
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int r16 = lane & 15, g = lane >> 4;
    const int64_t wn = n0 + r16 < a.columns ? n0 + r16 : a.columns - 1;  // clamped: never stored
    const uint8_t* wrow = reinterpret_cast<const uint8_t*>(a.w) + wn * K * (WB / 8);
    const _Float16* xrow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int64_t m = mb * 16 + r16 < a.rows ? mb * 16 + r16 : a.rows - 1;  // clamped: never stored
        xrow[mb] = a.x + m * K;
    }
    v4f_t acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
    const int64_t steps = (K + 63) / 64;
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    // P steps per trip, all their loads issued before any MFMA (a wave's
    // steps are 16 apart, so a trip covers 16 P consecutive steps of the
    // workgroup): at K = 4096 every load of the workgroup is in flight at
    // once. Steps past K load nothing and meet zeros.
    constexpr int P = MB <= 2 ? 4 : 2;
    auto load = [&](int64_t st, v4u (&wv)[WB / 8], uint4 (&xv)[MB][2]) {
        const int64_t k = st * 64 + 16 * g;
        // K % 16 == 0: a lane's 16-element block is wholly inside or outside.
        if (k < K) {
#pragma unroll
            for (int u = 0; u < WB / 8; ++u)
                wv[u] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wrow + k * (WB / 8)) + u);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                xv[mb][0] = reinterpret_cast<const uint4*>(xrow[mb] + k)[0];
                xv[mb][1] = reinterpret_cast<const uint4*>(xrow[mb] + k)[1];
            }
        } else {
#pragma unroll
            for (int u = 0; u < WB / 8; ++u) wv[u] = v4u{0u, 0u, 0u, 0u};
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) xv[mb][0] = xv[mb][1] = make_uint4(0, 0, 0, 0);
        }
    };
    auto compute = [&](const v4u (&wv)[WB / 8], const uint4 (&xv)[MB][2]) {
        v8h b0, b1;
        if constexpr (WB == 8) {
            v2h h[8];
            i8x4_to_f16x4(wv[0].x, h[0], h[1]);
            i8x4_to_f16x4(wv[0].y, h[2], h[3]);
            i8x4_to_f16x4(wv[0].z, h[4], h[5]);
            i8x4_to_f16x4(wv[0].w, h[6], h[7]);
            b0 = v8h{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
            b1 = v8h{h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
        } else {
            __builtin_memcpy(&b0, &wv[0], 16);
            __builtin_memcpy(&b1, &wv[WB / 8 - 1], 16);
        }
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            v8h a0, a1;
            __builtin_memcpy(&a0, &xv[mb][0], 16);
            __builtin_memcpy(&a1, &xv[mb][1], 16);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc[mb], 0, 0, 0);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc[mb], 0, 0, 0);
        }
    };
    for (int64_t st = wave; st < steps; st += 16 * P) {
        v4u wv[P][WB / 8];
        uint4 xv[P][MB][2];
#pragma unroll
        for (int p = 0; p < P; ++p) load(st + 16 * p, wv[p], xv[p]);
#pragma unroll
        for (int p = 0; p < P; ++p) compute(wv[p], xv[p]);
    }
    // 16 x 16 accumulator layout: lane holds column lane % 16, rows
    // 4 (lane / 16) .. +3.
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_part[wave][mb][(4 * g + r) * 16 + r16] = acc[mb][r];
    __syncthreads();
    if (tid < MB * 256) {
        const int mb = tid >> 8, e = tid & 255;
        const int64_t m = mb * 16 + (e >> 4), n = n0 + (e & 15);
        if (m < a.rows && n < a.columns) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < 16; ++w) sum += s_part[w][mb][e];
            const float bi = a.bias ? (float)a.bias[n] : 0.0f;
            const float sc = WB == 8 ? (float)a.scale[n] : 1.0f;
            a.out[m * a.columns + n] = (_Float16)(sum * sc + bi);
        }
    }
}

// Skinny GEMM for up to 16 activation rows with K <= 4096, K % 64 == 0: the
// layout of w8a16_skinny_kernel (16 weight rows per 1024-lane workgroup, K
// split over 16 waves in steps of 64, two v_mfma_f32_16x16x32_f16 per step),
// but the activations x[0:16][0:K] are first staged into LDS by contiguous
// 16-byte loads (every fetched line used whole), rows padded by 16 bytes so
// that the 16 lanes reading one fragment column hit distinct banks; the x
// loads go out before the weight loads, so x is in LDS while the weights
// stream. The per-wave 16 x 16 partials are then reduced through the same
// LDS. Measured on MI355X at 16 x 4096 x 4096: 7.2 us against 8.1 us for the
// per-wave fragment loads of w8a16_skinny_kernel. KF > 0 builds the kernel
// for K == KF, a multiple of 1024: every wave then has KF / 1024 steps and
// every lane KF / 512 x pieces, so no range check or clamp is left and the
// LDS holds 16 rows of KF (16 x 4096 x 4096: 7.05 us against 7.50 for the
// same kernel with K read at run time).
constexpr int kSkinnyLdsMaxK = 4096;

template <int WB, int KF = 0>
__global__ __launch_bounds__(1024) void w8a16_skinny_lds_kernel(W8A16Args a) {
    static_assert(KF % 1024 == 0 && KF <= kSkinnyLdsMaxK, "KF: a multiple of 1024 up to the maximum");
    constexpr int kK = KF > 0 ? KF : kSkinnyLdsMaxK;   // K the LDS and the unrolled loops are sized for
    constexpr int RS = kK * 2 + 16;                     // LDS bytes per x row
    constexpr int kMaxPieces = 16 * kK / 8 / 1024;      // 16-byte x pieces per lane
    constexpr int kMaxSteps = kK / 64 / 16;             // K steps per wave
    __shared__ __attribute__((aligned(16))) uint8_t sx[16 * RS];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t K = KF > 0 ? KF : a.width;
    const int steps = (int)(K / 64);
    const int pieces_per_row = (int)(K / 8);
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int r16 = lane & 15, g = lane >> 4;
    // Piece idx of the flat x[0:16][0:K] is x[row][8 col .. 8 col + 8) with
    // row = idx / pieces_per_row, taken as trunc((idx + 1/2) / pieces_per_row)
    // in f32: idx < 2^13 and pieces_per_row >= 8 keep the quotient at least
    // 1/(2 pieces_per_row) from an integer, far beyond the f32 error, so it
    // is exact without an integer division per piece.
    const float inv_ppr = 1.0f / (float)pieces_per_row;
    int rowv[kMaxPieces], colv[kMaxPieces];
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i) {
        const int idx = i * 1024 + tid;
        rowv[i] = KF > 0 ? idx / (KF / 8) : (int)(((float)idx + 0.5f) * inv_ppr);
        colv[i] = idx - rowv[i] * pieces_per_row;
    }
    // x first (rows past the activations are zero), then the weights.
    uint4 xv[kMaxPieces];
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i) {
        xv[i] = make_uint4(0, 0, 0, 0);
        if ((KF > 0 || rowv[i] < 16) && rowv[i] < a.rows)
            xv[i] = reinterpret_cast<const uint4*>(a.x + rowv[i] * K)[colv[i]];
    }
    const int64_t wn = n0 + r16 < a.columns ? n0 + r16 : a.columns - 1;  // clamped: never stored
    const uint8_t* wrow = reinterpret_cast<const uint8_t*>(a.w) + wn * K * (WB / 8);
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u wv[kMaxSteps][WB / 8];
#pragma unroll
    for (int j = 0; j < kMaxSteps; ++j) {
        const int st = wave + 16 * j;
        const int64_t k = (int64_t)(KF > 0 || st < steps ? st : steps - 1) * 64 + 16 * g;
#pragma unroll
        for (int u = 0; u < WB / 8; ++u)
            wv[j][u] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wrow + k * (WB / 8)) + u);
    }
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i)
        if (KF > 0 || rowv[i] < 16) *reinterpret_cast<uint4*>(sx + rowv[i] * RS + colv[i] * 16) = xv[i];
    __syncthreads();
    v4f_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kMaxSteps; ++j) {
        const int st = wave + 16 * j;
        if (KF == 0 && st >= steps) break;  // wave-uniform
        v8h b0, b1;
        if constexpr (WB == 8) {
            v2h h[8];
            i8x4_to_f16x4(wv[j][0].x, h[0], h[1]);
            i8x4_to_f16x4(wv[j][0].y, h[2], h[3]);
            i8x4_to_f16x4(wv[j][0].z, h[4], h[5]);
            i8x4_to_f16x4(wv[j][0].w, h[6], h[7]);
            b0 = v8h{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
            b1 = v8h{h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
        } else {
            __builtin_memcpy(&b0, &wv[j][0], 16);
            __builtin_memcpy(&b1, &wv[j][WB / 8 - 1], 16);
        }
        const uint8_t* px = sx + r16 * RS + (64 * st + 16 * g) * 2;
        v8h a0, a1;
        __builtin_memcpy(&a0, px, 16);
        __builtin_memcpy(&a1, px + 16, 16);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc1, 0, 0, 0);
    }
    __syncthreads();  // every wave is done with x; its LDS now holds the partials
    float* s_part = reinterpret_cast<float*>(sx);  // [16 waves][256]
    // 16 x 16 accumulator layout: lane holds column lane % 16, rows 4 (lane / 16) .. +3.
#pragma unroll
    for (int r = 0; r < 4; ++r) s_part[wave * 256 + (4 * g + r) * 16 + r16] = acc0[r] + acc1[r];
    __syncthreads();
    if (tid < 256) {
        const int64_t m = tid >> 4, n = n0 + (tid & 15);
        if (m < a.rows && n < a.columns) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < 16; ++w) sum += s_part[w * 256 + tid];
            const float bi = a.bias ? (float)a.bias[n] : 0.0f;
            const float sc = WB == 8 ? (float)a.scale[n] : 1.0f;
            a.out[m * a.columns + n] = (_Float16)(sum * sc + bi);
        }
    }
}

// Split-K skinny GEMM for up to 16 activation rows (int8 weights): a unit
// is 64 columns x KS = K / splits of K (KS % 64 == 0, 256 <= KS <= 1024), so each
// CU takes in 16 x KS x 2 bytes of x and 64 x KS bytes of weights (at
// 16 x 4096 x 4096 and four splits: 32 KB + 64 KB, against 128 KB + 64 KB
// for a 16-column unit over all of K). The x slice is staged into LDS as in
// w8a16_skinny_lds_kernel; wave w takes column block w % 4 (16 columns) and
// K quarter w / 4 in 64-element steps, two v_mfma_f32_16x16x32_f16 per step;
// the four quarters are added through LDS and the unit's f32 sums go to
// partial[split][row][column], which w8a16_split_reduce_kernel adds in
// order before scale and bias. WB = 4 (W4A16): 16 codes (8 bytes) per lane
// per step, dequantised to f16(q * s) with their group's scale, loaded
// beside them; the reduction then adds only the bias.
constexpr int kSkinnySplitMaxKS = 1024;

// KSF > 0 builds the kernel for units of exactly KSF = 1024 values of K:
// every wave then has four steps and every lane two x pieces, with no range
// check.
template <int WB = 8, int KSF = 0>
__global__ __launch_bounds__(1024) void w8a16_skinny_split_kernel(W8A16Args a, int splits) {
    static_assert(KSF == 0 || KSF == kSkinnySplitMaxKS, "KSF: the whole unit size");
    constexpr int RS = kSkinnySplitMaxKS * 2 + 16;  // LDS bytes per x row
    constexpr int kMaxPieces = 16 * kSkinnySplitMaxKS / 8 / 1024;
    constexpr int kMaxSteps = kSkinnySplitMaxKS / 4 / 64;
    __shared__ __attribute__((aligned(16))) uint8_t sx[16 * RS];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int64_t K = a.width;
    const int KS = KSF > 0 ? KSF : (int)(K / splits);
    const int tiles_n = (int)((a.columns + 63) / 64);
    const int sp = (int)(blockIdx.x / tiles_n);
    const int64_t n0 = (int64_t)(blockIdx.x % tiles_n) * 64;
    const int64_t k0 = (int64_t)sp * KS;
    const int cb = wave & 3, kq = wave >> 2;
    // The unit's KS / 64 steps of 64 elements split over the four K
    // quarters as evenly as they go (KS >= 256: every quarter has one).
    const int s_lo = kq * (KS / 64) / 4, steps = KSF > 0 ? KSF / 256 : (kq + 1) * (KS / 64) / 4 - s_lo;
    const int r16 = lane & 15, g = lane >> 4;
    const int pieces_per_row = KS / 8;
    // Piece idx of x[0:16][k0 : k0 + KS] is 8 consecutive values; row =
    // idx / pieces_per_row exactly via f32 (idx < 2^11, pieces_per_row >= 32).
    const float inv_ppr = 1.0f / (float)pieces_per_row;
    uint4 xv[kMaxPieces];
    int rowv[kMaxPieces], colv[kMaxPieces];
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i) {
        const int idx = i * 1024 + tid;
        rowv[i] = KSF > 0 ? idx / (KSF / 8) : (int)(((float)idx + 0.5f) * inv_ppr);
        colv[i] = idx - rowv[i] * pieces_per_row;
        xv[i] = make_uint4(0, 0, 0, 0);
        if ((KSF > 0 || rowv[i] < 16) && rowv[i] < a.rows)
            xv[i] = *reinterpret_cast<const uint4*>(a.x + rowv[i] * K + k0 + 8 * colv[i]);
    }
    const int64_t wn = min(n0 + 16 * cb + r16, a.columns - 1);  // clamped: never stored
    const int64_t kw = k0 + 64 * s_lo;  // this wave's first k
    const uint8_t* wrow = reinterpret_cast<const uint8_t*>(a.w) + (wn * K + kw) * WB / 8;
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    v4u wv[WB == 8 ? kMaxSteps : 1];
    typedef unsigned v2u __attribute__((ext_vector_type(2)));
    v2u wq[WB == 4 ? kMaxSteps : 1];
    uint16_t sq[WB == 4 ? kMaxSteps : 1];
#pragma unroll
    for (int j = 0; j < kMaxSteps; ++j) {
        const int st = KSF > 0 || j < steps ? j : steps - 1;
        if constexpr (WB == 8) {
            wv[j] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wrow + 64 * st + 16 * g));
        } else {
            wq[j] = __builtin_nontemporal_load(reinterpret_cast<const v2u*>(wrow + 32 * st + 8 * g));
            // (32-bit divisions: K < 2^31 on this path)
            sq[j] = a.gscale[wn * (int64_t)((unsigned)K / (unsigned)a.group) +
                             (unsigned)(kw + 64 * st + 16 * g) / (unsigned)a.group];
        }
    }
#pragma unroll
    for (int i = 0; i < kMaxPieces; ++i)
        if (KSF > 0 || rowv[i] < 16) *reinterpret_cast<uint4*>(sx + rowv[i] * RS + colv[i] * 16) = xv[i];
    __syncthreads();
    v4f_t acc0 = {0.0f, 0.0f, 0.0f, 0.0f}, acc1 = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kMaxSteps; ++j) {
        if (KSF == 0 && j >= steps) break;  // uniform
        v2h h[8];
        if constexpr (WB == 8) {
            i8x4_to_f16x4(wv[j].x, h[0], h[1]);
            i8x4_to_f16x4(wv[j].y, h[2], h[3]);
            i8x4_to_f16x4(wv[j].z, h[4], h[5]);
            i8x4_to_f16x4(wv[j].w, h[6], h[7]);
        } else {
            i4x16_dequant(wq[j].x, wq[j].y, (_Float16)bf16_to_f32(sq[j]), h);
        }
        const v8h b0 = v8h{h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
        const v8h b1 = v8h{h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
        const uint8_t* px = sx + r16 * RS + (64 * (s_lo + j) + 16 * g) * 2;
        v8h a0, a1;
        __builtin_memcpy(&a0, px, 16);
        __builtin_memcpy(&a1, px + 16, 16);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc1, 0, 0, 0);
    }
    __syncthreads();  // every wave is done with x; its LDS now holds the partials
    float* s_part = reinterpret_cast<float*>(sx);  // [16 waves][256]
    // 16 x 16 accumulator layout: lane holds column lane % 16, rows 4 (lane / 16) .. +3.
#pragma unroll
    for (int r = 0; r < 4; ++r) s_part[wave * 256 + (4 * g + r) * 16 + r16] = acc0[r] + acc1[r];
    __syncthreads();
    {
        const int c4 = tid >> 8, within = tid & 255;  // column block, (row, column) in it
        const int64_t m = within >> 4, n = n0 + 16 * c4 + (within & 15);
        if (m < a.rows && n < a.columns) {
            float sum = 0.0f;
#pragma unroll
            for (int q = 0; q < 4; ++q) sum += s_part[(4 * q + c4) * 256 + within];
            a.partial[((int64_t)sp * a.rows + m) * a.columns + n] = sum;
        }
    }
}

template <int WB = 8>
hipError_t launch_skinny_split(const W8A16Args& a, int splits, hipStream_t stream);
int cu_count();

// Split count for the split-K skinny kernel (1: not split): rows <= 16, int8
// weights, K / splits a multiple of 64 from 256 to 1024, and the partial
// sums fit the workspace. By default it splits only where the unsplit
// LDS-staged kernel (16 columns per workgroup, K <= 4096) needs two or more
// rounds of workgroups: measured on MI355X, 16 x 4096 -> 14336 21.7 us split
// four ways against 25.7, 16 x 2048 -> 8192 9.4 against 10.5, 16 x 3584 ->
// 18944 (896-element units) 24.9 against 29.3, but config 1 (16 x 4096 ->
// 4096, one round) 9.6 against 7.8, and 8 x 3584 -> 4608 12.3 against 10.6:
// one round is bound by the cold fetch of x and the first weight latency, not
// by the x traffic the split saves, and the reduction launch adds ~1.5 us.
// OMNI_W8A16_SKINNY_SPLIT=<n> pins n (0: off; test aid, a tuning knob).
int skinny_splits(int64_t rows, int64_t width, int64_t columns, int64_t partial_elems, int cus) {
    if (rows > 16 || width % 64 != 0) return 1;
    int want = knob(Knob::W8A16SkinnySplit, -1);
    if (want == 0) return 1;
    if (want < 0) {
        if (width > kSkinnyLdsMaxK || columns < 32LL * cus) return 1;
        want = 1;
        while (width / want > kSkinnySplitMaxKS) want *= 2;
    }
    if (want < 2 || width % (64LL * want) != 0 || width / want < 256 || width / want > kSkinnySplitMaxKS)
        return 1;
    if (want * rows * columns > partial_elems) return 1;
    return want;
}

// OMNI_W8A16_SKINNY=1 keeps 5..16-row calls on w8a16_skinny_kernel instead
// of the LDS-staged kernel (test aid; a tuning knob).
int skinny_route() { return knob(Knob::W8A16Skinny, 0); }

template <int MB, int WB>
hipError_t launch_skinny_cfg(const W8A16Args& a, hipStream_t stream) {
    const int64_t grid = (a.columns + 15) / 16;
    hipLaunchKernelGGL((w8a16_skinny_kernel<MB, WB>), dim3((unsigned)grid), dim3(1024), 0, stream, a);
    return hipGetLastError();
}

template <int WB>
hipError_t launch_skinny(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    if constexpr (WB == 8) {
        const int sp = skinny_splits(a.rows, a.width, a.columns, a.partial ? a.partial_elems : 0, cu_count());
        if (sp > 1) return launch_skinny_split(a, sp, stream);
    }
    if (a.rows <= 16 && a.width % 64 == 0 && a.width <= kSkinnyLdsMaxK && skinny_route() != 1) {
        const dim3 grid((unsigned)((a.columns + 15) / 16)), block(1024);
        switch (a.width) {
            case 1024: hipLaunchKernelGGL((w8a16_skinny_lds_kernel<WB, 1024>), grid, block, 0, stream, a); break;
            case 2048: hipLaunchKernelGGL((w8a16_skinny_lds_kernel<WB, 2048>), grid, block, 0, stream, a); break;
            case 3072: hipLaunchKernelGGL((w8a16_skinny_lds_kernel<WB, 3072>), grid, block, 0, stream, a); break;
            case 4096: hipLaunchKernelGGL((w8a16_skinny_lds_kernel<WB, 4096>), grid, block, 0, stream, a); break;
            default: hipLaunchKernelGGL((w8a16_skinny_lds_kernel<WB>), grid, block, 0, stream, a);
        }
        return hipGetLastError();
    }
    if (a.rows <= 16) return launch_skinny_cfg<1, WB>(a, stream);
    if (a.rows <= 32) return launch_skinny_cfg<2, WB>(a, stream);
    if (a.rows <= 48) return launch_skinny_cfg<3, WB>(a, stream);
    return launch_skinny_cfg<4, WB>(a, stream);
}

// ---------------------------------------------------------------------------
// W4A16: packed int4 weights, bf16 scales per group of K values.
// ---------------------------------------------------------------------------

// Decode GEMV (rows <= 4) for int4 weights: the W8A16 GEMV's design with 32
// codes (16 bytes) per lane per row: a lane's 32-value chunk lies in one
// scale group (group % 32 == 0), so the chunk's dot is taken on the codes
// (with more weight rows than activation rows per lane: as 1024 + nibble,
// less 1032 * sum(x) once per chunk, four VALU per eight codes fewer than
// exact decoding) and multiplied by its scale once. Products
// are exact and the f32 sums stay below 2^13 * sum|x|, so the correction
// costs ~1e-4 of the result relative and nothing on integer data. A
// workgroup of T = 64 * ceil(K / 2048) lanes owns R weight rows; every weight
// load is issued up front. KF > 0 and GF > 0 build the kernel for K == KF,
// a multiple of 2048 (every lane then owns one chunk), and group == GF: no
// clamp, and the scale index without a 64-bit division.
// TEAMS > 1 (K == KF builds only): the workgroup holds TEAMS teams of
// T = KF / 32 lanes, team t taking the R * B rows after team t - 1's, so a
// 2-wave team's rows share a workgroup (and its launch) with the next team's
// (MI355X, 4096 x 4096: 3.71 against 3.88 us with one team of 4 rows). KF
// builds are bounded by their exact workgroup size.
template <int MR, int R, int B = 1, int KF = 0, int GF = 0, int TEAMS = 1>
__global__ __launch_bounds__(KF > 0 ? KF / 32 * TEAMS : 1024) void w4a16_gemv_kernel(W8A16Args a) {
    constexpr int V = R * MR;
    constexpr int RB = R * B;  // rows per team: B batches of R
    static_assert((V & (V - 1)) == 0 && V <= 64, "power-of-two partial count");
    static_assert(KF % 2048 == 0 && (KF == 0) == (GF == 0), "KF: a multiple of 2048, with GF");
    static_assert(TEAMS == 1 || (KF > 0 && KF / 32 * TEAMS <= 1024), "teams: K == KF builds within 1024 lanes");
    __shared__ float s_part[16][B * V];
    typedef unsigned v4u __attribute__((ext_vector_type(4)));
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int T = KF > 0 ? KF / 32 : (int)blockDim.x;
    const int team = TEAMS > 1 ? tid / T : 0;
    const int tt = TEAMS > 1 ? tid - team * T : tid;  // lane within the team
    const int64_t K = KF > 0 ? KF : a.width;
    const int64_t group = GF > 0 ? GF : a.group;
    const int64_t chunks = K / 32;
    const int64_t gpr = K / group;  // scale groups per weight row
    const int64_t n0 = ((int64_t)blockIdx.x * TEAMS + team) * RB;
    const bool live = KF > 0 || tt < chunks;
    const int64_t c = live ? tt : chunks - 1;  // clamped: meets zero activations

    // x: 32 halves of each row's chunk as 16 f16 pairs, in the order of
    // i4x8_to_f16x8_biased's weight pairs: (x0, x2), (x1, x3), (x4, x6),
    // (x5, x7) of every eight; xc = 1032 * (their sum), accumulated in the
    // same pair order as the dot products it corrects.
    // The re-pairing and xc cost 32 VALU per activation row and save 16 per
    // weight row, so they pay when a lane has more weight rows than
    // activation rows; otherwise x keeps its order and codes are exact.
    constexpr bool kBiased = RB > MR;
    // Every load goes out before any arithmetic: x's raw chunks (rows past
    // a.rows read row 0, zeroed below, so no load sits in a branch), then the
    // group scales, then the weights. (With x loaded and re-paired inside a
    // per-row branch, the generated code waited for x before issuing a single
    // weight load; MI355X, 4096 x 4096: 3.88 against 4.15 us, 4 rows at
    // 4096 x 14336: 13.0 against 14.35, 14336 x 4096: 8.5 against 8.3.) The scales come
    // before the weights because memory operations retire in order: a scale
    // issued after every weight row would hold row 0's arithmetic until the
    // last row had landed.
    uint4 xq[MR][4];
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const int64_t mr = m < a.rows ? m : 0;
        const uint4* p = reinterpret_cast<const uint4*>(a.x + mr * K + c * 32);
#pragma unroll
        for (int q = 0; q < 4; ++q) xq[m][q] = p[q];
    }
    v4u wv[RB];
    float sc[RB];
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int64_t n = n0 + r < a.columns ? n0 + r : a.columns - 1;
        sc[r] = bf16_to_f32(a.gscale[n * gpr + (c * 32) / group]);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
        const int64_t n = n0 + r < a.columns ? n0 + r : a.columns - 1;
        wv[r] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(a.w + n * (K / 2) + c * 16));
    }
    __builtin_amdgcn_sched_barrier(0);
    v2h xr[MR][16];
    float xc[MR];
    const v2h k1032 = {(_Float16)1032.0f, (_Float16)1032.0f};
#pragma unroll
    for (int m = 0; m < MR; ++m) {
        const bool keep = live && m < a.rows;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint4 v = keep ? xq[m][q] : make_uint4(0, 0, 0, 0);
            if constexpr (kBiased) {
                xr[m][4 * q] = bits_half2(__builtin_amdgcn_perm(v.y, v.x, 0x05040100u));
                xr[m][4 * q + 1] = bits_half2(__builtin_amdgcn_perm(v.y, v.x, 0x07060302u));
                xr[m][4 * q + 2] = bits_half2(__builtin_amdgcn_perm(v.w, v.z, 0x05040100u));
                xr[m][4 * q + 3] = bits_half2(__builtin_amdgcn_perm(v.w, v.z, 0x07060302u));
            } else {
                xr[m][4 * q] = bits_half2(v.x);
                xr[m][4 * q + 1] = bits_half2(v.y);
                xr[m][4 * q + 2] = bits_half2(v.z);
                xr[m][4 * q + 3] = bits_half2(v.w);
            }
        }
        xc[m] = 0.0f;
        if constexpr (kBiased) {
#pragma unroll
            for (int e = 0; e < 16; ++e) xc[m] = __builtin_amdgcn_fdot2(k1032, xr[m][e], xc[m], false);
        }
    }
    const u32 k64 = 0x64646464u;
    const int64_t n_ep = min(n0 + (tt / MR) % RB, a.columns - 1);
    const _Float16 bi_h = a.bias ? a.bias[n_ep] : (_Float16)0.0f;

#pragma unroll
    for (int b = 0; b < B; ++b) {
    float part[V];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        float d[MR];
#pragma unroll
        for (int m = 0; m < MR; ++m) d[m] = 0.0f;
        const v4u wq = wv[b * R + r];
        const u32 words[4] = {wq.x, wq.y, wq.z, wq.w};
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            v2h h[4];
            if constexpr (kBiased)
                i4x8_to_f16x8_biased(words[q], k64, h);
            else
                i4x8_to_f16x8(words[q], h);
#pragma unroll
            for (int m = 0; m < MR; ++m)
#pragma unroll
                for (int j = 0; j < 4; ++j) d[m] = __builtin_amdgcn_fdot2(h[j], xr[m][4 * q + j], d[m], false);
        }
#pragma unroll
        for (int m = 0; m < MR; ++m) part[r * MR + m] = (d[m] - xc[m]) * sc[b * R + r];
    }
    Fold<V, 32>::run(part, lane);
    if ((lane & (64 / V - 1)) == 0) s_part[wave][b * V + fold_index<V>(lane)] = part[0];
    }
    __syncthreads();
    if (tt < B * V) {
        const int r = tt / MR, m = tt % MR;
        const int64_t n = n0 + r;
        if (n < a.columns && m < a.rows) {
            float acc = 0.0f;
            for (int w = 0; w < T / 64; ++w) acc += s_part[team * (T / 64) + w][tt];
            a.out[(int64_t)m * a.columns + n] = (_Float16)(acc + (float)bi_h);
        }
    }
}

// Skinny GEMM (5..64 rows) for int4 weights: the W8A16 skinny kernel with
// 16 codes (8 bytes) per lane per 64-value K step, dequantised to f16(q * s).
template <int MB>
__global__ __launch_bounds__(1024) void w4a16_skinny_kernel(W8A16Args a) {
    __shared__ float s_part[16][MB][256];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int64_t K = a.width;
    const int64_t gpr = K / a.group;
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int r16 = lane & 15, g = lane >> 4;
    const int64_t wn = n0 + r16 < a.columns ? n0 + r16 : a.columns - 1;  // clamped: never stored
    const uint8_t* wrow = reinterpret_cast<const uint8_t*>(a.w) + wn * (K / 2);
    const uint16_t* srow = a.gscale + wn * gpr;
    const _Float16* xrow[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        const int64_t m = mb * 16 + r16 < a.rows ? mb * 16 + r16 : a.rows - 1;
        xrow[mb] = a.x + m * K;
    }
    v4f_t acc[MB];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) acc[mb] = v4f_t{0.0f, 0.0f, 0.0f, 0.0f};
    const int64_t steps = (K + 63) / 64;
    auto step = [&](int64_t st) {
        const int64_t k = st * 64 + 16 * g;
        uint2 wv = make_uint2(0x88888888u, 0x88888888u);  // codes 0
        _Float16 s = (_Float16)0.0f;
        uint4 xv[MB][2];
        if (k < K) {  // K % 16 == 0: a lane's 16 values are wholly inside or outside
            wv = *reinterpret_cast<const uint2*>(wrow + k / 2);
            s = (_Float16)bf16_to_f32(srow[k / a.group]);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                xv[mb][0] = reinterpret_cast<const uint4*>(xrow[mb] + k)[0];
                xv[mb][1] = reinterpret_cast<const uint4*>(xrow[mb] + k)[1];
            }
        } else {
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) xv[mb][0] = xv[mb][1] = make_uint4(0, 0, 0, 0);
        }
        v2h h[8];
        i4x16_dequant(wv.x, wv.y, s, h);
        const v8h b0 = {h[0][0], h[0][1], h[1][0], h[1][1], h[2][0], h[2][1], h[3][0], h[3][1]};
        const v8h b1 = {h[4][0], h[4][1], h[5][0], h[5][1], h[6][0], h[6][1], h[7][0], h[7][1]};
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            v8h a0, a1;
            __builtin_memcpy(&a0, &xv[mb][0], 16);
            __builtin_memcpy(&a1, &xv[mb][1], 16);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0, acc[mb], 0, 0, 0);
            acc[mb] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a1, b1, acc[mb], 0, 0, 0);
        }
    };
    int64_t st = wave;
    for (; st + 16 < steps; st += 32) {
        step(st);
        step(st + 16);
    }
    if (st < steps) step(st);
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int r = 0; r < 4; ++r) s_part[wave][mb][(4 * g + r) * 16 + r16] = acc[mb][r];
    __syncthreads();
    if (tid < MB * 256) {
        const int mb = tid >> 8, e = tid & 255;
        const int64_t m = mb * 16 + (e >> 4), n = n0 + (e & 15);
        if (m < a.rows && n < a.columns) {
            float sum = 0.0f;
#pragma unroll
            for (int w = 0; w < 16; ++w) sum += s_part[w][mb][e];
            const float bi = a.bias ? (float)a.bias[n] : 0.0f;
            a.out[m * a.columns + n] = (_Float16)(sum + bi);
        }
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
// WBITS 8: int8 weights, per-column f16 scale in the epilogue; WBITS 4:
// packed int4 weights dequantised to f16(q * s) per K group while staged;
// WBITS 16: f16 weights staged as they are (the fp16 linear), no scale.
template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GROUP_M, int WBITS = 8>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N, 1) void w8a16_mfma_kernel(W8A16Args a) {
    constexpr int kThreads = 64 * WAVES_M * WAVES_N;
    constexpr int WM = BM / WAVES_M, WN = BN / WAVES_N;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int kRowBytes = BK * 2;
    constexpr int kChunks = kRowBytes / 16;  // 16-byte chunks (8 halves) per row
    static_assert(kChunks == 8, "BK = 64 halves");
    constexpr int kALoads = BM * kChunks / kThreads;        // x: 8 halves per load
    constexpr int kBPer = WBITS == 16 ? 8 : 16;             // weights per B load
    constexpr int kBLoads = BN * (BK / kBPer) / kThreads;
    static_assert(kALoads * kThreads == BM * kChunks, "even A loads");
    static_assert(kBLoads * kThreads == BN * (BK / kBPer), "even B loads");

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
            const int r = id / (BK / kBPer), c = id % (BK / kBPer);
            const int64_t gr = n0 + r, gk = k0 + c * kBPer;
            if constexpr (WBITS == 16) {
                const _Float16* wh = reinterpret_cast<const _Float16*>(a.w);
                rb[i] = (gr < a.columns && gk < K) ? *reinterpret_cast<const uint4*>(wh + gr * K + gk)
                                                   : make_uint4(0, 0, 0, 0);
            } else if constexpr (WBITS == 8) {
                rb[i] = (gr < a.columns && gk < K) ? *reinterpret_cast<const uint4*>(a.w + gr * K + gk)
                                                   : make_uint4(0, 0, 0, 0);
            } else {
                // 16 codes = 8 bytes, and their group's bf16 scale in .z
                if (gr < a.columns && gk < K) {
                    const uint2 q = *reinterpret_cast<const uint2*>(a.w + gr * (K / 2) + gk / 2);
                    rb[i] = make_uint4(q.x, q.y, a.gscale[gr * (K / a.group) + gk / a.group], 0);
                } else {
                    rb[i] = make_uint4(0x88888888u, 0x88888888u, 0, 0);  // codes 0
                }
            }
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
            const int r = id / (BK / kBPer), c = id % (BK / kBPer);
            if constexpr (WBITS == 16) {
                *reinterpret_cast<uint4*>(dB + r * kRowBytes + swz(r, c) * 16) = rb[i];
            } else {
                // 16 codes -> 16 halves = two 16-byte chunks 2c and 2c+1.
                v2h h[8];
                if constexpr (WBITS == 8) {
                    const u32 words[4] = {rb[i].x, rb[i].y, rb[i].z, rb[i].w};
#pragma unroll
                    for (int q = 0; q < 4; ++q) i8x4_to_f16x4(words[q], h[2 * q], h[2 * q + 1]);
                } else {
                    i4x16_dequant(rb[i].x, rb[i].y, (_Float16)bf16_to_f32((uint16_t)rb[i].z), h);
                }
                uint4 lo = make_uint4(half2_bits(h[0]), half2_bits(h[1]), half2_bits(h[2]), half2_bits(h[3]));
                uint4 hi = make_uint4(half2_bits(h[4]), half2_bits(h[5]), half2_bits(h[6]), half2_bits(h[7]));
                *reinterpret_cast<uint4*>(dB + r * kRowBytes + swz(r, 2 * c) * 16) = lo;
                *reinterpret_cast<uint4*>(dB + r * kRowBytes + swz(r, 2 * c + 1) * 16) = hi;
            }
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
        // int4: scaled per group already; f16: no scale
        const float sc = WBITS == 8 ? (float)a.scale[col] : 1.0f;
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

// Persistent LDS-DMA ring GEMM on fp16 MFMA (K % 64 == 0), the W8A8 ring
// kernel's pipeline with an f16 activation operand. One workgroup of 4 waves
// (2 x 2) per CU walks BM x BN output tiles; each wave owns a BM/2 x BN/2
// block of 32x32 f32 accumulators. A K tile is 64 elements: the stage holds
// x's k 0..31 and k 32..63 as two [BM][64-byte] halves and W as one
// [BN][64-byte] block, all copied by global_load_lds_dwordx4 with the W8A8
// ring's XOR swizzle of 16-byte chunks, in a 3-stage ring.
//
// Fragments, per pair p of 16-k MFMA steps (k 32p .. 32p+31 of the tile):
// lane (row r = lane % 32, h = lane / 32) reads W codes 32p + 16h .. +16 of
// column r (one ds_read_b128, chunk 2p + h) and x halves 32p + 16h .. +16 of
// row r (two ds_read_b128, chunks 2h and 2h + 1 of half p). The first
// v_mfma_f32_32x32x16_f16 takes codes and halves 0..7, the second 8..15: A and
// B share one lane-to-k map, so every product pairs matching k and the 32 k
// of the pair are summed once. Codes become f16 exactly in registers (v_perm
// and one subtract, as in the GEMV): a pair's codes are read before its x
// halves and converted four at a time in the MFMA slots of the pair before
// the one that uses them, so the conversion overlaps MFMAs instead of
// preceding them. The schedule is the W8A8 ring's: one
// fragment read and one copy behind each MFMA, one barrier per K tile between
// the two pairs, the next tile's first copies issued before the epilogue. A
// stage is refilled as soon as the barrier after its last fragment reads has
// passed (tile kt+S into stage kt % S), so two tiles are in flight.
//
// WB = 16 (the fp16 linear): W is f16 and staged like x, as two [BN][64-byte]
// halves, and its fragments are read like x's (two ds_read_b128 per pair);
// there is no scale.
// KP = 1 (f16 weights only): K tiles of 32 elements, one MFMA pair each, so
// a stage is half as large and a 256 x 256 tile fits three of them.
//
// OCC = 2 (tiles whose ring fits half the LDS): two workgroups share a CU
// (at most 256 registers per lane each), so one workgroup's prologue and
// epilogue overlap the other's K loop; the persistent grid is two per CU.
//
// SK (split K, `splits` > 1): the work units are (tile, split) pairs, split s
// covering K tiles [s * kts, min(ktiles, (s + 1) * kts)) with kts =
// ceil(ktiles / splits) (the host keeps every split non-empty); a unit stores
// its unscaled f32 sums to partial[s][rows][columns] and
// w8a16_split_reduce_kernel adds the splits in order and applies scale and
// bias. Units of one split are consecutive, so the workgroups of an XCD
// share that split's K range of x and W.
//
// NW = 8: eight waves (two per SIMD) share the ring, each owning half as
// many accumulators, so one wave's MFMAs can issue while the other waits.
//
// WB = 4 (W4A16, packed int4 codes plus 8, low nibble first, bf16 scales per
// group of `group` values along K, group % 64 == 0): a K tile's 64 codes are
// 32 bytes per weight row, so one 64-byte stage row holds two weight rows
// (logical chunks 0, 1: the even row's bytes 0..15, 16..31; 2, 3: the odd
// row's), copied with the same swizzle. A lane's 16 codes of a pair are one
// 8-byte read; they become f16(q * s) (nibble as 1024 + n, minus 1032, times
// the group scale in f16), four codes at a time spread over the MFMA slots
// of the pair before the one that uses them, so the conversion overlaps the
// MFMAs. The scales ride in the ring too: behind each stage's
// rows, the aligned bf16 pair holding the tile's group for every column (one
// 4-byte-per-lane copy per wave per K tile, 64 columns each).
template <int BM, int BN, int WB = 8, int WMW = 2, int S = 3, int KP = 2, int OCC = 1, bool SK = false, int NW = 4>
__global__ __launch_bounds__(64 * NW, OCC) void w8a16_ring_kernel(W8A16Args a, int splits) {
    static_assert(S == 2 || S == 3, "2 or 3 stages");
    static_assert(KP == 2 || (KP == 1 && WB == 16), "32-element K tiles need f16 weights");
    static_assert(WB == 4 || WB == 8 || WB == 16, "int4, int8 or f16 weights");
    constexpr int WNW = NW / WMW;             // waves along N
    constexpr int WM = BM / WMW, WN = BN / WNW;
    constexpr int FM = WM / 32, FN = WN / 32;
    constexpr int kWH = WB == 16 ? 2 : 1;     // 64-byte W rows per column per 64 K (int4: half of one)
    constexpr int kXR = KP;                   // 64-byte x rows per row per K tile
    constexpr int kWR = KP == 2 ? kWH : 1;    // 64-byte W rows per column per K tile
    constexpr int kWRows = WB == 4 ? BN / 2 : kWR * BN;  // W stage rows per K tile
    constexpr int kWBytes = 32 * KP * WB / 8;  // bytes of a W row per K tile
    constexpr int kRows = kXR * BM + kWRows;  // 64-byte stage rows: x k 0..31 (, x k 32..63), W
    constexpr int kScOff = kRows * 64;        // int4: scale dwords [BN] behind the rows
    constexpr int kStage = kRows * 64 + (WB == 4 ? BN * 4 : 0);
    constexpr int kCpw = kRows / (16 * NW);   // 1 KiB copies per wave per K tile
    constexpr int kOps = kCpw + (WB == 4 ? 1 : 0);  // vector-memory ops per wave per K tile
    constexpr int kFrags = 2 * FM + kWH * FN; // fragment reads per pair
    static_assert(kRows % (16 * NW) == 0 && FM >= 1 && FN >= 1 && WMW * WNW == NW, "tile shape");
    static_assert(kCpw <= 2 * FM * FN && kFrags <= 2 * FM * FN, "one read and copy per MFMA slot");
    static_assert((S - 1) * kOps < 64, "ops in flight within vmcnt");
    static_assert(WB != 4 || (KP == 2 && FM >= 2 && BN % 64 == 0 && BN <= 64 * NW), "int4 ring shape");
    // int4 and int8 codes: converted ahead, spread over the previous pair's
    // MFMA slots (int8: 3-16 % faster than converting at the start of the
    // pair on the four-wave and the eight-wave 256 x 256 rings, MI355X).
    constexpr bool kPipe = WB == 4 || WB == 8;
    constexpr int FN4 = kPipe ? FN : 1;
    static_assert(S * kStage + 4 * BN * 4 <= 160 * 1024 / OCC, "LDS");
    __shared__ __attribute__((aligned(1024))) uint8_t st0[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t st1[kStage];
    __shared__ __attribute__((aligned(1024))) uint8_t st2[S > 2 ? kStage : 1024];
    __shared__ float sScale[2][BN];
    __shared__ float sBias[2][BN];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave / WNW, wn = wave % WNW;
    const int tiles_m = (int)((a.rows + BM - 1) / BM);
    const int tiles_n = (int)((a.columns + BN - 1) / BN);
    const int total = tiles_m * tiles_n;
    const int units = SK ? total * splits : total;
    const int64_t K = a.width;
    const int ktiles_all = (int)(K / (32 * KP));
    const int kts = SK ? (ktiles_all + splits - 1) / splits : ktiles_all;
    // K tiles [kbase, kbase + ktiles) of the unit being copied; split index.
    int kbase = 0, ktiles = ktiles_all, split = 0;
    const bool has_bias = a.bias != nullptr;
    constexpr int kGroupM = 4;
    auto stage = [&](int s) -> uint8_t* { return s == 0 ? st0 : s == 1 ? st1 : st2; };
    const unsigned stage_lds[3] = {lds_addr(st0), lds_addr(st1), S > 2 ? lds_addr(st2) : 0u};

    // Copy c fills stage rows 16c .. 16c+15; lane l reads logical chunk
    // (l % 4) ^ ((l / 16) % 4) of row l / 4, landing at physical chunk l % 4.
    const int cp_row = lane >> 2;
    const int cp_chunk = (lane & 3) ^ ((lane >> 4) & 3);
    unsigned voff[kCpw];
    unsigned voff_sc = 0;  // int4: this lane's scale column, byte offset of its row
    int64_t m0 = 0, n0 = 0;
    // A tile's column scales and biases, held between their load and their
    // store into the idle parameter buffer: kPP per thread, as BN may exceed
    // the workgroup's 64 * NW threads (column tid + 64 NW i for slot i).
    constexpr int kPP = (BN + 64 * NW - 1) / (64 * NW);
    float p_sc[kPP], p_bi[kPP];
#pragma unroll
    for (int i = 0; i < kPP; ++i) p_sc[i] = p_bi[i] = 0.0f;
    auto tile_origin = [&](int u, int64_t& tm0, int64_t& tn0) {
        const int l = SK ? u % total : u;
        const int group_size = kGroupM * tiles_n;
        const int first_m = (l / group_size) * kGroupM;
        const int gm = min(tiles_m - first_m, kGroupM);
        tm0 = (int64_t)__builtin_amdgcn_readfirstlane(first_m + (l % group_size) % gm) * BM;
        tn0 = (int64_t)__builtin_amdgcn_readfirstlane((l % group_size) / gm) * BN;
    };
    // The wave's j-th copy fills stage block slot(j) (rows 16 slot .. +15).
    // On 256-row tiles the issue order pairs the two 64-byte halves of the
    // same 16 rows (x, and W when it is f16): a wave copies half 0 and then
    // half 1 of one row block, so the second read finds the 128-byte lines
    // the first one brought into the CU's L1 (MI355X, 4096 x 4096 x 12288:
    // 1-4 % faster). Smaller tiles keep block order, in which two waves copy
    // the two halves side by side (pairing there measured 3-7 % slower on
    // config 5's M = 1024 shapes).
    auto slot = [&](int j) -> int {
        const int g = wave * kCpw + j;  // wave-uniform
        constexpr int nx = kXR * BM / 16, nw = kWR * BN / 16;
        // (An odd kCpw lets one pair straddle two waves: still correct.)
        if constexpr (KP == 2 && BM >= 256) {
            if (g < nx) return (g & 1) * (BM / 16) + (g >> 1);
            if constexpr (WB == 16) {
                const int gw = g - nx;
                if (gw < nw) return nx + (gw & 1) * (BN / 16) + (gw >> 1);
            }
        }
        return g;
    };
    // Copy j reads one matrix (x or W, wave-uniform) at a per-lane 32-bit byte
    // offset from its base (the host keeps both matrices under 4 GiB); the K
    // tile advance is added to the scalar base.
    auto setup_copies = [&]() {
#pragma unroll
        for (int j = 0; j < kCpw; ++j) {
            const int c16 = slot(j) * 16;  // wave-uniform
            if (c16 < kXR * BM) {
                const int half = c16 >= BM;
                const int64_t row = min(m0 + (c16 - half * BM) + cp_row, a.rows - 1);
                voff[j] = (unsigned)(row * K * 2) + half * 64 + cp_chunk * 16;
            } else if constexpr (WB == 4) {
                // stage row rel + cp_row holds weight rows 2 (rel + cp_row) and +1
                const int rel = c16 - kXR * BM;
                const int64_t row = min(n0 + 2 * (rel + cp_row) + (cp_chunk >> 1), a.columns - 1);
                voff[j] = (unsigned)(row * (K / 2)) + (cp_chunk & 1) * 16;
            } else {
                const int rel = c16 - kXR * BM;
                const int half = WB == 16 && rel >= BN;
                const int64_t row = min(n0 + (rel - half * BN) + cp_row, a.columns - 1);
                voff[j] = (unsigned)(row * K * kWH) + half * 64 + cp_chunk * 16;
            }
        }
        if constexpr (WB == 4) {
            const int64_t col = min(n0 + (wave % (BN / 64)) * 64 + lane, a.columns - 1);
            voff_sc = (unsigned)(col * (K / a.group) * 2);
        }
    };
    auto load_params = [&](int64_t pn0) {
#pragma unroll
        for (int i = 0; i < kPP; ++i) {
            const int c = tid + 64 * NW * i;
            if (c < BN) {
                const int64_t col = min(pn0 + c, a.columns - 1);
                p_sc[i] = WB == 8 ? (float)a.scale[col] : 1.0f;
                p_bi[i] = has_bias ? (float)a.bias[col] : 0.0f;
            }
        }
    };
    auto store_params = [&](int par) {
#pragma unroll
        for (int i = 0; i < kPP; ++i) {
            const int c = tid + 64 * NW * i;
            if (c < BN) {
                sScale[par][c] = p_sc[i];
                sBias[par][c] = p_bi[i];
            }
        }
    };
    auto unit_k = [&](int u) {
        if constexpr (SK) {
            split = __builtin_amdgcn_readfirstlane(u / total);
            kbase = split * kts;
            ktiles = min(kts, ktiles_all - kbase);
        }
    };
    // int4: group of K tile kk (a scale pair holds groups 2i, 2i + 1).
    const int gdiv = WB == 4 ? (int)(a.group / 64) : 1;
    auto copy_one = [&](int kt, int s, int j) {
        const int64_t kk = kbase + min(kt, ktiles - 1);
        const int c = slot(j);
        const bool is_x = c * 16 < kXR * BM;  // wave-uniform
        const uint8_t* base = is_x ? reinterpret_cast<const uint8_t*>(a.x) + kk * 64 * KP
                                   : reinterpret_cast<const uint8_t*>(a.w) + kk * kWBytes;
        lds_copy16_saddr(voff[j], base, stage_lds[s] + c * 1024);
        if constexpr (WB == 4) {
            if (j == kCpw - 1) {
                const int g = (int)kk / gdiv;
                lds_copy4_saddr(voff_sc, a.gscale + (g & ~1),
                                stage_lds[s] + kScOff + (wave % (BN / 64)) * 256);
            }
        }
    };
    auto copy_tile = [&](int kt, int s) {
#pragma unroll
        for (int j = 0; j < kCpw; ++j) copy_one(kt, s, j);
    };

    // Fragment offsets within a stage.
    const int fr = lane & 31, fh = lane >> 5, fq = (fr >> 2) & 3;
    auto offA = [&](int p, int j) { return (p * BM + wm * WM + fr) * 64 + (((2 * fh + j) ^ fq) << 4); };
    auto offB = [&](int p) { return (kXR * BM + wn * WN + fr) * 64 + (((2 * p + fh) ^ fq) << 4); };
    auto offB16 = [&](int p, int j) {
        return (kXR * BM + p * BN + wn * WN + fr) * 64 + (((2 * fh + j) ^ fq) << 4);
    };
    // int4: column c = wn WN + fr (+ 32 per block) sits in stage row c / 2,
    // logical chunk 2 (c % 2) + p, whose swizzle key is (c / 8) % 4.
    auto offB4 = [&](int p) {
        return (kXR * BM + (wn * WN + fr) / 2) * 64 + ((((fr & 1) * 2 + p) ^ ((fr >> 3) & 3)) << 4) + 8 * fh;
    };
    v4i xa0[FM][2], xb0[FN][kWH], xa1[FM][2], xb1[FN][kWH];
    v8h bh0[FN4][2], bh1[FN4][2];  // int4 / int8: converted codes of a pair
    uint16_t sc[FN4];              // int4: the K tile's bf16 scales (read with pair 0's codes)
    // Fragment idx of a pair: f16 weights read A (i, j) for idx < 2 FM, then
    // B block (idx - 2 FM) / 2, half (idx - 2 FM) % 2; int8 and int4 codes
    // read their B blocks first, idx < FN (int4 with pair 0: the tile's
    // scales too), then A idx - FN. kt is the K tile in stage s.
    auto read_frag = [&](int s, int p, int idx, v4i (&xa)[FM][2], v4i (&xb)[FN][kWH], int kt) {
        if constexpr (kPipe) {
            if (idx < FN) {
                if constexpr (WB == 8) {
                    xb[idx][0] = *reinterpret_cast<const v4i*>(stage(s) + offB(p) + idx * 32 * 64);
                } else {
                    const uint2 w2 = *reinterpret_cast<const uint2*>(stage(s) + offB4(p) + idx * 16 * 64);
                    xb[idx][0] = v4i{(int)w2.x, (int)w2.y, 0, 0};
                    if (p == 0) {
                        const int g = (int)(kbase + kt) / gdiv;
                        sc[idx] = *reinterpret_cast<const uint16_t*>(stage(s) + kScOff +
                                                                     (wn * WN + 32 * idx + fr) * 4 + (g & 1) * 2);
                    }
                }
            } else {
                const int i = idx - FN;
                xa[i >> 1][i & 1] = *reinterpret_cast<const v4i*>(stage(s) + offA(p, i & 1) + (i >> 1) * 32 * 64);
            }
        } else if (idx < 2 * FM) {
            xa[idx >> 1][idx & 1] =
                *reinterpret_cast<const v4i*>(stage(s) + offA(p, idx & 1) + (idx >> 1) * 32 * 64);
        } else {
            const int b = idx - 2 * FM;
            xb[b >> 1][b & 1] = *reinterpret_cast<const v4i*>(stage(s) + offB16(p, b & 1) + (b >> 1) * 32 * 64);
        }
    };

    // Piece pc of a pair's conversion: codes 4 (pc % 4) .. +3 of block pc / 4
    // (int4: i4x8_to_f16x8's steps, then times the scale, eight VALU ops;
    // int8: i8x4_to_f16x4, five).
    auto conv4 = [&](int pc, v4i (&xb)[FN][kWH], v8h (&bh)[FN4][2]) {
        if constexpr (WB == 4) {
            const int jn = pc >> 2, w = (pc >> 1) & 1, hc = pc & 1;
            const u32 word = (u32)xb[jn][0][w];
            const u32 c = __builtin_amdgcn_perm(word >> 4, word, hc ? 0x07030602u : 0x05010400u) & 0x0F0F0F0Fu;
            const v2h k1032 = {(_Float16)1032.0f, (_Float16)1032.0f};
            const _Float16 sh = (_Float16)bf16_to_f32(sc[jn]);  // (converted at first use)
            const v2h s2 = {sh, sh};
            const v2h h0 = (bits_half2(__builtin_amdgcn_perm(0x64646464u, c, 0x04010400u)) - k1032) * s2;
            const v2h h1 = (bits_half2(__builtin_amdgcn_perm(0x64646464u, c, 0x04030402u)) - k1032) * s2;
            bh[jn][w][4 * hc] = h0[0];
            bh[jn][w][4 * hc + 1] = h0[1];
            bh[jn][w][4 * hc + 2] = h1[0];
            bh[jn][w][4 * hc + 3] = h1[1];
        } else if constexpr (WB == 8) {
            const int jn = pc >> 2, q = pc & 3;
            v2h h0, h1;
            i8x4_to_f16x4((u32)xb[jn][0][q], h0, h1);
            bh[jn][q >> 1][4 * (q & 1)] = h0[0];
            bh[jn][q >> 1][4 * (q & 1) + 1] = h0[1];
            bh[jn][q >> 1][4 * (q & 1) + 2] = h1[0];
            bh[jn][q >> 1][4 * (q & 1) + 3] = h1[1];
        }
    };
    // After MFMA slot q: the conversion pieces that slot carries, spread
    // evenly from slot 3 on (block jn's codes are read at slot jn).
    auto conv_at = [&](int q, v4i (&xb)[FN][kWH], v8h (&bh)[FN4][2]) {
        if constexpr (kPipe) {
            constexpr int ns = 2 * FM * FN, np = 4 * FN, c0 = 3;
#pragma unroll
            for (int i = 0; i < np; ++i)
                if (c0 + i * (ns - c0) / np == q) conv4(i, xb, bh);
        }
    };
    v16f acc[FM][FN];
    // One pair of MFMA steps on fragments xa and xb (f16 weights, fed to the
    // MFMA straight from their fragment registers) or bq (int8 / int4 codes
    // converted during the previous pair), with one read (and one copy, and
    // conversion pieces) issued after each MFMA. The k 0..7 products of all
    // FM x FN blocks run, then the k 8..15 ones, so no MFMA waits for the one
    // just before it (two back-to-back MFMAs into one accumulator would
    // serialise).
    auto pair_mfmas = [&](v4i (&xa)[FM][2], v4i (&xb)[FN][kWH], const v8h (&bq)[FN4][2], auto&& after) {
#pragma unroll
        for (int half = 0; half < 2; ++half) {
#pragma unroll
            for (int jn = 0; jn < FN; ++jn) {
#pragma unroll
                for (int i = 0; i < FM; ++i) {
                    v8h av, bv;
                    __builtin_memcpy(&av, &xa[i][half], 16);
                    if constexpr (kPipe)
                        bv = bq[jn][half];
                    else
                        __builtin_memcpy(&bv, &xb[jn][half * (kWH - 1)], 16);
                    acc[i][jn] = __builtin_amdgcn_mfma_f32_32x32x16_f16(av, bv, acc[i][jn], 0, 0, 0);
                    after(half * FM * FN + jn * FM + i);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    };

    int L = xcd_remap(blockIdx.x, gridDim.x);
    if (L >= units) return;
    tile_origin(L, m0, n0);
    unit_k(L);
    setup_copies();
    load_params(n0);
    store_params(0);
#pragma unroll
    for (int u = 0; u < S; ++u) copy_tile(u, u);
    int parity = 0;

    while (true) {
        const int Ln = L + gridDim.x;
        const bool more = Ln < units;
        int64_t nm0 = 0, nn0 = 0;
        if (more) {
            tile_origin(Ln, nm0, nn0);
            load_params(nn0);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = v16f{};

        s_waitcnt_vm<(S - 1) * kOps, true>();
        lds_barrier();
#pragma unroll
        for (int idx = 0; idx < kFrags; ++idx) read_frag(0, 0, idx, xa0, xb0, 0);
#pragma unroll
        for (int pc = 0; pc < 4 * FN4; ++pc) conv4(pc, xb0, bh0);

        if constexpr (KP == 2) {
            for (int t0 = 0; t0 < ktiles; t0 += S) {
#pragma unroll
                for (int u = 0; u < S; ++u) {
                    const int kt = t0 + u;
                    if (kt < ktiles) {  // uniform across the workgroup
                        // Pair 0 of tile kt; reads of pair 1.
                        pair_mfmas(xa0, xb0, bh0, [&](int q) {
                            if (q < kFrags) read_frag(u, 1, q, xa1, xb1, kt);
                            conv_at(q, xb1, bh1);
                        });
                        s_waitcnt_vm<(S - 2) * kOps, true>();
                        lds_barrier();  // tile kt+1 landed everywhere; stage u is read
                        // Pair 1 of tile kt; copies of tile kt+S into stage u; reads of tile kt+1, pair 0.
                        pair_mfmas(xa1, xb1, bh1, [&](int q) {
                            if (q < kCpw) copy_one(kt + S, u, q);
                            if (q < kFrags) read_frag((u + 1) % S, 0, q, xa0, xb0, kt + 1);
                            conv_at(q, xb0, bh0);
                        });
                    }
                }
            }
        } else {
            // One pair per K tile; the fragment buffers alternate by tile, so
            // the unrolled body covers 2 S tiles (stage kt % S, buffer kt % 2).
            for (int t0 = 0; t0 < ktiles; t0 += 2 * S) {
#pragma unroll
                for (int u2 = 0; u2 < 2 * S; ++u2) {
                    const int kt = t0 + u2;
                    const int u = u2 % S;
                    if (kt < ktiles) {  // uniform across the workgroup
                        // Tile kt's fragments were read during tile kt-1: once
                        // tile kt+1 has landed and every wave has passed here,
                        // stage u may be refilled with tile kt+S.
                        s_waitcnt_vm<(S - 2) * kOps, true>();
                        lds_barrier();
                        if (u2 % 2 == 0) {
                            pair_mfmas(xa0, xb0, bh0, [&](int q) {
                                if (q < kCpw) copy_one(kt + S, u, q);
                                if (q < kFrags) read_frag((u + 1) % S, 0, q, xa1, xb1, kt + 1);
                            });
                        } else {
                            pair_mfmas(xa1, xb1, bh1, [&](int q) {
                                if (q < kCpw) copy_one(kt + S, u, q);
                                if (q < kFrags) read_frag((u + 1) % S, 0, q, xa0, xb0, kt + 1);
                            });
                        }
                    }
                }
            }
        }

        const int64_t em0 = m0, en0 = n0;
        const int esplit = split;
        s_waitcnt_vm<(S - 1) * kOps, true>();
        lds_barrier();  // every wave is done reading the ring
        if (more) {
            m0 = nm0;
            n0 = nn0;
            unit_k(Ln);
            setup_copies();
            store_params(parity ^ 1);
#pragma unroll
            for (int u = 0; u < S; ++u) copy_tile(u, u);
        }

        // Epilogue: out = f16(acc * scale[n] + bias[n]). 32x32 accumulator
        // layout: lane holds column lane % 32, rows 8 (r / 4) + 4 (lane / 32) + r % 4.
        // Offsets are 32-bit from the tile's first element (the host keeps
        // 256 * columns below 2^31); the lane indices pass through an empty
        // asm so the compiler does not precompute every store address.
        const float* pScale = sScale[parity];
        const float* pBias = sBias[parity];
        if constexpr (SK) {
            // Unscaled f32 sums of this split (plain stores: the reduction
            // reads them back right after).
            const int N = (int)a.columns;
            float* outt = a.partial + (int64_t)esplit * a.rows * a.columns + em0 * a.columns + en0;
            const int rows_last = (int)min((int64_t)BM, a.rows - em0) - 1;
            const int cols_last = (int)min((int64_t)BN, a.columns - en0) - 1;
            int efr = fr, efh = fh;
            asm volatile("" : "+v"(efr), "+v"(efh));
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int lc = wn * WN + j * 32 + efr;
                    const int lr0 = wm * WM + i * 32 + 4 * efh;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int lr = lr0 + 8 * (r >> 2) + (r & 3);
                        if (lc <= cols_last && lr <= rows_last) outt[(unsigned)(lr * N + lc)] = acc[i][j][r];
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        } else {
            const int N = (int)a.columns;
            _Float16* outt = a.out + em0 * a.columns + en0;
            const int rows_last = (int)min((int64_t)BM, a.rows - em0) - 1;
            const int cols_last = (int)min((int64_t)BN, a.columns - en0) - 1;
            int efr = fr, efh = fh;
            asm volatile("" : "+v"(efr), "+v"(efh));
#pragma unroll
            for (int i = 0; i < FM; ++i) {
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int lc = wn * WN + j * 32 + efr;
                    const float sc = pScale[lc];
                    const float bi = pBias[lc];
                    const int lr0 = wm * WM + i * 32 + 4 * efh;
#pragma unroll
                    for (int r = 0; r < 16; ++r) {
                        const int lr = lr0 + 8 * (r >> 2) + (r & 3);
                        if (lc <= cols_last && lr <= rows_last)
                            __builtin_nontemporal_store((_Float16)(acc[i][j][r] * sc + bi),
                                                        outt + (unsigned)(lr * N + lc));
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
        if (!more) break;
        L = Ln;
        parity ^= 1;
    }
    s_waitcnt_vm<0>();  // copies of clamped K tiles may still be landing
}

// The ring kernel's limits: 64-element K tiles, per-lane copy offsets of x
// and W rows in 32 bits, in-tile output offsets in 32 bits.
bool ring16_fits(const W8A16Args& a) {
    const int64_t lim = int64_t(1) << 32;
    return a.width % 64 == 0 && a.rows * a.width * 2 < lim && a.columns * a.width * 2 < lim &&
           a.columns < (int64_t(1) << 23);
}

// Split-K reduction: out[r][c] = f16((sum over s in order of partial[s][r][c])
// * scale[c] + bias[c]), four consecutive elements per lane.
// S > 0 builds the kernel for exactly S splits: every partial load, and the
// four columns' scales and biases, go out before the first add (with the
// split count read at run time each add waited on its own load: config 5's
// down projection, four splits, 7.2 us). The adds keep split order.
template <int S = 0>
__global__ __launch_bounds__(256) void w8a16_split_reduce_kernel(W8A16Args a, int splits) {
    const int64_t n = a.rows * a.columns;
    const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i >= n) return;
    float v[4];
    int e_end = 4;
    int64_t c = i % a.columns;
    if (a.columns % 4 == 0) {
        // The four elements are consecutive columns c .. c + 3 of one row.
        // Scale and bias are loaded unconditionally (from the partial sums,
        // in range, where a pointer is null: int4 weights are scaled in the
        // kernel), so that no load sits in a branch that waits for it.
        const bool has_sc = a.scale != nullptr, has_bi = a.bias != nullptr;
        const _Float16* sp = has_sc ? a.scale : reinterpret_cast<const _Float16*>(a.partial);
        const _Float16* bp = has_bi ? a.bias : reinterpret_cast<const _Float16*>(a.partial);
        _Float16 sh[4], bh[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            sh[e] = sp[c + e];
            bh[e] = bp[c + e];
        }
        float4 s;
        if constexpr (S > 0) {
            float4 t[S];
#pragma unroll
            for (int p = 0; p < S; ++p) t[p] = *reinterpret_cast<const float4*>(a.partial + p * n + i);
            s = t[0];
#pragma unroll
            for (int p = 1; p < S; ++p) {
                s.x += t[p].x;
                s.y += t[p].y;
                s.z += t[p].z;
                s.w += t[p].w;
            }
        } else {
            s = *reinterpret_cast<const float4*>(a.partial + i);
            for (int p = 1; p < splits; ++p) {
                const float4 t = *reinterpret_cast<const float4*>(a.partial + p * n + i);
                s.x += t.x;
                s.y += t.y;
                s.z += t.z;
                s.w += t.w;
            }
        }
        const float r[4] = {s.x, s.y, s.z, s.w};
        _Float16 o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float sc = has_sc ? (float)sh[e] : 1.0f;
            const float bi = has_bi ? (float)bh[e] : 0.0f;
            o[e] = (_Float16)(r[e] * sc + bi);
        }
        if (reinterpret_cast<uintptr_t>(a.out + i) % 8 == 0) {
            typedef _Float16 h4 __attribute__((ext_vector_type(4)));
            *reinterpret_cast<h4*>(a.out + i) = h4{o[0], o[1], o[2], o[3]};
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e) a.out[i + e] = o[e];
        }
        return;
    }
    e_end = (int)min((int64_t)4, n - i);
    for (int e = 0; e < e_end; ++e) {
        float s = a.partial[i + e];
        for (int p = 1; p < splits; ++p) s += a.partial[p * n + i + e];
        v[e] = s;
    }
    _Float16 o[4];
    for (int e = 0; e < e_end; ++e) {
        if (e > 0 && ++c == a.columns) c = 0;
        const float sc = a.scale ? (float)a.scale[c] : 1.0f;  // int4: scaled in the kernel
        const float bi = a.bias ? (float)a.bias[c] : 0.0f;
        o[e] = (_Float16)(v[e] * sc + bi);
    }
    for (int e = 0; e < e_end; ++e) a.out[i + e] = o[e];
}

// The reduction launch: the build for exactly `splits` splits from 2 to 8.
hipError_t launch_split_reduce(const W8A16Args& a, int splits, hipStream_t stream) {
    const int64_t quads = (a.rows * a.columns + 3) / 4;
    const dim3 grid((unsigned)((quads + 255) / 256)), block(256);
    switch (splits) {
        case 2: hipLaunchKernelGGL((w8a16_split_reduce_kernel<2>), grid, block, 0, stream, a, splits); break;
        case 3: hipLaunchKernelGGL((w8a16_split_reduce_kernel<3>), grid, block, 0, stream, a, splits); break;
        case 4: hipLaunchKernelGGL((w8a16_split_reduce_kernel<4>), grid, block, 0, stream, a, splits); break;
        case 5: hipLaunchKernelGGL((w8a16_split_reduce_kernel<5>), grid, block, 0, stream, a, splits); break;
        case 6: hipLaunchKernelGGL((w8a16_split_reduce_kernel<6>), grid, block, 0, stream, a, splits); break;
        case 7: hipLaunchKernelGGL((w8a16_split_reduce_kernel<7>), grid, block, 0, stream, a, splits); break;
        case 8: hipLaunchKernelGGL((w8a16_split_reduce_kernel<8>), grid, block, 0, stream, a, splits); break;
        default: hipLaunchKernelGGL((w8a16_split_reduce_kernel<0>), grid, block, 0, stream, a, splits);
    }
    return hipGetLastError();
}

template <int WB>
hipError_t launch_skinny_split(const W8A16Args& a, int splits, hipStream_t stream) {
    const int64_t units = ((a.columns + 63) / 64) * splits;
    if (a.width == (int64_t)kSkinnySplitMaxKS * splits)
        hipLaunchKernelGGL((w8a16_skinny_split_kernel<WB, kSkinnySplitMaxKS>), dim3((unsigned)units), dim3(1024), 0,
                           stream, a, splits);
    else
        hipLaunchKernelGGL((w8a16_skinny_split_kernel<WB>), dim3((unsigned)units), dim3(1024), 0, stream, a, splits);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_split_reduce(a, splits, stream);
}

int cu_count() { return num_cus(); }

// Largest split count <= want that leaves every split of ktiles K tiles
// non-empty and whose partial sums fit in a.partial_elems floats.
int fit_splits(const W8A16Args& a, int ktiles, int want) {
    int s = want < ktiles ? want : ktiles;
    while (s > 1) {
        const int kts = (ktiles + s - 1) / s;
        if ((s - 1) * kts < ktiles && a.partial && s * a.rows * a.columns <= a.partial_elems) break;
        --s;
    }
    return s < 1 ? 1 : s;
}

template <int BM, int BN, int WB = 8, int WMW = 2, int S = 3, int KP = 2, int OCC = 1, int NW = 4>
hipError_t launch_ring16_cfg(const W8A16Args& a, hipStream_t stream, int splits = 1) {
    const int64_t tiles = ((a.rows + BM - 1) / BM) * ((a.columns + BN - 1) / BN);
    const int64_t slots = (int64_t)cu_count() * OCC;
    if constexpr (WB == 8 || WB == 4) {
        // Split K when asked for and the partial sums fit (else fewer splits).
        if (splits > 1) splits = fit_splits(a, (int)(a.width / 64), splits);
        while (splits > 1 && tiles * splits > INT32_MAX) --splits;  // unit indices are int
        if (splits > 1) {
            const int64_t units = tiles * splits;
            const int64_t grid = units < slots ? units : slots;
            hipLaunchKernelGGL((w8a16_ring_kernel<BM, BN, WB, WMW, S, KP, OCC, true, NW>), dim3((unsigned)grid),
                               dim3(64 * NW), 0, stream, a, splits);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            return launch_split_reduce(a, splits, stream);
        }
    }
    const int64_t grid = tiles < slots ? tiles : slots;
    hipLaunchKernelGGL((w8a16_ring_kernel<BM, BN, WB, WMW, S, KP, OCC, false, NW>), dim3((unsigned)grid),
                       dim3(64 * NW), 0, stream, a, 1);
    return hipGetLastError();
}

template <int BM, int BN, int BK, int WAVES_M, int WAVES_N, int GROUP_M, int WBITS = 8>
hipError_t launch_mfma16_cfg(const W8A16Args& a, hipStream_t stream) {
    auto kernel = w8a16_mfma_kernel<BM, BN, BK, WAVES_M, WAVES_N, GROUP_M, WBITS>;
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
        case 1: return launch_gemv_m<1, 8>(a, stream);
        case 2: return launch_gemv_m<2, 8>(a, stream);
        default: return launch_gemv_m<4, 8>(a, stream);  // 3 rows run with one zero row
    }
}

hipError_t launch_w8a16_skinny(const W8A16Args& a, hipStream_t stream) { return launch_skinny<8>(a, stream); }

// OMNI_W8A16_TILE=<n> pins the prefill GEMM kernel (tuning and test aid):
// 1 = tiled 128 x 128, 2 = tiled 64 x 64, 4/5/6 = ring 256 x 128 / 128 x 128 /
// 256 x 256 (2 x 2 waves), 7 = ring 256 x 256 (1 x 4 waves), 8 = ring
// 64 x 128, 9 = ring 256 x 192, 10 = ring 128 x 128 two workgroups per CU,
// 11 / 12 = ring 64 x 128 two / three per CU, 16 / 17 / 18 = ring 128 x 256 /
// 256 x 256 (waves 64 x 128) / 256 x 256 (waves 128 x 64) with eight waves,
// 19 / 20 / 21 = ring 128 x 320 / 64 x 192 / 128 x 192 (rings: K % 64 == 0
// only). OMNI_W8A16_SPLITS=<n>
// adds n-way split K to a pinned ring (or to the shape rule's choice) when
// the call brings a workspace. Both are tuning knobs (omni::knob).
int w8a16_tile_override() { return knob(Knob::W8A16Tile, 0); }

// The kernel and split count launch_w8a16_mfma runs for a shape: cfg as
// OMNI_W8A16_TILE numbers them (0: the register-staged kernels), splits > 1
// for split K (needs splits * rows * columns floats of partial sums).
struct W16Plan {
    int cfg;
    int splits;
};

// ws_limited: split only as far as a.partial holds (a launch); else assume
// the workspace the plan asks for (the size query).
W16Plan plan_w8a16(const W8A16Args& a, int cus, bool ws_limited) {
    const int split_override = knob(Knob::W8A16Splits, 0);
    const bool ring_ok = ring16_fits(a);
    const int ov = w8a16_tile_override();
    if (ov == 1 || ov == 2 || (ov >= 4 && ov <= 12 && ring_ok) || (ov >= 16 && ov <= 21 && ring_ok))
        return {ov, ov >= 4 && split_override > 1 ? split_override : 1};
    if (!ring_ok) {
        const int64_t big_tiles = ((a.rows + 127) / 128) * ((a.columns + 127) / 128);
        return {big_tiles >= 512 ? 1 : 2, 1};
    }
    auto with_splits = [&](int cfg) { return W16Plan{cfg, split_override > 1 ? split_override : 1}; };
    // Split K (f32 partial sums, one reduction launch) when even 64 x 128
    // tiles leave CUs idle and K is long: 128 x 128 tiles two per CU, K split
    // 2..4 ways to about one unit per CU (MI355X, weights rotated past the
    // MALL: 1024 x 8960 -> 1536 46.9 us against 54.2 unsplit, 256 x 12288 ->
    // 4096 41.0 against 76.7, 256 x 4096 -> 4096 24.6 against 28.5). On K =
    // 1536 the partial sums' traffic costs more than the split saves.
    const int64_t tiles64 = ((a.rows + 63) / 64) * ((a.columns + 127) / 128);
    if (a.width >= 4096 && tiles64 < cus) {
        // K >= 8192 with as many 128 x 192 tiles as divide the CUs 2-4 ways:
        // those tiles split that many ways fill every CU exactly once
        // (config 5's down projection, 1024 x 8960 -> 1536: 64 tiles, four
        // splits, 40.9 us against 45.9 on 128 x 128 tiles split two ways; on
        // K = 4096, or splits that leave CUs idle, the rule below wins).
        const int64_t tiles192 = ((a.rows + 127) / 128) * ((a.columns + 191) / 192);
        if (a.width >= 8192 && split_override <= 1 && cus % tiles192 == 0) {
            const int sp = (int)(cus / tiles192);
            if (sp >= 2 && sp <= 4 && (!ws_limited || fit_splits(a, (int)(a.width / 64), sp) == sp))
                return {21, sp};
        }
        const int64_t tiles128 = ((a.rows + 127) / 128) * ((a.columns + 127) / 128);
        const int64_t want = cus / tiles128;
        const int sp = split_override > 1 ? split_override : (int)(want < 2 ? 2 : want > 4 ? 4 : want);
        if (!ws_limited || fit_splits(a, (int)(a.width / 64), sp) > 1) return {10, sp};
    }
    // Cost model over the one-workgroup-per-CU rings, fitted to MI355X
    // timings (weights rotated past the MALL) of every ring on twelve prefill
    // shapes, M 512..4096, K 1536..4096, N 1536..17920: tiles run in rounds
    // of one per CU, a round costs BM * BN * (c * K + e), a partial last
    // round with fill f costs 0.7 + 0.3 f of a full one. It picks within
    // 1.2 % of the fastest ring on all twelve (the fixed rules it replaces:
    // up to 40 % off). Candidates: 256 x 192 (four waves), 128 x 256 and
    // 256 x 256 with eight waves (two per SIMD; the 256 x 256 one measured
    // 4-15 % faster than the four-wave 256 x 256 ring with the waves side by
    // side along N on seven shapes, so it takes that ring's fit less 4 %).
    struct Cand {
        double t;
        int id;
        int64_t tiles;
    };
    auto cost = [&](int id, double c, double e, int64_t bm, int64_t bn) {
        const int64_t tiles = ((a.rows + bm - 1) / bm) * ((a.columns + bn - 1) / bn);
        const int64_t full = tiles / cus, rem = tiles % cus;
        const double rounds = (double)full + (rem ? 0.7 + 0.3 * (double)rem / (double)cus : 0.0);
        return Cand{(double)(bm * bn) * (c * (double)a.width + e) * rounds, id, tiles};
    };
    // (The 256 x 256 and 256 x 192 fits are scaled by 0.94 and 0.90: spreading
    // the code conversion over the MFMA slots made those rings 3-14 % and
    // 6-16 % faster on eight of these shapes, the 128 x 256 one 0-3 % slower.
    // The 256 x 256 candidate is then the eight-wave ring with two waves
    // along M (each 128 x 64, half the conversions per MFMA of the 64 x 128
    // one): 0.93-0.96 of that one's time on five shapes, so 0.95 of its fit.)
    // 128 x 320 (four waves of 64 x 160; 2 BM + BN = 9 x 64 stage rows, so
    // the copies divide over the waves) gives the M = 1024 and 2048 shapes
    // 8 x 28 / 16 x 28 tiles where 256 x 192 leaves a quarter of the CUs idle
    // (1024 x 1536 -> 8960: 188 tiles): fitted on MI355X at K = 1536 and
    // 4096 (1024 x K -> 8960: 36.8 / 79.1 us), it changes the pick on eight
    // of 38 swept shapes, each 5-13 % faster (1024 x 1536 -> 17920: 72.5
    // against 83.8 us), and on no other.
    Cand best = cost(18, 0.3184, 358.8, 256, 256);
    for (const Cand& c : {cost(9, 0.3846, 359.2, 256, 192), cost(16, 0.4289, 201.6, 128, 256),
                          cost(19, 0.4186, 291.4, 128, 320)})
        if (c.t < best.t) best = c;
    // At most half a round of tiles and K >= 8192: split that ring's tiles
    // 2-4 ways to about one unit per CU (1024 x 18944 -> 3584: 128 x 256
    // tiles split two ways 155.9-158.7 us, against 194.6 on 64 x 128 tiles
    // three per CU; 1024 x 14336 -> 4096: 126.8 against 153.7 unsplit).
    if (a.width >= 8192 && 2 * best.tiles <= cus) {
        const int64_t want = cus / best.tiles;
        const int sp = split_override > 1 ? split_override : (int)(want < 2 ? 2 : want > 4 ? 4 : want);
        if (!ws_limited || fit_splits(a, (int)(a.width / 64), sp) > 1) return {best.id, sp};
    }
    if (2 * best.tiles >= cus) return with_splits(best.id);
    // Fewer tiles than half the CUs: 64 x 128 tiles three workgroups per CU
    // when they fit one round of those slots (config 5's 1024 x 1536 ->
    // 1536 / 2048 / 512: 13.4 / 13.4 / 11.9 us against 20.9 / 20.8 / 19.9
    // for 128 x 256), else 128 x 256.
    if (tiles64 <= 3 * (int64_t)cus) return with_splits(12);
    return with_splits(16);
}

int64_t w8a16_skinny_partial_elems(int64_t rows, int64_t columns, int64_t width) {
    if (rows <= 0 || columns <= 0) return 0;
    const int sp = skinny_splits(rows, width, columns, INT64_MAX, cu_count());
    return sp > 1 ? (int64_t)sp * rows * columns : 0;
}

int64_t w8a16_partial_elems(int64_t rows, int64_t columns, int64_t width) {
    if (rows <= 0 || columns <= 0) return 0;
    W8A16Args a{};
    a.rows = rows;
    a.columns = columns;
    a.width = width;
    const W16Plan p = plan_w8a16(a, cu_count(), false);
    return p.cfg >= 4 && p.splits > 1 ? (int64_t)p.splits * rows * columns : 0;
}

hipError_t launch_w8a16_mfma(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    const W16Plan p = plan_w8a16(a, cu_count(), true);
    const int sp = p.splits;
    switch (p.cfg) {
        case 1: return launch_mfma16_cfg<128, 128, 64, 2, 2, 4>(a, stream);
        case 2: return launch_mfma16_cfg<64, 64, 64, 2, 2, 4>(a, stream);
        case 4: return launch_ring16_cfg<256, 128>(a, stream, sp);
        case 5: return launch_ring16_cfg<128, 128>(a, stream, sp);
        case 6: return launch_ring16_cfg<256, 256>(a, stream, sp);
        case 7: return launch_ring16_cfg<256, 256, 8, 1>(a, stream, sp);
        case 8: return launch_ring16_cfg<64, 128>(a, stream, sp);
        case 9: return launch_ring16_cfg<256, 192>(a, stream, sp);
        case 10: return launch_ring16_cfg<128, 128, 8, 2, 3, 2, 2>(a, stream, sp);
        case 11: return launch_ring16_cfg<64, 128, 8, 2, 3, 2, 2>(a, stream, sp);
        case 16: return launch_ring16_cfg<128, 256, 8, 2, 3, 2, 1, 8>(a, stream, sp);
        case 17: return launch_ring16_cfg<256, 256, 8, 4, 3, 2, 1, 8>(a, stream, sp);
        case 18: return launch_ring16_cfg<256, 256, 8, 2, 3, 2, 1, 8>(a, stream, sp);
        case 19: return launch_ring16_cfg<128, 320>(a, stream, sp);
        case 20: return launch_ring16_cfg<64, 192>(a, stream, sp);
        case 21: return launch_ring16_cfg<128, 192>(a, stream, sp);
        default: return launch_ring16_cfg<64, 128, 8, 2, 3, 2, 3>(a, stream, sp);
    }
}

hipError_t launch_w4a16_gemv(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    const int64_t chunks = a.width / 32;
    const int64_t T = ((chunks + 63) / 64) * 64;
    if (T > 1024) return hipErrorInvalidValue;  // the caller keeps width <= 32768
    // OMNI_W4A16_GEMV=<r><b> pins r rows per batch and b batches per
    // workgroup (tuning aid); unset: the measured choice below.
    int cfg = knob(Knob::W4A16Gemv, 0);
    // Measured on MI355X: 4 rows per workgroup from 4 MB of codes (7.6 us
    // at 4096 x 14336), two batches of 4 from 64 MB (43 us at the 128256-row
    // vocabulary head), 2 rows below 4 MB. With 2-4 activation rows, 8 rows
    // per workgroup from 16 MB (4096 x 14336, 4 rows: 13.4 against 15.0 us;
    // 14336 x 4096, 3 rows: 13.0 against 14.5; 4096 x 4096 stays on 4 rows,
    // 6.3 against 7.9).
    const int64_t code_bytes = a.columns * a.width / 2;
    // One row at K = 4096, group 128, from 4 MB of codes: two 128-lane teams
    // of 8 rows per workgroup (MI355X, weights rotated past the MALL, against
    // one team of 4 or 2 x 4 rows: 4096 x 4096 3.71 against 3.88 us, 4096 x
    // 14336 7.65-7.7 against 7.85, the 128256-row head 41.4-41.8 against 42.2).
    if (cfg == 0 && a.rows == 1 && a.group == 128 && a.width == 4096 && code_bytes >= (4 << 20)) {
        const dim3 grid((unsigned)((a.columns + 15) / 16)), block(256);
        hipLaunchKernelGGL((w4a16_gemv_kernel<1, 8, 1, 4096, 128, 2>), grid, block, 0, stream, a);
        return hipGetLastError();
    }
    if (cfg == 0) {
        if (code_bytes >= (64 << 20)) cfg = 42;
        else if (a.rows >= 2 && code_bytes >= (16 << 20)) cfg = 81;
        else cfg = code_bytes >= (4 << 20) ? 41 : 21;
    }
    auto go = [&](auto rt, auto bt) {
        constexpr int R = decltype(rt)::value, B = decltype(bt)::value;
        const dim3 grid((unsigned)((a.columns + R * B - 1) / (R * B))), block((unsigned)T);
        // One-row decode at the benchmarked models' widths and group 128
        // runs the kernel built for them.
        if (a.rows == 1 && a.group == 128) {
            if (a.width == 4096) {
                hipLaunchKernelGGL((w4a16_gemv_kernel<1, R, B, 4096, 128>), grid, block, 0, stream, a);
                return hipGetLastError();
            }
            if (a.width == 14336) {
                hipLaunchKernelGGL((w4a16_gemv_kernel<1, R, B, 14336, 128>), grid, block, 0, stream, a);
                return hipGetLastError();
            }
        }
        switch (a.rows) {
            case 1: hipLaunchKernelGGL((w4a16_gemv_kernel<1, R, B>), grid, block, 0, stream, a); break;
            case 2: hipLaunchKernelGGL((w4a16_gemv_kernel<2, R, B>), grid, block, 0, stream, a); break;
            default: hipLaunchKernelGGL((w4a16_gemv_kernel<4, R, B>), grid, block, 0, stream, a); break;
        }
        return hipGetLastError();
    };
    using std::integral_constant;
    switch (cfg) {
        case 11: return go(integral_constant<int, 1>{}, integral_constant<int, 1>{});
        case 21: return go(integral_constant<int, 2>{}, integral_constant<int, 1>{});
        case 41: return go(integral_constant<int, 4>{}, integral_constant<int, 1>{});
        case 42: return go(integral_constant<int, 4>{}, integral_constant<int, 2>{});
        case 44: return go(integral_constant<int, 4>{}, integral_constant<int, 4>{});
        case 82: return go(integral_constant<int, 8>{}, integral_constant<int, 2>{});
        default: return go(integral_constant<int, 8>{}, integral_constant<int, 1>{});
    }
}

// Split count for the int4 split-K skinny kernel (1: not split): rows <= 16,
// K / splits a multiple of 64 from 256 to 1024, the partial sums within the
// workspace. By default only K of 3072..4096 split (3 or 4 ways), and only
// where the unsplit kernel needs two or more rounds of 16-column
// workgroups: MI355X, 16 x 4096 -> 14336 25.2 us split four ways against
// 31.1, the 128256-row head 153 against 226, 16 x 3584 -> 18944 27.1
// against 28.2 (8 rows: 25.2 against 23.9); 8 x 2048 -> 8192 10.1 split
// two ways against 8.5. OMNI_W4A16_SKINNY_SPLIT=<n> pins n (0: off; test aid, a
// tuning knob).
int w4_skinny_splits(int64_t rows, int64_t width, int64_t columns, int64_t partial_elems, int cus) {
    if (rows > 16 || width % 64 != 0 || width >= (int64_t(1) << 31)) return 1;
    int want = knob(Knob::W4A16SkinnySplit, -1);
    if (want == 0) return 1;
    if (want < 0) {
        if (columns < 32LL * cus || width < 3072 || width > 4 * kSkinnySplitMaxKS) return 1;
        want = (int)((width + kSkinnySplitMaxKS - 1) / kSkinnySplitMaxKS);
    }
    if (want < 2 || width % (64LL * want) != 0 || width / want < 256 || width / want > kSkinnySplitMaxKS)
        return 1;
    if (want * rows * columns > partial_elems) return 1;
    return want;
}

int64_t w4a16_skinny_partial_elems(int64_t rows, int64_t columns, int64_t width) {
    if (rows <= 0 || columns <= 0) return 0;
    const int sp = w4_skinny_splits(rows, width, columns, INT64_MAX, cu_count());
    return sp > 1 ? (int64_t)sp * rows * columns : 0;
}

hipError_t launch_w4a16_skinny(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    const int sp = w4_skinny_splits(a.rows, a.width, a.columns, a.partial ? a.partial_elems : 0, cu_count());
    if (sp > 1) return launch_skinny_split<4>(a, sp, stream);
    const dim3 grid((unsigned)((a.columns + 15) / 16)), block(1024);
    if (a.rows <= 16) hipLaunchKernelGGL((w4a16_skinny_kernel<1>), grid, block, 0, stream, a);
    else if (a.rows <= 32) hipLaunchKernelGGL((w4a16_skinny_kernel<2>), grid, block, 0, stream, a);
    else if (a.rows <= 48) hipLaunchKernelGGL((w4a16_skinny_kernel<3>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((w4a16_skinny_kernel<4>), grid, block, 0, stream, a);
    return hipGetLastError();
}

// OMNI_W4A16_TILE=<n> pins the W4A16 GEMM kernel (tuning and test aid):
// 1 / 2 = tiled 128 x 128 / 64 x 64 (codes dequantized through registers),
// rings 4 / 5 / 6 = 256 x 128 / 128 x 128 / 256 x 256, 10 = 128 x 128 at
// two workgroups per CU, 16 / 17 / 18 = eight-wave 128 x 256 / 256 x 256
// (waves 64 x 128) / 256 x 256 (waves 128 x 64) (rings: K % 64 == 0, group
// % 64 == 0, K / group even, scales 4-byte aligned); OMNI_W4A16_SPLITS=<n>
// adds n-way split K to a pinned ring when the call brings a workspace.
// Both are tuning knobs (omni::knob).
struct W4Plan {
    int cfg;     // tile id as above
    int splits;  // K splits (> 1 needs a workspace)
};

// (the ring copies a column's scales as aligned bf16 pairs: an even count
// per row, from a 4-byte aligned scale array)
bool w4_ring_ok(const W8A16Args& a) {
    return ring16_fits(a) && a.group % 64 == 0 && (a.width / a.group) % 2 == 0 &&
           reinterpret_cast<uintptr_t>(a.gscale) % 4 == 0;
}

W4Plan plan_w4a16(const W8A16Args& a, int cus, bool ws_limited) {
    const int split_override = knob(Knob::W4A16Splits, 0);
    const int t = knob(Knob::W4A16Tile, 0);
    const bool ring_ok = w4_ring_ok(a);
    if (t == 1 || t == 2) return {t, 1};
    if (ring_ok && (t == 4 || t == 5 || t == 6 || t == 10 || (t >= 16 && t <= 18)))
        return {t, split_override > 1 ? split_override : 1};
    if (!ring_ok) {
        const int64_t big_tiles = ((a.rows + 127) / 128) * ((a.columns + 127) / 128);
        return {big_tiles >= 512 ? 1 : 2, 1};
    }
    // Rings 256 x 256 (eight waves, each 128 x 64) / 256 x 128 / 128 x 128,
    // each unsplit or with K split 2-4 ways, whichever a rounds cost model
    // picks: units (tiles, or tiles x splits) run in rounds of one per CU, a
    // partial last round with fill f costs 0.7 + 0.3 f of a full one, a full
    // round costs c K' + e us for K' = K / splits (MI355X fits over M =
    // 256..4096, K = 3584..18944: 0.02488 K' + 31.4, 0.01435 K' + 24.2,
    // 0.0107 K' + 8.1), and a split adds its reduction, 1 us + (4 splits + 2)
    // bytes per output at 3.5 TB/s; K < 4096 is not split. On seven long-K
    // shapes its choice is within 5 % of the fastest of the ring/split
    // choices measured on five and 13-14 % off on two (1024 x 8192 -> 4096,
    // 1024 x 8960 -> 1536); against unsplit: 1024 x 14336 -> 4096 142 us
    // against 182, 1024 x 8960 -> 1536 56 against 86.
    const int ktiles = (int)(a.width / 64);
    double best_t = 0.0;
    W4Plan best{5, 1};
    auto consider = [&](int id, int64_t bm, int64_t bn, double c, double e) {
        const int64_t tiles = ((a.rows + bm - 1) / bm) * ((a.columns + bn - 1) / bn);
        for (int sp = 1; sp <= 4; ++sp) {
            if (sp > 1 && (a.width < 4096 || (ws_limited && fit_splits(a, ktiles, sp) != sp))) break;
            const int64_t units = tiles * sp;
            const int64_t full = units / cus, rem = units % cus;
            const double rounds = (double)full + (rem ? 0.7 + 0.3 * (double)rem / (double)cus : 0.0);
            double t = rounds * (c * (double)a.width / sp + e);
            if (sp > 1) t += 1.0 + (4.0 * sp + 2.0) * (double)a.rows * (double)a.columns / 3.5e6;
            if (best_t == 0.0 || t < best_t) {
                best_t = t;
                best = {id, sp};
            }
        }
    };
    consider(18, 256, 256, 0.02488, 31.4);
    consider(4, 256, 128, 0.01435, 24.2);
    consider(5, 128, 128, 0.0107, 8.1);
    if (split_override > 1 && (!ws_limited || fit_splits(a, ktiles, split_override) > 1))
        return {best.cfg, split_override};
    return best;
}

int64_t w4a16_partial_elems(int64_t rows, int64_t columns, int64_t width, int64_t group) {
    if (rows <= 0 || columns <= 0 || group <= 0) return 0;
    W8A16Args a{};
    a.rows = rows;
    a.columns = columns;
    a.width = width;
    a.group = group;
    const W4Plan p = plan_w4a16(a, cu_count(), false);
    return p.cfg >= 4 && p.splits > 1 ? (int64_t)p.splits * rows * columns : 0;
}

hipError_t launch_w4a16_mfma(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    const W4Plan p = plan_w4a16(a, cu_count(), true);
    const int sp = p.splits;
    switch (p.cfg) {
        case 1: return launch_mfma16_cfg<128, 128, 64, 2, 2, 4, 4>(a, stream);
        case 2: return launch_mfma16_cfg<64, 64, 64, 2, 2, 4, 4>(a, stream);
        case 4: return launch_ring16_cfg<256, 128, 4>(a, stream, sp);
        case 5: return launch_ring16_cfg<128, 128, 4>(a, stream, sp);
        case 6: return launch_ring16_cfg<256, 256, 4>(a, stream, sp);
        case 10: return launch_ring16_cfg<128, 128, 4, 2, 3, 2, 2>(a, stream, sp);
        case 16: return launch_ring16_cfg<128, 256, 4, 2, 3, 2, 1, 8>(a, stream, sp);
        case 17: return launch_ring16_cfg<256, 256, 4, 4, 3, 2, 1, 8>(a, stream, sp);
        default: return launch_ring16_cfg<256, 256, 4, 2, 3, 2, 1, 8>(a, stream, sp);
    }
}

// ---------------------------------------------------------------------------
// fp16 linear: the same kernels with f16 weights and no scale.
// ---------------------------------------------------------------------------

hipError_t launch_f16_gemv(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    switch (a.rows) {
        case 1: return launch_gemv_m<1, 16>(a, stream);
        case 2: return launch_gemv_m<2, 16>(a, stream);
        default: return launch_gemv_m<4, 16>(a, stream);
    }
}

hipError_t launch_f16_skinny(const W8A16Args& a, hipStream_t stream) { return launch_skinny<16>(a, stream); }

// OMNI_F16_TILE=<n> pins the fp16 GEMM kernel (tuning and test aid):
// 1 = tiled 128 x 128, 2 = tiled 64 x 64, 4/5/6 = ring 256 x 128 / 128 x 128 /
// 128 x 256, 7/8 = ring 256 x 256 / 256 x 128 on 32-element K tiles, 10 =
// eight-wave ring 256 x 128, 12 / 13 = eight-wave ring 256 x 256 on 32- /
// 64-element K tiles, 14 = the latter with waves 128 x 64 instead of 64 x 128
// (rings: K % 64 == 0 only). A tuning knob (omni::knob).
hipError_t launch_f16_mfma(const W8A16Args& a, hipStream_t stream) {
    if (a.rows == 0 || a.columns == 0) return hipSuccess;
    const bool ring_ok = ring16_fits(a);
    switch (knob(Knob::F16Tile, 0)) {
        case 1: return launch_mfma16_cfg<128, 128, 64, 2, 2, 4, 16>(a, stream);
        case 2: return launch_mfma16_cfg<64, 64, 64, 2, 2, 4, 16>(a, stream);
        case 4: if (ring_ok) return launch_ring16_cfg<256, 128, 16>(a, stream); break;
        case 5: if (ring_ok) return launch_ring16_cfg<128, 128, 16>(a, stream); break;
        case 6: if (ring_ok) return launch_ring16_cfg<128, 256, 16>(a, stream); break;
        case 7: if (ring_ok) return launch_ring16_cfg<256, 256, 16, 2, 3, 1>(a, stream); break;
        case 8: if (ring_ok) return launch_ring16_cfg<256, 128, 16, 2, 3, 1>(a, stream); break;
        case 10: if (ring_ok) return launch_ring16_cfg<256, 128, 16, 4, 3, 2, 1, 8>(a, stream); break;
        case 12: if (ring_ok) return launch_ring16_cfg<256, 256, 16, 4, 3, 1, 1, 8>(a, stream); break;
        case 13: if (ring_ok) return launch_ring16_cfg<256, 256, 16, 4, 2, 2, 1, 8>(a, stream); break;
        case 14: if (ring_ok) return launch_ring16_cfg<256, 256, 16, 2, 2, 2, 1, 8>(a, stream); break;
        default: break;
    }
    const int64_t cus = cu_count();
    // Eight-wave rings (two waves per SIMD, each 64 x 128 or 64 x 64) on
    // 64-element K tiles (whole 128-byte lines of x and W): 256 x 256 tiles
    // in a 2-stage ring or 256 x 128 tiles in a 3-stage ring, whichever a
    // rounds cost model picks: tiles run in rounds of one per CU, a partial
    // last round with fill f costs 0.7 + 0.3 f of a full one, and a 256 x 256
    // tile costs 1.80 times a 256 x 128 one (MI355X, best of three:
    // 4096 x 4096 x 12288 334.5 / 365.0 us, torch.matmul 321.0; 4352 x 4096 x
    // 12288 408.1 / 422.8, torch.matmul 418.7; 2048 x 4096 x 4096 80.4 /
    // 64.6, torch.matmul 62.5; the 256 x 256 ring on 32-element K tiles
    // 356.9 / 433.7 / 79.4).
    if (ring_ok && a.width >= 3072) {
        auto rounds = [&](int64_t bn) {
            const int64_t tiles = ((a.rows + 255) / 256) * ((a.columns + bn - 1) / bn);
            const int64_t full = tiles / cus, rem = tiles % cus;
            return (double)full + (rem ? 0.7 + 0.3 * (double)rem / (double)cus : 0.0);
        };
        if (1.80 * rounds(256) <= rounds(128)) return launch_ring16_cfg<256, 256, 16, 4, 2, 2, 1, 8>(a, stream);
        return launch_ring16_cfg<256, 128, 16, 4, 3, 2, 1, 8>(a, stream);
    }
    const int64_t big_tiles = ((a.rows + 127) / 128) * ((a.columns + 127) / 128);
    if (big_tiles >= 512) return launch_mfma16_cfg<128, 128, 64, 2, 2, 4, 16>(a, stream);
    return launch_mfma16_cfg<64, 64, 64, 2, 2, 4, 16>(a, stream);
}

bool w8a16_ring_usable(const W8A16Args& a) { return ring16_fits(a); }
bool w4a16_ring_usable(const W8A16Args& a) { return w4_ring_ok(a); }

}  // namespace omni
