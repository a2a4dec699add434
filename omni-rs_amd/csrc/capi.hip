// C ABI of libomni_int8: argument checks, the gfx950 gate and kernel dispatch.
// Declarations and contracts: include/omni_int8.h.
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <atomic>
#include <mutex>

#include "../../include/omni_int8.h"
#include "kernels.hpp"

namespace {

thread_local char g_last_error[512] = "";

int fail(int status, const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_last_error, sizeof g_last_error, fmt, ap);
    va_end(ap);
    return status;
}

int hip_status(hipError_t e, const char* what) {
    if (e == hipSuccess) return OMNI_OK;
    return fail(OMNI_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
}

// Per-device cache of the gfx950 probe: -1 unknown, 0 no, 1 yes.
// Replaces the OnceLock<Mutex<HashMap>> of crates/omni-kernel/src/int8_tensorops.rs:26-43.
constexpr int kMaxDevices = 64;
int g_arch[kMaxDevices];
std::once_flag g_arch_once;
std::mutex g_arch_mutex;

int probe_arch(int device) {
    std::call_once(g_arch_once, [] {
        for (int& v : g_arch) v = -1;
    });
    if (device < 0 || device >= kMaxDevices) return 0;
    std::lock_guard<std::mutex> lock(g_arch_mutex);
    if (g_arch[device] < 0) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, device) != hipSuccess) {
            (void)hipGetLastError();
            return 0;  // not cached: a later call may succeed
        }
        g_arch[device] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 ? 1 : 0;
    }
    return g_arch[device];
}

int check_current_device() {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess) {
        (void)hipGetLastError();
        return fail(OMNI_NO_DEVICE, "no HIP device");
    }
    if (!probe_arch(device)) return fail(OMNI_NO_DEVICE, "device %d is not gfx950", device);
    return OMNI_OK;
}

// The scalar lowering is forced by the reference's own switch,
// OMNI_CONVROT_TENSOROPS=0 (matmul2d_lowered, int8_tensorops.rs:15-20, which
// reads it on every call), or by OMNI_INT8_FORCE_SCALAR=1; both are read on
// every call, as the reference does.
bool force_scalar() {
    const char* tensorops = std::getenv("OMNI_CONVROT_TENSOROPS");
    if (tensorops && std::strcmp(tensorops, "0") == 0) return true;
    const char* v = std::getenv("OMNI_INT8_FORCE_SCALAR");
    return v && v[0] == '1';
}

bool aligned(const void* p, size_t a) { return reinterpret_cast<uintptr_t>(p) % a == 0; }

// Tuning knobs (omni::knob): the environment as read once per process, and
// tests' overrides (omni_int8_set_tuning). An override state is 0 (none:
// the environment's value applies), 1 (the knob reads as unset) or 2 (it
// reads as the override value).
constexpr int kKnobs = (int)omni::Knob::Count;
constexpr const char* kKnobNames[kKnobs] = {
    "OMNI_W8A8_TILE",   "OMNI_W8A8_SPLITS",      "OMNI_W8A16_GEMV",  "OMNI_F16_GEMV",
    "OMNI_W8A16_SKINNY", "OMNI_W8A16_SKINNY_SPLIT", "OMNI_W8A16_TILE", "OMNI_W8A16_SPLITS",
    "OMNI_W8A16_ROUTE", "OMNI_W4A16_GEMV",       "OMNI_W4A16_SKINNY_SPLIT", "OMNI_W4A16_SPLITS",
    "OMNI_W4A16_TILE",  "OMNI_F16_TILE"};
std::once_flag g_knob_once;
bool g_knob_env_set[kKnobs];
int g_knob_env[kKnobs];
std::atomic<int> g_knob_state[kKnobs];
std::atomic<int> g_knob_value[kKnobs];

void read_knob_environment() {
    std::call_once(g_knob_once, [] {
        for (int i = 0; i < kKnobs; ++i) {
            const char* v = std::getenv(kKnobNames[i]);
            g_knob_env_set[i] = v != nullptr;
            g_knob_env[i] = v ? std::atoi(v) : 0;
        }
    });
}

// Compute units per device, cached (0: not yet asked).
std::atomic<int> g_cus[kMaxDevices];

// OMNI_W8A16_ROUTE=1 keeps 5..64-row W8A16 and W4A16 calls on the skinny
// kernel, =2 sends them to the tiled MFMA GEMM (test aids, a tuning knob);
// unset, the measured rule below.
int w8a16_route() { return omni::knob(omni::Knob::W8A16Route, 0); }

// 17..64 rows: the skinny kernel streams the weights once per 16 rows, the
// GEMM once per 64 to 256, so the GEMM wins on big matrices (MI355X, W8A16
// 4096 -> 14336: 24.5 against 37.7 us at 24 rows, 27.4 against 70.5 at 64;
// 4096 -> 4096 stays skinny to 48 rows: 15.5 against 16.8). W4A16 over a
// long K (14336 -> 4096) stays skinny to 48 rows (40.3 against 43.4 at 32).
// Those GEMM times are the ring kernels'. Where no ring can run (K % 64 !=
// 0 and the like) the register-staged GEMM takes only more than 48 rows of
// at least 32 M weights (W8A16 K = 4112: 48 x 9000 39.2 us skinny against
// 43.4, 24 x 16000 36.3 against 42.5, 64 x 12000 51.8 against 43.5).
bool midrows_take_gemm(int64_t rows, int64_t columns, int64_t width, bool int4, bool ring_ok) {
    const double elems = (double)columns * (double)width;
    if (!ring_ok) return rows > 48 && elems >= 32e6;
    if (rows > 48 && elems >= 16e6) return true;
    if (int4 && columns < 2 * width) return false;
    return elems >= 32e6;
}

// The W8A16 route: 0 GEMV, 1 skinny MFMA, 2 the GEMM. `a` gives the shape
// (and, for W4A16, the group and scale layout) the ring check reads.
int w8a16_kind(const omni::W8A16Args& a) {
    const int64_t rows = a.rows, columns = a.columns, width = a.width;
    // The GEMV spreads a row over one workgroup of at most 1024 lanes, one
    // 16-element chunk per lane: width <= 16384.
    if (rows <= 4 && width <= 16384) return 0;
    if (rows > 64) return 2;
    // 5..64 rows: the weights are streamed once by a GEMV-shaped MFMA kernel
    // up to 16 rows, and on small matrices beyond.
    const int r = w8a16_route();
    if (r == 1) return 1;
    if (r == 2) return 2;
    return rows > 16 && midrows_take_gemm(rows, columns, width, false, omni::w8a16_ring_usable(a)) ? 2 : 1;
}

// The same for W4A16 (its GEMV takes width <= 32768).
int w4a16_kind(const omni::W8A16Args& a) {
    const int64_t rows = a.rows, columns = a.columns, width = a.width;
    if (rows <= 4 && width <= 32768) return 0;
    if (rows > 64) return 2;
    const int r = w8a16_route();
    if (r == 1) return 1;
    if (r == 2) return 2;
    return rows > 16 && midrows_take_gemm(rows, columns, width, true, omni::w4a16_ring_usable(a)) ? 2 : 1;
}

// The shape fields of W8A16Args (no pointers: the size queries).
omni::W8A16Args shape_args(int64_t rows, int64_t columns, int64_t width, int64_t group = 0) {
    omni::W8A16Args a{};
    a.rows = rows;
    a.columns = columns;
    a.width = width;
    a.group = group;
    return a;
}

size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// A split-K GEMM workspace: int32 partial sums (none: no split).
struct SplitWorkspace {
    int32_t* partial = nullptr;
    int64_t partial_elems = 0;
};

SplitWorkspace split_workspace(void* workspace, size_t bytes) {
    SplitWorkspace w;
    if (!workspace) return w;
    w.partial = static_cast<int32_t*>(workspace);
    w.partial_elems = (int64_t)(bytes / sizeof(int32_t));
    return w;
}

int run_w8a8(const int32_t* x_packed, const float* x_scale, const int32_t* x_sum,
             const int32_t* w_packed, const float* w_scale, const int32_t* w_zero,
             const float* bias, int64_t rows, int64_t columns, int64_t width, void* out,
             int out_dtype, int32_t* acc_dump, int lowering, hipStream_t stream,
             SplitWorkspace split = SplitWorkspace()) {
    omni::W8A8Args a;
    a.x = reinterpret_cast<const uint8_t*>(x_packed);
    a.x_scale = x_scale;
    a.x_sum = x_sum;
    a.w = reinterpret_cast<const uint8_t*>(w_packed);
    a.w_scale = w_scale;
    a.w_zero = w_zero;
    a.bias = bias;
    a.out = out;
    a.acc_dump = acc_dump;
    a.rows = rows;
    a.columns = columns;
    a.width = width;
    a.out_f16 = out_dtype == OMNI_F16;
    a.partial = split.partial;
    a.partial_elems = split.partial_elems;
    int chosen = lowering == OMNI_LOWERING_AUTO ? omni_w8a8_lowering(width) : lowering;
    // The MFMA kernels need 16-byte rows and keep in-tile output offsets in
    // 32 bits (in bytes: 256 * columns * 4 < 2^32).
    if (chosen == OMNI_LOWERING_MFMA &&
        (width % 16 != 0 || !aligned(x_packed, 16) || !aligned(w_packed, 16) ||
         columns >= (int64_t(1) << 22)))
        chosen = OMNI_LOWERING_SCALAR;
    if (chosen == OMNI_LOWERING_MFMA)
        return hip_status(omni::launch_w8a8_mfma(a, stream), "w8a8 mfma launch");
    return hip_status(omni::launch_w8a8_scalar(a, stream), "w8a8 scalar launch");
}

// Shared body of the two fp16 linears once the reference's guard has passed.
int f16_linear(const char* name, const uint16_t* x, const uint16_t* w, int64_t rows,
               int64_t columns, int64_t width, uint16_t* out, void* stream) {
    if (!x || !w || !out) return fail(OMNI_BAD_ARGUMENT, "%s: null pointer", name);
    if (!aligned(x, 16) || !aligned(w, 16))
        return fail(OMNI_BAD_ARGUMENT, "%s: x and w must be 16-byte aligned", name);
    int st = check_current_device();
    if (st != OMNI_OK) return st;
    omni::W8A16Args a;
    a.x = reinterpret_cast<const _Float16*>(x);
    a.w = reinterpret_cast<const int8_t*>(w);
    a.scale = nullptr;
    a.bias = nullptr;
    a.out = reinterpret_cast<_Float16*>(out);
    a.rows = rows;
    a.columns = columns;
    a.width = width;
    hipStream_t s = static_cast<hipStream_t>(stream);
    // The GEMV gives a row to one workgroup of at most 1024 lanes with up to
    // four 8-element chunks each: width <= 32768.
    if (rows <= 4 && width <= 32768) return hip_status(omni::launch_f16_gemv(a, s), "f16 gemv launch");
    if (rows <= 64) return hip_status(omni::launch_f16_skinny(a, s), "f16 skinny launch");
    return hip_status(omni::launch_f16_mfma(a, s), "f16 mfma launch");
}

// OMNI_QWEN_TENSOROPS=0 turns omni_f16_gemm off (NOT_HANDLED), read once per
// process as crates/qwen-image/src/metal_tensorops.rs:165-169 reads it.
bool qwen_tensorops_enabled() {
    static const bool value = [] {
        const char* v = std::getenv("OMNI_QWEN_TENSOROPS");
        return !(v && std::strcmp(v, "0") == 0);
    }();
    return value;
}

// Static device scratch of omni_try_int8_gemm_noalloc: the codes, row scales
// and row sums that omni_try_int8_gemm keeps in its workspace argument. Each
// GPU the library runs on holds one copy for the life of the process; calls
// on one GPU share it, so calls that overlap in time on one GPU (different
// streams, or host threads) race on it. Nothing in it needs clearing: the
// quantiser writes every code, scale and sum it later reads.
constexpr size_t kScratchBytes = OMNI_NOALLOC_SCRATCH_BYTES;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

// Per-device address of `scratch`, looked up once per device with that
// device current. In host code the name `scratch` is a host-side stand-in,
// never a device address; only the looked-up pointer is passed to kernels.
uint8_t* g_scratch_ptr[kMaxDevices];
std::mutex g_scratch_mutex;

int scratch_of_current_device(uint8_t** out) {
    int device = 0;
    if (hipGetDevice(&device) != hipSuccess || device < 0 || device >= kMaxDevices) {
        (void)hipGetLastError();
        return fail(OMNI_NO_DEVICE, "try_int8_gemm_noalloc: no usable current device");
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[device]) {
        void* p = nullptr;
        hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p) {
            (void)hipGetLastError();
            return fail(OMNI_HIP_ERROR, "try_int8_gemm_noalloc: hipGetSymbolAddress(scratch): %s",
                        hipGetErrorString(e));
        }
        g_scratch_ptr[device] = static_cast<uint8_t*>(p);
    }
    *out = g_scratch_ptr[device];
    return OMNI_OK;
}

// Shape guard of try_int8_gemm, crates/omni-kernel/src/int8_matmul.rs:517-521,
// and the argument checks shared by its two entry points.
int try_int8_gemm_checks(const char* name, const void* x, int x_dtype, int64_t rows,
                         int64_t width, const int32_t* w_packed, int64_t w_packed_len,
                         const float* w_scale, int64_t scale_len, const int32_t* w_zero,
                         int64_t zero_len, float* out) {
    const int64_t columns = scale_len;
    if (rows < 0 || width < 0 || columns < 0) return fail(OMNI_BAD_ARGUMENT, "%s: negative size", name);
    if (width % 4 != 0 || w_packed_len != columns * width / 4 || zero_len != columns)
        return fail(OMNI_NOT_HANDLED,
                    "%s: shapes disagree (width=%lld packed=%lld columns=%lld zero=%lld)", name,
                    (long long)width, (long long)w_packed_len, (long long)columns,
                    (long long)zero_len);
    if (x_dtype != OMNI_F32 && x_dtype != OMNI_F16)
        return fail(OMNI_BAD_ARGUMENT, "%s: unknown dtype %d", name, x_dtype);
    if (rows == 0 || columns == 0) return OMNI_OK;
    if (!x || !w_packed || !w_scale || !w_zero || !out)
        return fail(OMNI_BAD_ARGUMENT, "%s: null pointer", name);
    return OMNI_OK;
}

int try_int8_gemm_run(const void* x, int x_dtype, int64_t rows, int64_t width,
                      const int32_t* w_packed, const float* w_scale, int64_t columns,
                      const int32_t* w_zero, float* out, uint8_t* ws, size_t ws_bytes, void* stream);

int w8a8_gemm_checked(const int32_t* x_packed, const float* x_scale, const int32_t* x_sum,
                      const int32_t* w_packed, const float* w_scale, const int32_t* w_zero,
                      const float* bias, int64_t rows, int64_t columns, int64_t width, void* out,
                      int out_dtype, int32_t* acc_dump, int lowering, SplitWorkspace split, void* stream);

// The activation block of the operator workspaces: codes, row scales, row
// sums, each 256-byte aligned; a split-K GEMM workspace follows it.
size_t activation_bytes(int64_t rows, int64_t width) {
    return round_up((size_t)rows * (size_t)width, 256) + round_up((size_t)rows * 4, 256) +
           round_up((size_t)rows * 4, 256);
}

}  // namespace

namespace omni {

int knob(Knob k, int unset) {
    read_knob_environment();
    const int i = (int)k;
    if (i < 0 || i >= kKnobs) return unset;
    switch (g_knob_state[i].load(std::memory_order_acquire)) {
        case 1: return unset;
        case 2: return g_knob_value[i].load(std::memory_order_relaxed);
        default: return g_knob_env_set[i] ? g_knob_env[i] : unset;
    }
}

int num_cus() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        (void)hipGetLastError();
        return 256;
    }
    int n = g_cus[dev].load(std::memory_order_relaxed);
    if (n > 0) return n;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        n = 256;
    }
    g_cus[dev].store(n, std::memory_order_relaxed);  // every thread stores the same value
    return n;
}

}  // namespace omni

extern "C" {

int omni_int8_set_tuning(const char* name, int mode, int value) {
    if (!name) return fail(OMNI_BAD_ARGUMENT, "set_tuning: null name");
    if (mode < 0 || mode > 2) return fail(OMNI_BAD_ARGUMENT, "set_tuning: mode %d", mode);
    read_knob_environment();
    for (int i = 0; i < kKnobs; ++i) {
        if (std::strcmp(name, kKnobNames[i]) != 0) continue;
        g_knob_value[i].store(value, std::memory_order_relaxed);
        g_knob_state[i].store(mode, std::memory_order_release);
        return OMNI_OK;
    }
    return fail(OMNI_BAD_ARGUMENT, "set_tuning: unknown knob %s", name);
}

int omni_int8_arch_supported(int device) { return probe_arch(device); }

int omni_w8a8_lowering(int64_t width) {
    if (force_scalar()) return OMNI_LOWERING_SCALAR;
    return width % 16 == 0 ? OMNI_LOWERING_MFMA : OMNI_LOWERING_SCALAR;
}

const char* omni_int8_last_error(void) { return g_last_error; }

int omni_int8_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t width,
                            int64_t ld_x, int32_t* x_packed, float* x_scale, int32_t* x_sum,
                            void* stream) {
    if (rows < 0 || width < 0 || ld_x < width)
        return fail(OMNI_BAD_ARGUMENT, "quantize_rows: bad sizes rows=%lld width=%lld ld=%lld",
                    (long long)rows, (long long)width, (long long)ld_x);
    if (x_dtype != OMNI_F32 && x_dtype != OMNI_F16)
        return fail(OMNI_BAD_ARGUMENT, "quantize_rows: unknown dtype %d", x_dtype);
    if (width % 4 != 0) return fail(OMNI_NOT_HANDLED, "quantize_rows: width %% 4 != 0");
    if (rows > 0 && (!x || !x_packed || !x_scale))
        return fail(OMNI_BAD_ARGUMENT, "quantize_rows: null pointer");
    if (!aligned(x_packed, 4)) return fail(OMNI_BAD_ARGUMENT, "quantize_rows: x_packed misaligned");
    if (rows > 0x7fffffffLL) return fail(OMNI_BAD_ARGUMENT, "quantize_rows: too many rows");
    int st = check_current_device();
    if (st != OMNI_OK) return st;
    return hip_status(omni::launch_quantize_rows(x, x_dtype == OMNI_F16, rows, width, ld_x,
                                                 reinterpret_cast<uint8_t*>(x_packed), x_scale,
                                                 x_sum, static_cast<hipStream_t>(stream)),
                      "quantize_rows launch");
}

int omni_w8a8_gemm(const int32_t* x_packed, const float* x_scale, const int32_t* x_sum,
                   const int32_t* w_packed, const float* w_scale, const int32_t* w_zero,
                   const float* bias, int64_t rows, int64_t columns, int64_t width, void* out,
                   int out_dtype, int32_t* acc_dump, int lowering, void* stream) {
    return omni_w8a8_gemm_ws(x_packed, x_scale, x_sum, w_packed, w_scale, w_zero, bias, rows, columns, width, out,
                             out_dtype, acc_dump, lowering, nullptr, 0, stream);
}

size_t omni_w8a8_gemm_workspace_size(int64_t rows, int64_t columns, int64_t width) {
    if (rows <= 0 || columns <= 0 || width <= 0 || width % 16 != 0 || width > 131072 ||
        columns >= (int64_t(1) << 22) || omni_w8a8_lowering(width) != OMNI_LOWERING_MFMA)
        return 0;
    return (size_t)omni::w8a8_partial_elems(rows, columns, width) * sizeof(int32_t);
}

int omni_w8a8_gemm_ws(const int32_t* x_packed, const float* x_scale, const int32_t* x_sum,
                      const int32_t* w_packed, const float* w_scale, const int32_t* w_zero,
                      const float* bias, int64_t rows, int64_t columns, int64_t width, void* out,
                      int out_dtype, int32_t* acc_dump, int lowering, void* workspace,
                      size_t workspace_bytes, void* stream) {
    if (workspace_bytes > 0 && (!workspace || !aligned(workspace, 256)))
        return fail(OMNI_BAD_ARGUMENT, "w8a8_gemm: workspace must be 256-byte aligned");
    return w8a8_gemm_checked(x_packed, x_scale, x_sum, w_packed, w_scale, w_zero, bias, rows, columns, width,
                             out, out_dtype, acc_dump, lowering, split_workspace(workspace, workspace_bytes),
                             stream);
}

}  // extern "C"

namespace {

// omni_w8a8_gemm_ws after its workspace check (shared with the operators,
// which carve the split-K workspace out of their own).
int w8a8_gemm_checked(const int32_t* x_packed, const float* x_scale, const int32_t* x_sum,
                      const int32_t* w_packed, const float* w_scale, const int32_t* w_zero,
                      const float* bias, int64_t rows, int64_t columns, int64_t width, void* out,
                      int out_dtype, int32_t* acc_dump, int lowering, SplitWorkspace split, void* stream) {
    if (rows < 0 || columns < 0 || width < 0)
        return fail(OMNI_BAD_ARGUMENT, "w8a8_gemm: negative size");
    if (out_dtype != OMNI_F32 && out_dtype != OMNI_F16)
        return fail(OMNI_BAD_ARGUMENT, "w8a8_gemm: unknown out dtype %d", out_dtype);
    if (lowering < OMNI_LOWERING_AUTO || lowering > OMNI_LOWERING_SCALAR)
        return fail(OMNI_BAD_ARGUMENT, "w8a8_gemm: unknown lowering %d", lowering);
    if (width % 4 != 0) return fail(OMNI_NOT_HANDLED, "w8a8_gemm: width %% 4 != 0");
    if (width > 131072) return fail(OMNI_NOT_HANDLED, "w8a8_gemm: width > 131072 may overflow int32");
    if (rows > 0 && columns > 0 &&
        (!x_packed || !x_scale || !w_packed || !w_scale || !out || (w_zero && !x_sum)))
        return fail(OMNI_BAD_ARGUMENT, "w8a8_gemm: null pointer");
    if (!aligned(x_packed, 4) || !aligned(w_packed, 4))
        return fail(OMNI_BAD_ARGUMENT, "w8a8_gemm: operands must be 4-byte aligned");
    if (((rows + 255) / 256) * ((columns + 127) / 128) > 0x7fffffffLL || rows > 0x7fffffffLL)
        return fail(OMNI_BAD_ARGUMENT, "w8a8_gemm: problem too large");
    int st = check_current_device();
    if (st != OMNI_OK) return st;
    return run_w8a8(x_packed, x_scale, x_sum, w_packed, w_scale, w_zero, bias, rows, columns,
                    width, out, out_dtype, acc_dump, lowering, static_cast<hipStream_t>(stream), split);
}

}  // namespace

extern "C" {

size_t omni_try_int8_gemm_workspace_size(int64_t rows, int64_t width) {
    if (rows < 0 || width < 0) return 0;
    return activation_bytes(rows, width);
}

size_t omni_try_int8_gemm_split_workspace_size(int64_t rows, int64_t columns, int64_t width) {
    if (rows < 0 || width < 0 || columns < 0) return 0;
    return activation_bytes(rows, width) + omni_w8a8_gemm_workspace_size(rows, columns, width);
}

int omni_try_int8_gemm(const void* x, int x_dtype, int64_t rows, int64_t width,
                       const int32_t* w_packed, int64_t w_packed_len, const float* w_scale,
                       int64_t scale_len, const int32_t* w_zero, int64_t zero_len, float* out,
                       void* workspace, size_t workspace_bytes, void* stream) {
    int st = try_int8_gemm_checks("try_int8_gemm", x, x_dtype, rows, width, w_packed, w_packed_len,
                                  w_scale, scale_len, w_zero, zero_len, out);
    if (st != OMNI_OK || rows == 0 || scale_len == 0) return st;
    if (workspace_bytes < omni_try_int8_gemm_workspace_size(rows, width))
        return fail(OMNI_BAD_ARGUMENT, "try_int8_gemm: workspace of %zu bytes, need %zu",
                    workspace_bytes, omni_try_int8_gemm_workspace_size(rows, width));
    if (!workspace) return fail(OMNI_BAD_ARGUMENT, "try_int8_gemm: null pointer");
    if (!aligned(workspace, 256)) return fail(OMNI_BAD_ARGUMENT, "try_int8_gemm: workspace must be 256-byte aligned");
    return try_int8_gemm_run(x, x_dtype, rows, width, w_packed, w_scale, scale_len, w_zero, out,
                             static_cast<uint8_t*>(workspace), workspace_bytes, stream);
}

int omni_try_int8_gemm_noalloc(const void* x, int x_dtype, int64_t rows, int64_t width,
                               const int32_t* w_packed, int64_t w_packed_len, const float* w_scale,
                               int64_t scale_len, const int32_t* w_zero, int64_t zero_len,
                               float* out, void* stream) {
    int st = try_int8_gemm_checks("try_int8_gemm_noalloc", x, x_dtype, rows, width, w_packed,
                                  w_packed_len, w_scale, scale_len, w_zero, zero_len, out);
    if (st != OMNI_OK || rows == 0 || scale_len == 0) return st;
    const size_t need = omni_try_int8_gemm_workspace_size(rows, width);
    if (need > kScratchBytes)
        return fail(OMNI_BAD_ARGUMENT,
                    "try_int8_gemm_noalloc: %lld x %lld activations need %zu bytes of scratch, "
                    "more than the static %zu (use omni_try_int8_gemm with a workspace)",
                    (long long)rows, (long long)width, need, kScratchBytes);
    st = check_current_device();
    if (st != OMNI_OK) return st;
    uint8_t* ws = nullptr;
    st = scratch_of_current_device(&ws);
    if (st != OMNI_OK) return st;
    return try_int8_gemm_run(x, x_dtype, rows, width, w_packed, w_scale, scale_len, w_zero, out,
                             ws, kScratchBytes, stream);
}

int omni_convrot_quantize_rows(const void* x, int x_dtype, int64_t rows, int64_t width,
                               int64_t ld_x, int64_t group, int32_t* x_packed, float* x_scale,
                               int32_t* x_sum, void* stream) {
    if (rows < 0 || width < 0 || ld_x < width)
        return fail(OMNI_BAD_ARGUMENT, "convrot_quantize_rows: bad sizes rows=%lld width=%lld ld=%lld",
                    (long long)rows, (long long)width, (long long)ld_x);
    if (x_dtype != OMNI_F32 && x_dtype != OMNI_F16)
        return fail(OMNI_BAD_ARGUMENT, "convrot_quantize_rows: unknown dtype %d", x_dtype);
    // crates/qwen-image/src/convrot.rs:12 (GROUP = 256) and :39-43 (the width
    // must split into whole groups).
    if (group != 256)
        return fail(OMNI_NOT_HANDLED, "convrot_quantize_rows: group %lld (only 256 is supported)",
                    (long long)group);
    if (width % 256 != 0)
        return fail(OMNI_NOT_HANDLED, "convrot_quantize_rows: width %lld is not a multiple of 256",
                    (long long)width);
    if (rows == 0 || width == 0) return OMNI_OK;
    if (!x || !x_packed || !x_scale)
        return fail(OMNI_BAD_ARGUMENT, "convrot_quantize_rows: null pointer");
    const int64_t elem = x_dtype == OMNI_F16 ? 2 : 4;
    if (!aligned(x, 16) || (ld_x * elem) % 16 != 0)
        return fail(OMNI_BAD_ARGUMENT, "convrot_quantize_rows: x rows must start 16-byte aligned");
    if (!aligned(x_packed, 16)) return fail(OMNI_BAD_ARGUMENT, "convrot_quantize_rows: x_packed must be 16-byte aligned");
    if (rows > 0x7fffffffLL) return fail(OMNI_BAD_ARGUMENT, "convrot_quantize_rows: too many rows");
    int st = check_current_device();
    if (st != OMNI_OK) return st;
    return hip_status(omni::launch_convrot_quantize(x, x_dtype == OMNI_F16, rows, width, ld_x,
                                                    reinterpret_cast<uint8_t*>(x_packed), x_scale,
                                                    x_sum, static_cast<hipStream_t>(stream)),
                      "convrot_quantize_rows launch");
}

int omni_convrot_linear(const void* x, int x_dtype, int64_t rows, int64_t width,
                        const int32_t* w_packed, int64_t w_packed_len, const float* w_scale,
                        int64_t scale_len, const int32_t* w_zero, int64_t zero_len, void* out,
                        int out_dtype, void* workspace, size_t workspace_bytes, void* stream) {
    // Int8Linear::forward (crates/qwen-image/src/convrot.rs:81-92): the width
    // must match the layer (:84 asserts it), the layer's tensors must agree
    // (try_int8_gemm's guard, int8_matmul.rs:517-521), the width must split
    // into groups of 256 (:39-43).
    const int64_t columns = scale_len;
    if (rows < 0 || width < 0 || columns < 0)
        return fail(OMNI_BAD_ARGUMENT, "convrot_linear: negative size");
    if (width % 256 != 0 || w_packed_len != columns * width / 4 || zero_len != columns)
        return fail(OMNI_NOT_HANDLED,
                    "convrot_linear: shapes disagree (width=%lld packed=%lld columns=%lld zero=%lld)",
                    (long long)width, (long long)w_packed_len, (long long)columns, (long long)zero_len);
    if (x_dtype != OMNI_F32 && x_dtype != OMNI_F16)
        return fail(OMNI_BAD_ARGUMENT, "convrot_linear: unknown dtype %d", x_dtype);
    if (out_dtype != OMNI_F32 && out_dtype != OMNI_F16)
        return fail(OMNI_BAD_ARGUMENT, "convrot_linear: unknown out dtype %d", out_dtype);
    if (workspace_bytes < omni_try_int8_gemm_workspace_size(rows, width))
        return fail(OMNI_BAD_ARGUMENT, "convrot_linear: workspace of %zu bytes, need %zu",
                    workspace_bytes, omni_try_int8_gemm_workspace_size(rows, width));
    if (rows == 0 || columns == 0) return OMNI_OK;
    if (!x || !w_packed || !w_scale || !w_zero || !out || !workspace)
        return fail(OMNI_BAD_ARGUMENT, "convrot_linear: null pointer");
    if (!aligned(workspace, 256)) return fail(OMNI_BAD_ARGUMENT, "convrot_linear: workspace must be 256-byte aligned");
    uint8_t* ws = static_cast<uint8_t*>(workspace);
    int32_t* x_packed = reinterpret_cast<int32_t*>(ws);
    float* x_scale = reinterpret_cast<float*>(ws + round_up((size_t)rows * width, 256));
    int32_t* x_sum = reinterpret_cast<int32_t*>(ws + round_up((size_t)rows * width, 256) +
                                                round_up((size_t)rows * 4, 256));
    // Beyond the activation block: the split-K partial sums.
    const size_t act = activation_bytes(rows, width);
    const SplitWorkspace split = split_workspace(ws + act, workspace_bytes - act);
    int st = omni_convrot_quantize_rows(x, x_dtype, rows, width, width, 256, x_packed, x_scale, x_sum, stream);
    if (st != OMNI_OK) return st;
    // The reference casts the f32 result to the model precision after the op
    // (convrot.rs:91); the GEMM's f16 epilogue applies that same one rounding.
    return w8a8_gemm_checked(x_packed, x_scale, x_sum, w_packed, w_scale, w_zero, nullptr, rows, columns,
                             width, out, out_dtype, nullptr, OMNI_LOWERING_AUTO, split, stream);
}

size_t omni_w8a16_gemm_workspace_size(int64_t rows, int64_t columns, int64_t width) {
    if (rows <= 0 || columns <= 0 || width <= 0 || width % 16 != 0) return 0;
    switch (w8a16_kind(shape_args(rows, columns, width))) {
        case 1: return (size_t)omni::w8a16_skinny_partial_elems(rows, columns, width) * sizeof(float);
        case 2: return (size_t)omni::w8a16_partial_elems(rows, columns, width) * sizeof(float);
        default: return 0;
    }
}

int omni_w8a16_gemm(const uint16_t* x, const int8_t* w, const uint16_t* scale,
                    const uint16_t* bias, int64_t rows, int64_t columns, int64_t width,
                    uint16_t* out, void* stream) {
    return omni_w8a16_gemm_ws(x, w, scale, bias, rows, columns, width, out, nullptr, 0, stream);
}

int omni_w8a16_gemm_ws(const uint16_t* x, const int8_t* w, const uint16_t* scale,
                       const uint16_t* bias, int64_t rows, int64_t columns, int64_t width,
                       uint16_t* out, void* workspace, size_t workspace_bytes, void* stream) {
    if (rows < 0 || columns < 0 || width < 0)
        return fail(OMNI_BAD_ARGUMENT, "w8a16_gemm: negative size");
    if (width % 16 != 0) return fail(OMNI_NOT_HANDLED, "w8a16_gemm: width %% 16 != 0");
    if (rows == 0 || columns == 0) return OMNI_OK;
    if (!x || !w || !scale || !out) return fail(OMNI_BAD_ARGUMENT, "w8a16_gemm: null pointer");
    if (!aligned(x, 16) || !aligned(w, 16))
        return fail(OMNI_BAD_ARGUMENT, "w8a16_gemm: x and w must be 16-byte aligned");
    if (workspace_bytes > 0 && (!workspace || !aligned(workspace, 256)))
        return fail(OMNI_BAD_ARGUMENT, "w8a16_gemm: workspace must be 256-byte aligned");
    if (((rows + 63) / 64) * ((columns + 63) / 64) > 0x7fffffffLL)
        return fail(OMNI_BAD_ARGUMENT, "w8a16_gemm: problem too large");
    int st = check_current_device();
    if (st != OMNI_OK) return st;
    omni::W8A16Args a;
    a.x = reinterpret_cast<const _Float16*>(x);
    a.w = w;
    a.scale = reinterpret_cast<const _Float16*>(scale);
    a.bias = reinterpret_cast<const _Float16*>(bias);
    a.out = reinterpret_cast<_Float16*>(out);
    a.rows = rows;
    a.columns = columns;
    a.width = width;
    a.partial = static_cast<float*>(workspace);
    a.partial_elems = (int64_t)(workspace_bytes / sizeof(float));
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (w8a16_kind(a)) {
        case 0: return hip_status(omni::launch_w8a16_gemv(a, s), "w8a16 gemv launch");
        case 1: return hip_status(omni::launch_w8a16_skinny(a, s), "w8a16 skinny launch");
        default: return hip_status(omni::launch_w8a16_mfma(a, s), "w8a16 mfma launch");
    }
}

size_t omni_w4a16_gemm_workspace_size(int64_t rows, int64_t columns, int64_t width, int64_t group) {
    if (rows <= 0 || columns <= 0 || width <= 0 || group <= 0 || width % 32 != 0 || group % 32 != 0 ||
        width % group != 0)
        return 0;
    switch (w4a16_kind(shape_args(rows, columns, width, group))) {
        case 1: return (size_t)omni::w4a16_skinny_partial_elems(rows, columns, width) * sizeof(float);
        case 2: return (size_t)omni::w4a16_partial_elems(rows, columns, width, group) * sizeof(float);
        default: return 0;
    }
}

int omni_w4a16_gemm(const uint16_t* x, const uint8_t* w_packed, const uint16_t* scale_bf16,
                    int64_t group, const uint16_t* bias, int64_t rows, int64_t columns,
                    int64_t width, uint16_t* out, void* stream) {
    return omni_w4a16_gemm_ws(x, w_packed, scale_bf16, group, bias, rows, columns, width, out, nullptr, 0,
                              stream);
}

int omni_w4a16_gemm_ws(const uint16_t* x, const uint8_t* w_packed, const uint16_t* scale_bf16,
                       int64_t group, const uint16_t* bias, int64_t rows, int64_t columns,
                       int64_t width, uint16_t* out, void* workspace, size_t workspace_bytes,
                       void* stream) {
    if (rows < 0 || columns < 0 || width < 0 || group <= 0)
        return fail(OMNI_BAD_ARGUMENT, "w4a16_gemm: bad sizes");
    // 32 values (16 bytes) per GEMV lane, and a lane's values in one group.
    if (width % 32 != 0 || group % 32 != 0 || width % group != 0)
        return fail(OMNI_NOT_HANDLED, "w4a16_gemm: width %lld / group %lld (need width %% group == 0, group %% 32 == 0)",
                    (long long)width, (long long)group);
    if (rows == 0 || columns == 0) return OMNI_OK;
    if (!x || !w_packed || !scale_bf16 || !out) return fail(OMNI_BAD_ARGUMENT, "w4a16_gemm: null pointer");
    if (!aligned(x, 16) || !aligned(w_packed, 16))
        return fail(OMNI_BAD_ARGUMENT, "w4a16_gemm: x and w_packed must be 16-byte aligned");
    if (workspace_bytes > 0 && (!workspace || !aligned(workspace, 256)))
        return fail(OMNI_BAD_ARGUMENT, "w4a16_gemm: workspace must be 256-byte aligned");
    if (((rows + 63) / 64) * ((columns + 63) / 64) > 0x7fffffffLL)
        return fail(OMNI_BAD_ARGUMENT, "w4a16_gemm: problem too large");
    int st = check_current_device();
    if (st != OMNI_OK) return st;
    omni::W8A16Args a;
    a.x = reinterpret_cast<const _Float16*>(x);
    a.w = reinterpret_cast<const int8_t*>(w_packed);
    a.scale = nullptr;
    a.bias = reinterpret_cast<const _Float16*>(bias);
    a.out = reinterpret_cast<_Float16*>(out);
    a.rows = rows;
    a.columns = columns;
    a.width = width;
    a.gscale = scale_bf16;
    a.group = group;
    a.partial = static_cast<float*>(workspace);
    a.partial_elems = (int64_t)(workspace_bytes / sizeof(float));
    hipStream_t s = static_cast<hipStream_t>(stream);
    switch (w4a16_kind(a)) {
        case 0: return hip_status(omni::launch_w4a16_gemv(a, s), "w4a16 gemv launch");
        case 1: return hip_status(omni::launch_w4a16_skinny(a, s), "w4a16 skinny launch");
        default: return hip_status(omni::launch_w4a16_mfma(a, s), "w4a16 mfma launch");
    }
}

int omni_f16_gemv(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t columns,
                  int64_t width, uint16_t* out, void* stream) {
    // crates/breeze-tts/src/metal_depth.rs:94-104
    if (rows < 1 || rows > 64 || width <= 0 || width % 32 != 0 || columns <= 0 || columns > 4096)
        return fail(OMNI_NOT_HANDLED, "f16_gemv: rows %lld, width %lld, columns %lld outside 1..=64, "
                    "width %% 32 == 0, 1..=4096", (long long)rows, (long long)width, (long long)columns);
    return f16_linear("f16_gemv", x, w, rows, columns, width, out, stream);
}

int omni_f16_gemm(const uint16_t* x, const uint16_t* w, int64_t rows, int64_t columns,
                  int64_t width, uint16_t* out, void* stream) {
    if (!qwen_tensorops_enabled()) return fail(OMNI_NOT_HANDLED, "f16_gemm: OMNI_QWEN_TENSOROPS=0");
    // crates/qwen-image/src/metal_tensorops.rs:174-187
    if (rows < 256 || rows > 65535 || width % 64 != 0 || columns % 64 != 0 || width < 4096 ||
        columns < 4096 || width > 12288 || columns > 12288)
        return fail(OMNI_NOT_HANDLED, "f16_gemm: rows %lld, width %lld, columns %lld outside 256..=65535, "
                    "4096..=12288 in steps of 64", (long long)rows, (long long)width, (long long)columns);
    return f16_linear("f16_gemm", x, w, rows, columns, width, out, stream);
}

}  // extern "C"

namespace {

// Quantise x into the workspace (codes, then row scales, then row sums, each
// 256-byte aligned), then the GEMM with the reference's f32 epilogue. What
// the workspace holds beyond that block is the GEMM's split-K partial sums.
int try_int8_gemm_run(const void* x, int x_dtype, int64_t rows, int64_t width,
                      const int32_t* w_packed, const float* w_scale, int64_t columns,
                      const int32_t* w_zero, float* out, uint8_t* ws, size_t ws_bytes, void* stream) {
    int32_t* x_packed = reinterpret_cast<int32_t*>(ws);
    float* x_scale = reinterpret_cast<float*>(ws + round_up((size_t)rows * width, 256));
    int32_t* x_sum = reinterpret_cast<int32_t*>(ws + round_up((size_t)rows * width, 256) +
                                                round_up((size_t)rows * 4, 256));
    const size_t act = activation_bytes(rows, width);
    const SplitWorkspace split = split_workspace(ws + act, ws_bytes - act);
    int st = omni_int8_quantize_rows(x, x_dtype, rows, width, width, x_packed, x_scale, x_sum, stream);
    if (st != OMNI_OK) return st;
    return w8a8_gemm_checked(x_packed, x_scale, x_sum, w_packed, w_scale, w_zero, nullptr, rows, columns,
                             width, out, OMNI_F32, nullptr, OMNI_LOWERING_AUTO, split, stream);
}

}  // namespace
