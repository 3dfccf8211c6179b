// Library-wide pieces of the C ABI: version, error text, row sizes.
#include <atomic>
#include <climits>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <vector>

#include "miq_internal.h"

namespace miq {

static thread_local char g_err[512] = "";

void set_error(const char *fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof(g_err), fmt, ap);
    va_end(ap);
}

int check_launch(const char *what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error("%s: %s", what, hipGetErrorString(e));
        return MIQ_EHIP;
    }
    return MIQ_OK;
}

// Library-held device buffers.
//
// Split-K scratch, one per device: partial tiles plus the arrival counters
// that let the last workgroup of a tile reduce them; and workspace slots (the
// prefill's converted activation and partials, the u4 K-part sums).  Grown on
// demand by a call outside stream capture (the reference's per-queue GEMM
// workspace grows the same way); a call made while its stream captures a graph
// never allocates: if the buffers an earlier call left are too small it
// returns MIQ_UNSUPPORTED, so a caller warms each shape up once before
// capturing it.  A buffer that growth replaces is retired, never freed before
// the process ends: graphs captured earlier and work still queued keep
// pointing at it.  The counters are zeroed once at allocation and every kernel
// that uses them leaves them at zero.  Launches that share a device share this
// memory: calls that use it must not overlap on one device (one stream per
// device, as the reference serialises engine execution).
namespace {
struct Scratch {
    float *part = nullptr;
    size_t part_bytes = 0;
    uint32_t *cnt = nullptr;
    size_t n_cnt = 0;
};
constexpr int kMaxDevices = 64;
Scratch g_scr[kMaxDevices];
std::mutex g_scr_mu;
// buffers replaced by growth (held under g_scr_mu; never freed)
std::vector<void *> g_retired;

int current_device(int *dev) {
    if (hipGetDevice(dev) != hipSuccess || *dev < 0 || *dev >= kMaxDevices) {
        set_error("miq: no current device");
        return MIQ_EHIP;
    }
    return MIQ_OK;
}

// Growth is refused while the stream captures (hipMalloc/hipFree/hipMemset
// would break or invalidate the capture); an unanswerable query counts as
// capturing.
int may_grow(hipStream_t stream, const char *what, size_t have, size_t want) {
    hipStreamCaptureStatus st = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(stream, &st) != hipSuccess) {
        (void)hipGetLastError();
        st = hipStreamCaptureStatusActive;
    }
    if (st == hipStreamCaptureStatusNone) return MIQ_OK;
    set_error("%s: needs %zu bytes (has %zu) while the stream captures a graph; run the same call once before "
              "capturing it", what, want, have);
    return MIQ_UNSUPPORTED;
}
}  // namespace

// ---- the no-allocation entry point's scratch (miq_i8_gemm_noalloc)
//
// A file-scope device array, one copy per GPU for the life of the process:
// partial tiles first, the arrival counters at the end.  Host code never
// passes `scratch` itself (on the host it names a stand-in, not device
// memory): each device's address comes from hipGetSymbolAddress, taken once
// with that device current.  The counters start at zero (a fill kernel at
// set-up) and every kernel that uses them leaves them at zero; the partials
// keep the last call's contents.  Calls that overlap on one device race.
constexpr size_t kStaticPartBytes = (size_t)16 << 20;
constexpr size_t kStaticCnt = (size_t)64 << 10;
static __device__ __align__(256) uint8_t scratch[kStaticPartBytes + kStaticCnt * sizeof(uint32_t)];

namespace {
uint8_t *g_static_ptr[kMaxDevices];
std::mutex g_static_mu;
thread_local bool g_static_mode = false;  // set for the duration of a miq_i8_gemm_noalloc call

__global__ __launch_bounds__(256) void zero_u32_kernel(uint32_t *p, size_t n) {
    for (size_t i = blockIdx.x * 256 + threadIdx.x; i < n; i += (size_t)gridDim.x * 256) p[i] = 0;
}

struct StaticMode {
    StaticMode() { g_static_mode = true; }
    ~StaticMode() { g_static_mode = false; }
};
}  // namespace

static int static_scratch_get(hipStream_t stream, size_t part_bytes, size_t n_cnt, float **part, uint32_t **cnt) {
    if (part_bytes > kStaticPartBytes || n_cnt > kStaticCnt) {
        set_error("miq_i8_gemm_noalloc: the shape needs %zu bytes of partials and %zu counters, beyond the static "
                  "scratch (%zu bytes, %zu counters)", part_bytes, n_cnt, kStaticPartBytes, kStaticCnt);
        return MIQ_UNSUPPORTED;
    }
    int dev = 0;
    if (current_device(&dev) != MIQ_OK) return MIQ_EHIP;
    std::lock_guard<std::mutex> lk(g_static_mu);
    if (!g_static_ptr[dev]) {  // set-up, once per device, with the device current
        uint8_t *p = nullptr;
        if (hipGetSymbolAddress((void **)&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) {
            (void)hipGetLastError();
            set_error("miq_i8_gemm_noalloc: hipGetSymbolAddress of the static scratch failed");
            return MIQ_EHIP;
        }
        // Until this point no call has used the array on this device, so it still
        // holds its load-time contents: a __device__ array without initialiser is
        // zero-initialised when the code object loads.  The clear below restates
        // that on a stream outside capture; under capture it is skipped rather than
        // recorded (it would rerun on every replay) and the load-time zeros serve.
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        if (hipStreamIsCapturing(stream, &cs) != hipSuccess) {
            (void)hipGetLastError();
            cs = hipStreamCaptureStatusActive;
        }
        if (cs == hipStreamCaptureStatusNone) {
            hipLaunchKernelGGL(zero_u32_kernel, dim3(64), dim3(256), 0, stream,
                               reinterpret_cast<uint32_t *>(p + kStaticPartBytes), kStaticCnt);
            if (check_launch("miq_i8_gemm_noalloc: clearing the static counters") != MIQ_OK) return MIQ_EHIP;
        }
        g_static_ptr[dev] = p;
    }
    *part = reinterpret_cast<float *>(g_static_ptr[dev]);
    *cnt = reinterpret_cast<uint32_t *>(g_static_ptr[dev] + kStaticPartBytes);
    return MIQ_OK;
}

int scratch_get(hipStream_t stream, size_t part_bytes, size_t n_cnt, float **part, uint32_t **cnt) {
    if (g_static_mode) return static_scratch_get(stream, part_bytes, n_cnt, part, cnt);
    int dev = 0;
    if (current_device(&dev) != MIQ_OK) return MIQ_EHIP;
    std::lock_guard<std::mutex> lk(g_scr_mu);
    Scratch &s = g_scr[dev];
    if (s.part_bytes < part_bytes) {
        if (const int rc = may_grow(stream, "split-K scratch", s.part_bytes, part_bytes)) return rc;
        const size_t want = part_bytes + part_bytes / 2;
        float *np = nullptr;
        if (hipMalloc(&np, want) != hipSuccess) {
            set_error("split-K scratch: hipMalloc(%zu) failed", want);
            return MIQ_EHIP;
        }
        if (s.part) g_retired.push_back(s.part);
        s.part = np;
        s.part_bytes = want;
    }
    if (s.n_cnt < n_cnt) {
        if (const int rc = may_grow(stream, "split-K counters", s.n_cnt * 4, n_cnt * 4)) return rc;
        const size_t want = n_cnt + n_cnt / 2 + 64;
        uint32_t *nc = nullptr;
        if (hipMalloc(&nc, want * sizeof(uint32_t)) != hipSuccess) {
            set_error("split-K scratch: counter allocation failed");
            return MIQ_EHIP;
        }
        // cleared on the caller's stream, so the clear is ordered before the
        // kernel that reads the counters whatever kind of stream it is
        hipLaunchKernelGGL(zero_u32_kernel, dim3(64), dim3(256), 0, stream, nc, want);
        if (check_launch("split-K scratch: clearing the counters") != MIQ_OK) return MIQ_EHIP;
        if (s.cnt) g_retired.push_back(s.cnt);
        s.cnt = nc;
        s.n_cnt = want;
    }
    *part = s.part;
    *cnt = s.cnt;
    return MIQ_OK;
}

namespace {
struct Ws {
    void *p = nullptr;
    size_t bytes = 0;
};
Ws g_ws[kMaxDevices][kWsSlots];
}  // namespace

int workspace_get(hipStream_t stream, int slot, size_t bytes, void **ptr, bool zero) {
    if (g_static_mode) {
        set_error("miq_i8_gemm_noalloc: this shape runs a kernel that needs a workspace (the prefill GEMM at 48 "
                  "tokens or more); only the decode kernels fit the static scratch");
        return MIQ_UNSUPPORTED;
    }
    int dev = 0;
    if (slot < 0 || slot >= kWsSlots || current_device(&dev) != MIQ_OK) {
        set_error("workspace: no current device or bad slot");
        return MIQ_EHIP;
    }
    std::lock_guard<std::mutex> lk(g_scr_mu);
    Ws &w = g_ws[dev][slot];
    if (w.bytes < bytes) {
        if (const int rc = may_grow(stream, "workspace", w.bytes, bytes)) return rc;
        const size_t want = (bytes + bytes / 4 + 3) & ~(size_t)3;
        void *np = nullptr;
        if (hipMalloc(&np, want) != hipSuccess) {
            set_error("workspace: hipMalloc(%zu) failed", want);
            return MIQ_EHIP;
        }
        if (zero) {  // on the caller's stream, ahead of the kernel that reads it
            hipLaunchKernelGGL(zero_u32_kernel, dim3(64), dim3(256), 0, stream, reinterpret_cast<uint32_t *>(np), want / 4);
            if (check_launch("workspace: clearing") != MIQ_OK) return MIQ_EHIP;
        }
        if (w.p) g_retired.push_back(w.p);
        w.p = np;
        w.bytes = want;
    }
    *ptr = w.p;
    return MIQ_OK;
}

namespace {
struct SwitchDef {
    const char *name;
    int dflt;
};
// names (the environment variable is MIQ_<name>) and defaults, in Switch order
constexpr SwitchDef kSwitches[kSwCount] = {
    {"M32_MIN_TB", 48}, {"GEMV_MAX_TB", 3}, {"PREFILL_FP16", 1}, {"FUSED_QUANT", 1},
    {"M16_WAVES", 0},   {"M16_FORM", 0},    {"MOE_GRP", 1},      {"M32_FILL", 1}};
std::atomic<int> g_sw[kSwCount];
std::once_flag g_sw_once;

int switch_env(int i) {
    char name[64];
    snprintf(name, sizeof(name), "MIQ_%s", kSwitches[i].name);
    const char *v = getenv(name);
    return v ? atoi(v) : kSwitches[i].dflt;
}
void switches_init() {
    for (int i = 0; i < kSwCount; i++) g_sw[i].store(switch_env(i), std::memory_order_relaxed);
}
}  // namespace

int sw(Switch s) {
    std::call_once(g_sw_once, switches_init);
    return g_sw[s].load(std::memory_order_relaxed);
}

int device_cus(int *n) {
    static int cus[kMaxDevices] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error("miq: no current device");
        return MIQ_EHIP;
    }
    if (!cus[dev] && hipDeviceGetAttribute(&cus[dev], hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) {
        set_error("miq: cannot query the CU count");
        return MIQ_EHIP;
    }
    *n = cus[dev];
    return MIQ_OK;
}

}  // namespace miq

extern "C" {

const char *miq_version(void) { return "miq 0.1 (gfx950)"; }

int miq_i8_gemm_noalloc(hipStream_t stream, const miq_seg *seg, int TB) {
    miq::StaticMode scope;
    return miq::run_gemm(stream, seg, TB, "miq_i8_gemm_noalloc");
}

const char *miq_last_error(void) { return miq::g_err; }

int miq_set_switch(const char *name, int value) {
    std::call_once(miq::g_sw_once, miq::switches_init);
    for (int i = 0; i < miq::kSwCount; i++) {
        if (name && !strcmp(name, miq::kSwitches[i].name)) {
            miq::g_sw[i].store(value == INT_MIN ? miq::switch_env(i) : value, std::memory_order_relaxed);
            return MIQ_OK;
        }
    }
    miq::set_error("miq_set_switch: unknown switch '%s'", name ? name : "(null)");
    return MIQ_EINVAL;
}

size_t miq_row_bytes(uint32_t type, int K) {
    const int vb = miq::block_values(type);
    if (miq::block_bytes(type) == 0 || K <= 0 || K % vb) return 0;
    return (size_t)(K / vb) * miq::block_bytes(type);
}

}  // extern "C"
