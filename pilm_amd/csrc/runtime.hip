// Library lifecycle, device registry, ISA report, stream selection, error
// reporting and buffer validation for the HIP libecpu.
//
// Mirrors src/ecpu/src/core/ecpu.c:1-81 (init/shutdown/version/last_error),
// src/ecpu/src/device/edevice_registry.c:1-51 (vtable registry),
// src/ecpu/src/device/ecpu_device.c:33-88 (host device) and
// src/ecpu/src/dispatch/isa_detect.c:12-40 (ISA report); the CUDA slot of
// src/ecpu/src/device/cuda_device.c:5-29 stays a reserved stub, and a HIP
// device is added whose memory is HBM.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <utility>
#include <vector>

#include <sys/sysinfo.h>

#include "internal.h"

namespace pilm {

static char g_err[512];
static std::mutex g_err_mu;

int fail(int rc, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    std::lock_guard<std::mutex> lk(g_err_mu);
    memcpy(g_err, buf, sizeof(g_err));
    return rc;
}

static hipStream_t g_stream = nullptr;

hipStream_t current_stream() { return g_stream; }

int check_device_buffer(const void *ptr, size_t bytes, const char *what, const char *fn) {
    if (!ptr) return fail(ECPU_ERR_PARAM, "%s: %s is NULL", fn, what);
    hipPointerAttribute_t attr;
    hipError_t e = hipPointerGetAttributes(&attr, ptr);
    if (e != hipSuccess || attr.type != hipMemoryTypeDevice) {
        (void)hipGetLastError();
        return fail(ECPU_ERR_PARAM, "%s: %s (%p) is not device memory; this library runs on the GPU "
                    "and takes HBM pointers only", fn, what, ptr);
    }
    if (bytes == 0) return ECPU_OK;
    hipDeviceptr_t base = nullptr;
    size_t size = 0;
    e = hipMemGetAddressRange(&base, &size, (hipDeviceptr_t)ptr);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(ECPU_ERR_PARAM, "%s: cannot resolve the allocation holding %s (%p): %s", fn, what,
                    ptr, hipGetErrorString(e));
    }
    const uintptr_t lo = (uintptr_t)base, p = (uintptr_t)ptr;
    if (p < lo || p - lo + bytes > size) {
        return fail(ECPU_ERR_PARAM, "%s: %s (%p) needs %zu bytes but its allocation ends %zu bytes "
                    "after it", fn, what, ptr, bytes, (size_t)(lo + size - p));
    }
    return ECPU_OK;
}

int check_launch(const char *fn) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(ECPU_ERR_DEVICE, "%s: kernel launch failed: %s", fn, hipGetErrorString(e));
    return ECPU_OK;
}

// ---- split-K scratch, one set per device ----------------------------------
// Shared by every stream of the device: two split-path calls that overlap in
// time on one GPU (different streams) would race on it.  A graph captured on
// any stream can use it as long as the set was sized before the capture.
struct Scratch {
    int dev;
    float *P;
    size_t nP;
    int *T;
    size_t nT;
    void *X;       // converted activations of the matrix-core path
    size_t nX;
    void *Y;       // intermediates of the fused entry points
    size_t nY;
};
static std::vector<Scratch> g_scratch;
static std::vector<std::pair<int, void *>> g_retired;
static std::mutex g_scratch_mu;

static void *dev_alloc(size_t bytes) {
    void *p = nullptr;
    if (hipMalloc(&p, bytes) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}

int split_scratch(hipStream_t stream, size_t nfloat, size_t nticket, float **P, int **T, const char *fn) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(ECPU_ERR_DEVICE, "%s: no current HIP device", fn);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    Scratch *sc = nullptr;
    (void)stream;
    for (auto &e : g_scratch)
        if (e.dev == dev) sc = &e;
    if (!sc) {
        g_scratch.push_back(Scratch{dev, nullptr, 0, nullptr, 0, nullptr, 0, nullptr, 0});
        sc = &g_scratch.back();
    }
    if (sc->nP < nfloat) {
        const size_t want = std::max<size_t>(nfloat, 1u << 18);
        float *p = (float *)dev_alloc(want * sizeof(float));
        if (!p) return fail(ECPU_ERR_MEM, "%s: hipMalloc of %zu bytes of split-K scratch failed", fn, want * 4);
        if (sc->P) g_retired.push_back({dev, sc->P});
        sc->P = p;
        sc->nP = want;
    }
    if (sc->nT < nticket) {
        const size_t want = std::max<size_t>(nticket, 4096);
        int *t = (int *)dev_alloc(want * sizeof(int));
        if (!t) return fail(ECPU_ERR_MEM, "%s: hipMalloc of split-K tickets failed", fn);
        if (hipMemset(t, 0, want * sizeof(int)) != hipSuccess) {
            (void)hipGetLastError();
            (void)hipFree(t);
            return fail(ECPU_ERR_DEVICE, "%s: clearing split-K tickets failed", fn);
        }
        if (sc->T) g_retired.push_back({dev, sc->T});
        sc->T = t;
        sc->nT = want;
    }
    *P = sc->P;
    *T = sc->T;
    return ECPU_OK;
}

int act_scratch(size_t bytes, void **X, const char *fn) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(ECPU_ERR_DEVICE, "%s: no current HIP device", fn);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    Scratch *sc = nullptr;
    for (auto &e : g_scratch)
        if (e.dev == dev) sc = &e;
    if (!sc) {
        g_scratch.push_back(Scratch{dev, nullptr, 0, nullptr, 0, nullptr, 0, nullptr, 0});
        sc = &g_scratch.back();
    }
    if (sc->nX < bytes) {
        const size_t want = std::max<size_t>(bytes, 1u << 20);
        void *p = dev_alloc(want);
        if (!p) return fail(ECPU_ERR_MEM, "%s: hipMalloc of %zu bytes of activation scratch failed", fn, want);
        if (sc->X) g_retired.push_back({dev, sc->X});
        sc->X = p;
        sc->nX = want;
    }
    *X = sc->X;
    return ECPU_OK;
}

int aux_scratch(size_t bytes, void **Y, const char *fn) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return fail(ECPU_ERR_DEVICE, "%s: no current HIP device", fn);
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    Scratch *sc = nullptr;
    for (auto &e : g_scratch)
        if (e.dev == dev) sc = &e;
    if (!sc) {
        g_scratch.push_back(Scratch{dev, nullptr, 0, nullptr, 0, nullptr, 0, nullptr, 0});
        sc = &g_scratch.back();
    }
    if (sc->nY < bytes) {
        const size_t want = std::max<size_t>(bytes, 1u << 20);
        void *p = dev_alloc(want);
        if (!p) return fail(ECPU_ERR_MEM, "%s: hipMalloc of %zu bytes of fused-op scratch failed", fn, want);
        if (sc->Y) g_retired.push_back({dev, sc->Y});
        sc->Y = p;
        sc->nY = want;
    }
    *Y = sc->Y;
    return ECPU_OK;
}

bool is_device_pointer(const void *p) {
    if (!p) return false;
    hipPointerAttribute_t attr;
    const hipError_t e = hipPointerGetAttributes(&attr, p);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return false;
    }
    return attr.type == hipMemoryTypeDevice;
}

static void free_scratch() {
    std::lock_guard<std::mutex> lk(g_scratch_mu);
    int cur = 0;
    (void)hipGetDevice(&cur);
    auto release = [](int dev, void *p) {
        (void)hipSetDevice(dev);
        (void)hipDeviceSynchronize();
        (void)hipFree(p);
    };
    for (auto &r : g_retired) release(r.first, r.second);
    for (auto &e : g_scratch) {
        if (e.P) release(e.dev, e.P);
        if (e.T) release(e.dev, e.T);
        if (e.X) release(e.dev, e.X);
        if (e.Y) release(e.dev, e.Y);
    }
    g_retired.clear();
    g_scratch.clear();
    (void)hipSetDevice(cur);
}

}  // namespace pilm

using namespace pilm;

// ============================================================ device vtables

static void *host_alloc(size_t bytes, size_t alignment) {
    if (alignment < sizeof(void *)) alignment = sizeof(void *);
    void *p = nullptr;
    return posix_memalign(&p, alignment, bytes) == 0 ? p : nullptr;
}
static void host_free(void *p) { free(p); }
static void host_copy(void *d, const void *s, size_t n) { memcpy(d, s, n); }
static int host_sync(void) { return 0; }
static size_t host_mem_total(void) {
    struct sysinfo si;
    return sysinfo(&si) == 0 ? (size_t)si.totalram * si.mem_unit : 0;
}
static size_t host_mem_free(void) {
    struct sysinfo si;
    return sysinfo(&si) == 0 ? (size_t)si.freeram * si.mem_unit : 0;
}
static int host_init(void) { return 0; }
static int host_shutdown(void) { return 0; }

static int cuda_init(void) { return -1; }   // reserved slot, never available
static int cuda_shutdown(void) { return 0; }

// HBM allocations are 256-byte aligned by hipMalloc, which covers the
// alignment any caller of the vtable asks for in practice (the reference
// asks for 64, eram.c:27).
static void *hip_alloc(size_t bytes, size_t alignment) {
    (void)alignment;
    void *p = nullptr;
    if (hipMalloc(&p, bytes ? bytes : 1) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return p;
}
static void hip_free_(void *p) { (void)hipFree(p); }
static void hip_h2d(void *d, const void *s, size_t n) { (void)hipMemcpy(d, s, n, hipMemcpyHostToDevice); }
static void hip_d2h(void *d, const void *s, size_t n) { (void)hipMemcpy(d, s, n, hipMemcpyDeviceToHost); }
static void hip_d2d(void *d, const void *s, size_t n) { (void)hipMemcpy(d, s, n, hipMemcpyDeviceToDevice); }
static int hip_sync(void) { return hipDeviceSynchronize() == hipSuccess ? 0 : -1; }
static size_t hip_mem_total(void) {
    size_t f = 0, t = 0;
    return hipMemGetInfo(&f, &t) == hipSuccess ? t : 0;
}
static size_t hip_mem_free(void) {
    size_t f = 0, t = 0;
    return hipMemGetInfo(&f, &t) == hipSuccess ? f : 0;
}
static int hip_init(void) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n <= 0) {
        (void)hipGetLastError();
        return -1;
    }
    return hipFree(nullptr) == hipSuccess ? 0 : -1;   // creates the context
}
static int hip_shutdown(void) { return 0; }

static const edevice_vtable_t HOST_VT = {
    "ecpu", EDEV_ECPU, EDEV_CAP_BF16, host_alloc, host_free, host_copy, host_copy, host_copy,
    host_sync, host_mem_total, host_mem_free, host_init, host_shutdown};
static const edevice_vtable_t CUDA_VT = {
    "cuda (reserved)", EDEV_CUDA, EDEV_CAP_NONE, nullptr, nullptr, nullptr, nullptr, nullptr,
    nullptr, nullptr, nullptr, cuda_init, cuda_shutdown};
static const edevice_vtable_t HIP_VT = {
    "hip (gfx950)", EDEV_HIP, EDEV_CAP_F16 | EDEV_CAP_BF16 | EDEV_CAP_FP8 | EDEV_CAP_MFMA,
    hip_alloc, hip_free_, hip_h2d, hip_d2h, hip_d2d, hip_sync, hip_mem_total, hip_mem_free,
    hip_init, hip_shutdown};

static edevice_vtable_t g_registry[EDEV_COUNT];
static int g_inited[EDEV_COUNT];
static edevice_t g_active = EDEV_HIP;
static int g_registered = 0;

static void register_all() {
    if (g_registered) return;
    g_registry[EDEV_ECPU] = HOST_VT;
    g_registry[EDEV_CUDA] = CUDA_VT;
    g_registry[EDEV_HIP] = HIP_VT;
    g_registered = 1;
}

extern "C" {

const edevice_vtable_t *edevice_get(edevice_t dev) {
    register_all();
    if ((int)dev < 0 || dev >= EDEV_COUNT) return nullptr;
    return g_registry[dev].name ? &g_registry[dev] : nullptr;
}

int edevice_register(edevice_t dev, const edevice_vtable_t *vt) {
    register_all();
    if ((int)dev < 0 || dev >= EDEV_COUNT || !vt) return -1;
    g_registry[dev] = *vt;
    return 0;
}

int edevice_set_active(edevice_t dev) {
    register_all();
    if ((int)dev < 0 || dev >= EDEV_COUNT || !g_registry[dev].name) return -1;
    g_active = dev;
    return 0;
}

const edevice_vtable_t *edevice_active(void) {
    register_all();
    return g_registry[g_active].name ? &g_registry[g_active] : nullptr;
}

int edevice_init_all(void) {
    register_all();
    int any = 0;
    for (int i = 0; i < EDEV_COUNT; i++) {
        if (g_registry[i].name && g_registry[i].init && !g_inited[i] && g_registry[i].init() == 0) {
            g_inited[i] = 1;
            any = 1;
        }
        if (g_inited[i]) any = 1;
    }
    return any ? 0 : -1;
}

void edevice_shutdown_all(void) {
    for (int i = 0; i < EDEV_COUNT; i++) {
        if (g_inited[i] && g_registry[i].shutdown) g_registry[i].shutdown();
        g_inited[i] = 0;
    }
    g_registered = 0;
    memset(g_registry, 0, sizeof(g_registry));
    g_active = EDEV_HIP;
}

// ------------------------------------------------------------ lifecycle

static int g_initialized = 0;
static ecpu_config_t g_config;

ecpu_config_t ecpu_config_default(void) {
    ecpu_config_t c;
    memset(&c, 0, sizeof(c));
    c.kv_cache_budget_bytes = 4ULL * 1024 * 1024 * 1024;
    c.device_type = EDEV_HIP;
    return c;
}

int ecpu_init(const ecpu_config_t *config) {
    if (g_initialized) return fail(ECPU_ERR_PARAM, "ecpu already initialized");
    register_all();
    g_config = config ? *config : ecpu_config_default();
    if (edevice_init_all() != 0) return fail(ECPU_ERR_DEVICE, "device init failed");
    if (!g_inited[g_config.device_type] || edevice_set_active(g_config.device_type) != 0)
        return fail(ECPU_ERR_DEVICE, "set active device failed (device %d not available)",
                    (int)g_config.device_type);
    const edevice_vtable_t *dev = edevice_active();
    if (!dev) return fail(ECPU_ERR_DEVICE, "no active device");
    g_initialized = 1;
    printf("[ecpu] initialized, device=%s, isa=%s\n", dev->name, ekernel_isa_name(ekernel_detect_isa()));
    return ECPU_OK;
}

void ecpu_shutdown(void) {
    if (!g_initialized) return;
    free_scratch();
    edevice_shutdown_all();
    g_initialized = 0;
    memset(g_err, 0, sizeof(g_err));
}

int ecpu_is_initialized(void) { return g_initialized; }

const char *ecpu_version(void) { return "0.1.0-hip-gfx950"; }

const char *ecpu_last_error(void) {
    std::lock_guard<std::mutex> lk(g_err_mu);
    return g_err[0] ? g_err : nullptr;
}

ekernel_isa_t ekernel_detect_isa(void) { return EKERNEL_ISA_GFX950; }

const char *ekernel_isa_name(ekernel_isa_t isa) {
    switch (isa) {
        case EKERNEL_ISA_SCALAR: return "scalar";
        case EKERNEL_ISA_AVX2: return "avx2";
        case EKERNEL_ISA_AVX512: return "avx512";
        case EKERNEL_ISA_AMX: return "amx";
        case EKERNEL_ISA_NEON: return "neon";
        case EKERNEL_ISA_SVE: return "sve";
        case EKERNEL_ISA_GFX950: return "gfx950";
        default: return "unknown";
    }
}

int ecpu_hip_set_stream(void *s) {
    g_stream = (hipStream_t)s;
    return ECPU_OK;
}

void *ecpu_hip_get_stream(void) { return (void *)g_stream; }

}  // extern "C"
