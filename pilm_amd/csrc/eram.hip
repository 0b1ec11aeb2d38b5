// Eram on MI355X: weight residency in HBM.
//
// piLM's Eram (src/ecpu/src/eram/eram.c, include/eram.h:34-41) allocates
// buffers through the active device and maps weight files (Windows only; the
// Linux branch returns NULL).  Here the same entry points allocate HBM
// through the HIP device vtable and map files read-only with mmap; and the
// bundle / cache loaders get one native upload path: file ranges are read
// into two pinned staging buffers in turn and copied to HBM on a copy stream
// of their own, so the disk read of one chunk overlaps the PCIe copy of the
// previous one.  Weights are uploaded once and every kernel then reads them
// in place.
#include <hip/hip_runtime.h>

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cerrno>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "internal.h"

struct eram_buffer {
    void *data;
    size_t size;
    int flags;
    int is_mmap;
};

namespace {

constexpr size_t kStageBytes = 16u << 20;   // per staging buffer

struct Uploader {
    std::mutex mu;
    int dev = -1;
    hipStream_t stream = nullptr;
    void *stage[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
};
Uploader g_up;

// One-time set-up for the current device (staging buffers are pinned host
// memory from hipHostMalloc).
int uploader_ready(const char *fn) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return pilm::fail(ECPU_ERR_DEVICE, "%s: no current HIP device", fn);
    if (g_up.dev == dev && g_up.stream) return ECPU_OK;
    if (g_up.stream) return pilm::fail(ECPU_ERR_UNSUPPORTED, "%s: the uploader serves device %d only", fn, g_up.dev);
    if (hipStreamCreateWithFlags(&g_up.stream, hipStreamNonBlocking) != hipSuccess)
        return pilm::fail(ECPU_ERR_DEVICE, "%s: creating the copy stream failed", fn);
    for (int b = 0; b < 2; ++b) {
        if (hipHostMalloc(&g_up.stage[b], kStageBytes, hipHostMallocDefault) != hipSuccess ||
            hipEventCreateWithFlags(&g_up.done[b], hipEventDisableTiming) != hipSuccess) {
            (void)hipGetLastError();
            return pilm::fail(ECPU_ERR_MEM, "%s: pinned staging allocation failed", fn);
        }
    }
    g_up.dev = dev;
    return ECPU_OK;
}

}  // namespace

extern "C" {

// ---- eram.h:34-37 --------------------------------------------------------
eram_buffer_t *eram_buffer_alloc(size_t bytes, eram_flags_t flags) {
    const edevice_vtable_t *dev = edevice_active();
    if (!dev || !dev->alloc) return nullptr;
    void *p = dev->alloc(bytes, 256);
    if (!p) return nullptr;
    eram_buffer_t *buf = (eram_buffer_t *)calloc(1, sizeof(*buf));
    if (!buf) {
        dev->free(p);
        return nullptr;
    }
    buf->data = p;
    buf->size = bytes;
    buf->flags = (int)flags;
    return buf;
}

void eram_buffer_free(eram_buffer_t *buf) {
    if (!buf) return;
    if (buf->is_mmap) {
        eram_munmap(buf);
        return;
    }
    const edevice_vtable_t *dev = edevice_active();
    if (dev && dev->free) dev->free(buf->data);
    free(buf);
}

void *eram_buffer_data(eram_buffer_t *buf) { return buf ? buf->data : nullptr; }
size_t eram_buffer_size(eram_buffer_t *buf) { return buf ? buf->size : 0; }

// ---- eram.h:39-41: read-only file mapping (host memory) ------------------
eram_buffer_t *eram_mmap(const char *path, eram_flags_t flags) {
    if (!path) return nullptr;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return nullptr;
    struct stat st;
    if (fstat(fd, &st) != 0 || st.st_size <= 0) {
        close(fd);
        return nullptr;
    }
    void *p = mmap(nullptr, (size_t)st.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (p == MAP_FAILED) return nullptr;
    eram_buffer_t *buf = (eram_buffer_t *)calloc(1, sizeof(*buf));
    if (!buf) {
        munmap(p, (size_t)st.st_size);
        return nullptr;
    }
    buf->data = p;
    buf->size = (size_t)st.st_size;
    buf->flags = (int)flags | ERAM_FLAG_MMAP;
    buf->is_mmap = 1;
    return buf;
}

int eram_munmap(eram_buffer_t *buf) {
    if (!buf || !buf->is_mmap) return ECPU_ERR_PARAM;
    munmap(buf->data, buf->size);
    free(buf);
    return ECPU_OK;
}

int eram_advise_random(eram_buffer_t *buf) {
    if (!buf) return ECPU_ERR_PARAM;
    if (buf->is_mmap) (void)madvise(buf->data, buf->size, MADV_RANDOM);
    return ECPU_OK;
}

// ---- additions: file -> HBM upload ----------------------------------------
int eram_hip_load_file(const char *path, size_t n, const size_t *file_offsets, const size_t *bytes,
                       void *const *dst) {
    const char *fn = "eram_hip_load_file";
    if (!path || (n && (!file_offsets || !bytes || !dst))) return pilm::fail(ECPU_ERR_PARAM, "%s: NULL argument", fn);
    for (size_t i = 0; i < n; ++i) {
        if (!dst[i]) return pilm::fail(ECPU_ERR_PARAM, "%s: destination %zu is NULL", fn, i);
        const int rc = pilm::check_device_buffer(dst[i], bytes[i], "destination", fn);
        if (rc != ECPU_OK) return rc;
    }
    std::lock_guard<std::mutex> lk(g_up.mu);
    int rc = uploader_ready(fn);
    if (rc != ECPU_OK) return rc;
    const int fd = open(path, O_RDONLY | O_CLOEXEC);
    if (fd < 0) return pilm::fail(ECPU_ERR_PARAM, "%s: cannot open %s: %s", fn, path, strerror(errno));
    struct stat st;
    if (fstat(fd, &st) != 0) {
        close(fd);
        return pilm::fail(ECPU_ERR_PARAM, "%s: cannot stat %s", fn, path);
    }
    for (size_t i = 0; i < n; ++i) {
        if (file_offsets[i] > (size_t)st.st_size || bytes[i] > (size_t)st.st_size - file_offsets[i]) {
            close(fd);
            return pilm::fail(ECPU_ERR_PARAM, "%s: range %zu (%zu + %zu bytes) is past the end of %s", fn, i,
                              file_offsets[i], bytes[i], path);
        }
    }
    (void)posix_fadvise(fd, 0, 0, POSIX_FADV_SEQUENTIAL);
    int b = 0;
    rc = ECPU_OK;
    for (size_t i = 0; i < n && rc == ECPU_OK; ++i) {
        size_t done = 0;
        while (done < bytes[i]) {
            const size_t chunk = bytes[i] - done < kStageBytes ? bytes[i] - done : kStageBytes;
            // the copy that last used this staging buffer must have finished
            if (hipEventSynchronize(g_up.done[b]) != hipSuccess) {
                rc = pilm::fail(ECPU_ERR_DEVICE, "%s: waiting for a staging copy failed", fn);
                break;
            }
            size_t got = 0;
            while (got < chunk) {
                const ssize_t r = pread(fd, (char *)g_up.stage[b] + got, chunk - got,
                                        (off_t)(file_offsets[i] + done + got));
                if (r <= 0) {
                    if (r < 0 && errno == EINTR) continue;
                    rc = pilm::fail(ECPU_ERR_PARAM, "%s: reading %s failed: %s", fn, path,
                                    r < 0 ? strerror(errno) : "unexpected end of file");
                    break;
                }
                got += (size_t)r;
            }
            if (rc != ECPU_OK) break;
            if (hipMemcpyAsync((char *)dst[i] + done, g_up.stage[b], chunk, hipMemcpyHostToDevice, g_up.stream) !=
                    hipSuccess ||
                hipEventRecord(g_up.done[b], g_up.stream) != hipSuccess) {
                rc = pilm::fail(ECPU_ERR_DEVICE, "%s: host-to-device copy failed", fn);
                break;
            }
            done += chunk;
            b ^= 1;
        }
    }
    close(fd);
    if (hipStreamSynchronize(g_up.stream) != hipSuccess && rc == ECPU_OK)
        rc = pilm::fail(ECPU_ERR_DEVICE, "%s: upload did not complete", fn);
    return rc;
}

}  // extern "C"
