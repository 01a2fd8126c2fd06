// Error state, device-attribute cache and the HBM-resident weight buffers.
//
// The buffers replace the reference's cuFile path (runtime/gds_io.cu:93-191):
// weights live fully resident in HBM, so a "read" is pread() into pinned host
// staging followed by an async copy, double-buffered so disk and PCIe overlap.

#include <fcntl.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <cstring>

#include <mutex>
#include <vector>

#include "common.h"

namespace gdsllm {

namespace {
thread_local std::string g_last_error;
constexpr int kMaxDevices = 64;
std::atomic<int> g_cu_count[kMaxDevices];
std::atomic<int> g_lds_bytes[kMaxDevices];
}  // namespace

int set_error(int code, const std::string& msg) {
    g_last_error = msg;
    return code;
}

int ok() {
    g_last_error.clear();
    return GDSLLM_OK;
}

int check_hip(hipError_t err, const char* what) {
    if (err == hipSuccess) return GDSLLM_OK;
    return set_error(GDSLLM_ERR_HIP, std::string(what) + ": " + hipGetErrorString(err));
}

static int device_attr(std::atomic<int>* cache, hipDeviceAttribute_t attr, int fallback) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return fallback;
    int v = cache[dev].load(std::memory_order_relaxed);
    if (v > 0) return v;
    if (hipDeviceGetAttribute(&v, attr, dev) != hipSuccess || v <= 0) return fallback;
    cache[dev].store(v, std::memory_order_relaxed);
    return v;
}

int cu_count() { return device_attr(g_cu_count, hipDeviceAttributeMultiprocessorCount, 256); }

int max_lds_bytes() {
    return device_attr(g_lds_bytes, hipDeviceAttributeMaxSharedMemoryPerBlock, 65536);
}

int prepare_lds(const void* fn, size_t lds) {
    if (lds <= 65536) return GDSLLM_OK;
    return check_hip(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(lds)),
                     "hipFuncSetAttribute");
}

int blocks_per_cu(const void* fn, size_t lds, int threads) {
    struct Entry {
        const void* fn;
        size_t lds;
        int threads, n;
    };
    static std::mutex mu;
    static std::vector<Entry> cache;
    std::lock_guard<std::mutex> lock(mu);
    for (const Entry& e : cache)
        if (e.fn == fn && e.lds == lds && e.threads == threads) return e.n;
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, lds) != hipSuccess || n <= 0) n = 1;
    cache.push_back({fn, lds, threads, n});
    return n;
}

}  // namespace gdsllm

using namespace gdsllm;

extern "C" const char* gdsllm_last_error(void) { return g_last_error.c_str(); }

extern "C" const char* gdsllm_version(void) { return "gdsllm_amd 0.1.0 (gfx950)"; }

extern "C" int gdsllm_buffer_alloc(size_t size, int device_id, void** dev_ptr,
                                   size_t* rounded_size) {
    if (dev_ptr == nullptr) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gdsllm_buffer_alloc: dev_ptr is null");
    *dev_ptr = nullptr;
    if (device_id < 0) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gdsllm_buffer_alloc: negative device id");
    // 4 KiB rounding as in gds_alloc (runtime/gds_io.cu:97-99).
    const size_t aligned = ((size + 4095) / 4096) * 4096;
    if (rounded_size) *rounded_size = aligned;
    int prev = 0;
    if (int rc = check_hip(hipGetDevice(&prev), "hipGetDevice")) return rc;
    if (int rc = check_hip(hipSetDevice(device_id), "hipSetDevice")) return rc;
    void* p = nullptr;
    hipError_t err = aligned ? hipMalloc(&p, aligned) : hipSuccess;
    (void)hipSetDevice(prev);
    if (err == hipErrorOutOfMemory)
        return set_error(GDSLLM_ERR_OUT_OF_MEMORY,
                         "gdsllm_buffer_alloc: out of memory allocating " + std::to_string(aligned) + " bytes");
    if (int rc = check_hip(err, "hipMalloc")) return rc;
    *dev_ptr = p;
    return ok();
}

extern "C" int gdsllm_buffer_free(void* dev_ptr, int device_id) {
    if (dev_ptr == nullptr) return ok();
    int prev = 0;
    if (int rc = check_hip(hipGetDevice(&prev), "hipGetDevice")) return rc;
    if (int rc = check_hip(hipSetDevice(device_id), "hipSetDevice")) return rc;
    hipError_t err = hipFree(dev_ptr);
    (void)hipSetDevice(prev);
    if (int rc = check_hip(err, "hipFree")) return rc;
    return ok();
}

extern "C" int gdsllm_buffer_read_file(void* dev_ptr, size_t buf_size, const char* path,
                                       size_t size, int64_t file_offset, int64_t buf_offset,
                                       int device_id, int64_t* bytes_read) {
    if (bytes_read) *bytes_read = 0;
    if (dev_ptr == nullptr) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: invalid buffer");
    if (path == nullptr) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: null path");
    if (file_offset < 0 || buf_offset < 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: negative offset");
    // Same bound as gds_read (runtime/gds_io.cu:140-142).
    if (static_cast<size_t>(buf_offset) + size > buf_size)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: read would exceed buffer size");

    int fd = open(path, O_RDONLY);
    if (fd < 0)
        return set_error(GDSLLM_ERR_IO, std::string("gds_read: cannot open file '") + path +
                                            "': " + strerror(errno));
    int prev = 0;
    if (int rc = check_hip(hipGetDevice(&prev), "hipGetDevice")) { close(fd); return rc; }
    if (int rc = check_hip(hipSetDevice(device_id), "hipSetDevice")) { close(fd); return rc; }

    constexpr size_t kChunk = 64u << 20;
    void* staging[2] = {nullptr, nullptr};
    hipEvent_t done[2] = {nullptr, nullptr};
    hipStream_t stream = nullptr;
    int rc = GDSLLM_OK;
    int64_t total = 0;
    size_t nstage = size < kChunk ? size : kChunk;
    if (size > 0) {
        rc = check_hip(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreate");
        for (int i = 0; i < 2 && rc == GDSLLM_OK; ++i) {
            rc = check_hip(hipHostMalloc(&staging[i], nstage, hipHostMallocDefault), "hipHostMalloc");
            if (rc == GDSLLM_OK) rc = check_hip(hipEventCreateWithFlags(&done[i], hipEventDisableTiming), "hipEventCreate");
        }
    }
    size_t pos = 0;
    int slot = 0;
    while (rc == GDSLLM_OK && pos < size) {
        // The copy that last used this staging slot must finish before refill.
        rc = check_hip(hipEventSynchronize(done[slot]), "hipEventSynchronize");
        if (rc) break;
        const size_t want = (size - pos) < nstage ? (size - pos) : nstage;
        size_t got = 0;
        while (got < want) {
            ssize_t n = pread(fd, static_cast<char*>(staging[slot]) + got, want - got,
                              static_cast<off_t>(file_offset + pos + got));
            if (n < 0) {
                if (errno == EINTR) continue;
                rc = set_error(GDSLLM_ERR_IO, std::string("gds_read: read failed for '") + path +
                                                  "': " + strerror(errno));
                break;
            }
            if (n == 0) break;  // end of file: short read, reported via bytes_read
            got += static_cast<size_t>(n);
        }
        if (rc) break;
        if (got > 0) {
            rc = check_hip(hipMemcpyAsync(static_cast<char*>(dev_ptr) + buf_offset + pos, staging[slot],
                                          got, hipMemcpyHostToDevice, stream),
                           "hipMemcpyAsync");
            if (rc == GDSLLM_OK) rc = check_hip(hipEventRecord(done[slot], stream), "hipEventRecord");
        }
        pos += got;
        total += static_cast<int64_t>(got);
        if (got < want) break;
        slot ^= 1;
    }
    if (stream) {
        hipError_t e = hipStreamSynchronize(stream);
        if (rc == GDSLLM_OK) rc = check_hip(e, "hipStreamSynchronize");
        (void)hipStreamDestroy(stream);
    }
    for (int i = 0; i < 2; ++i) {
        if (done[i]) (void)hipEventDestroy(done[i]);
        if (staging[i]) (void)hipHostFree(staging[i]);
    }
    close(fd);
    (void)hipSetDevice(prev);
    if (rc) return rc;
    if (bytes_read) *bytes_read = total;
    return ok();
}
