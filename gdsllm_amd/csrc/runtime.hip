// Error state, device-attribute cache and the HBM-resident weight buffers.
//
// The buffers replace the reference's cuFile path (runtime/gds_io.cu:93-191):
// weights live fully resident in HBM, so a "read" is pread() into pinned host
// staging followed by an async copy. Several reader threads each own two
// staging slots and a stream, so page-cache copies, disk reads and PCIe
// transfers of different chunks overlap.

#include <fcntl.h>
#include <unistd.h>

#include <atomic>
#include <cerrno>
#include <cstring>

#include <mutex>
#include <thread>
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

namespace {

// Pinned staging for file -> HBM reads, one pool per device, allocated on the
// first read and kept until the process ends (64 MiB of pinned host memory per
// device that has read a file). Reads on one device take the pool's mutex, so
// they run one at a time; reads on different devices run concurrently.
constexpr int kReaders = 4;
constexpr int kSlots = 2;
constexpr size_t kStageChunk = size_t(8) << 20;

struct StagingPool {
    std::mutex mu;
    bool ready = false;
    void* slot[kReaders][kSlots] = {};
    hipEvent_t done[kReaders][kSlots] = {};
    hipStream_t stream[kReaders] = {};
};
StagingPool g_pools[kMaxDevices];

// Called with pool.mu held and device_id current.
int pool_ready(StagingPool& pool) {
    if (pool.ready) return GDSLLM_OK;
    for (int t = 0; t < kReaders; ++t) {
        if (!pool.stream[t]) {
            if (int rc = check_hip(hipStreamCreateWithFlags(&pool.stream[t], hipStreamNonBlocking), "hipStreamCreate"))
                return rc;
        }
        for (int i = 0; i < kSlots; ++i) {
            if (!pool.slot[t][i]) {
                if (int rc = check_hip(hipHostMalloc(&pool.slot[t][i], kStageChunk, hipHostMallocDefault),
                                       "hipHostMalloc"))
                    return rc;
            }
            if (!pool.done[t][i]) {
                if (int rc = check_hip(hipEventCreateWithFlags(&pool.done[t][i], hipEventDisableTiming),
                                       "hipEventCreate"))
                    return rc;
            }
        }
    }
    pool.ready = true;
    return GDSLLM_OK;
}

struct ReadJob {
    int fd;
    const char* path;
    char* dst;             // device address of byte 0 of the region
    size_t size;
    int64_t file_offset;
    int device_id;
    size_t nchunks;
};

struct ReaderResult {
    int rc = GDSLLM_OK;
    std::string msg;
    size_t short_chunk = SIZE_MAX;  // first chunk that hit end of file
    size_t short_bytes = 0;         // bytes that chunk did hold
};

// Reader t handles chunks t, t + kReaders, ...: pread into its staging slot,
// then an async copy on its own stream; a slot is refilled once the copy that
// last used it has finished.
void run_reader(StagingPool& pool, const ReadJob& job, int t, ReaderResult& res) {
    if (hipSetDevice(job.device_id) != hipSuccess) {
        res.rc = GDSLLM_ERR_HIP;
        res.msg = "hipSetDevice failed in a reader thread";
        return;
    }
    int k = 0;
    for (size_t c = t; c < job.nchunks; c += kReaders, ++k) {
        const int i = k & 1;
        hipError_t e = hipEventSynchronize(pool.done[t][i]);
        if (e != hipSuccess) {
            res.rc = GDSLLM_ERR_HIP;
            res.msg = std::string("hipEventSynchronize: ") + hipGetErrorString(e);
            break;
        }
        const size_t pos = c * kStageChunk;
        const size_t want = job.size - pos < kStageChunk ? job.size - pos : kStageChunk;
        char* buf = static_cast<char*>(pool.slot[t][i]);
        size_t got = 0;
        while (got < want) {
            ssize_t n = pread(job.fd, buf + got, want - got, static_cast<off_t>(job.file_offset + pos + got));
            if (n < 0) {
                if (errno == EINTR) continue;
                res.rc = GDSLLM_ERR_IO;
                res.msg = std::string("gds_read: read failed for '") + job.path + "': " + strerror(errno);
                break;
            }
            if (n == 0) break;
            got += static_cast<size_t>(n);
        }
        if (res.rc) break;
        if (got > 0) {
            e = hipMemcpyAsync(job.dst + pos, buf, got, hipMemcpyHostToDevice, pool.stream[t]);
            if (e == hipSuccess) e = hipEventRecord(pool.done[t][i], pool.stream[t]);
            if (e != hipSuccess) {
                res.rc = GDSLLM_ERR_HIP;
                res.msg = std::string("hipMemcpyAsync: ") + hipGetErrorString(e);
                break;
            }
        }
        if (got < want) {  // end of file: later chunks of this reader are past it too
            res.short_chunk = c;
            res.short_bytes = got;
            break;
        }
    }
    hipError_t e = hipStreamSynchronize(pool.stream[t]);
    if (e != hipSuccess && res.rc == GDSLLM_OK) {
        res.rc = GDSLLM_ERR_HIP;
        res.msg = std::string("hipStreamSynchronize: ") + hipGetErrorString(e);
    }
}

}  // namespace

extern "C" int gdsllm_buffer_read_file(void* dev_ptr, size_t buf_size, const char* path,
                                       size_t size, int64_t file_offset, int64_t buf_offset,
                                       int device_id, int64_t* bytes_read) {
    if (bytes_read) *bytes_read = 0;
    if (dev_ptr == nullptr) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: invalid buffer");
    if (path == nullptr) return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: null path");
    if (file_offset < 0 || buf_offset < 0)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: negative offset");
    if (device_id < 0 || device_id >= kMaxDevices)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: device id out of range");
    // Same bound as gds_read (runtime/gds_io.cu:140-142).
    if (static_cast<size_t>(buf_offset) + size > buf_size)
        return set_error(GDSLLM_ERR_INVALID_ARGUMENT, "gds_read: read would exceed buffer size");

    int fd = open(path, O_RDONLY);
    if (fd < 0)
        return set_error(GDSLLM_ERR_IO, std::string("gds_read: cannot open file '") + path +
                                            "': " + strerror(errno));
    if (size == 0) {
        close(fd);
        return ok();
    }
    int prev = 0;
    if (int rc = check_hip(hipGetDevice(&prev), "hipGetDevice")) { close(fd); return rc; }
    if (int rc = check_hip(hipSetDevice(device_id), "hipSetDevice")) { close(fd); return rc; }

    StagingPool& pool = g_pools[device_id];
    std::lock_guard<std::mutex> lock(pool.mu);
    int rc = pool_ready(pool);
    ReaderResult res[kReaders];
    const ReadJob job{fd, path, static_cast<char*>(dev_ptr) + buf_offset, size, file_offset, device_id,
                      (size + kStageChunk - 1) / kStageChunk};
    if (rc == GDSLLM_OK) {
        const int nthreads = job.nchunks < size_t(kReaders) ? static_cast<int>(job.nchunks) : kReaders;
        std::vector<std::thread> workers;
        for (int t = 1; t < nthreads; ++t)
            workers.emplace_back(run_reader, std::ref(pool), std::cref(job), t, std::ref(res[t]));
        run_reader(pool, job, 0, res[0]);
        for (auto& w : workers) w.join();
        for (int t = 0; t < nthreads && rc == GDSLLM_OK; ++t)
            if (res[t].rc) rc = set_error(res[t].rc, res[t].msg);
    }
    close(fd);
    (void)hipSetDevice(prev);
    if (rc) return rc;
    // Bytes up to the first end-of-file chunk, as a sequential read would stop.
    size_t total = size;
    for (int t = 0; t < kReaders; ++t)
        if (res[t].short_chunk != SIZE_MAX) {
            const size_t upto = res[t].short_chunk * kStageChunk + res[t].short_bytes;
            if (upto < total) total = upto;
        }
    if (bytes_read) *bytes_read = static_cast<int64_t>(total);
    return ok();
}
