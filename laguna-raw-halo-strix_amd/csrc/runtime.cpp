// Runtime half of the C ABI: errors, devices, buffers, streams.
// Replaces the reference's VulkanContext / GpuBuffer (src/vulkan.rs:16-452):
// device-local HBM instead of host-visible coherent memory, explicit frees,
// asynchronous streams instead of one fence wait per dispatch.
#include <map>
#include <mutex>
#include <string>
#include <thread>
#include <tuple>
#include <vector>

#include "lg_common.hpp"

namespace lg {

static thread_local std::string g_err;
static bool g_blocking = false;

int fail(int status, const char *fmt, ...) {
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_err = buf;
    return status;
}

void clear_error() { g_err.clear(); }

// Compute units of the current device (cached per device; 256 if the query fails).
int device_cus() {
    static std::mutex mu;
    static int cus[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    std::lock_guard<std::mutex> lk(mu);
    if (!cus[dev]) {
        int c = 0;
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) c = 256;
        cus[dev] = c;
    }
    return cus[dev];
}

// Registry of live lg_buf_alloc allocations: base -> size.
static std::mutex g_mu;
static std::map<uintptr_t, uint64_t> g_allocs;

bool extent_ok(const void *p, uint64_t bytes) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_allocs.upper_bound(a);
    if (it == g_allocs.begin()) return true;  // below every known allocation
    --it;
    const uintptr_t base = it->first;
    const uint64_t size = it->second;
    if (a >= base + size) return true;  // not inside a known allocation
    return (a - base) + bytes <= size;
}

static thread_local int t_deferred = 0;
bool blocking() { return g_blocking && t_deferred == 0; }
DeferSync::DeferSync() { t_deferred++; }
DeferSync::~DeferSync() { t_deferred--; }

int after_launch(const char *what, hipStream_t s) {
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(LG_EHIP, "%s launch failed: %s", what, hipGetErrorString(e));
    if (blocking()) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        e = hipStreamIsCapturing(s, &cs);
        if (e != hipSuccess) return fail(LG_EHIP, "%s: %s", what, hipGetErrorString(e));
        if (cs != hipStreamCaptureStatusNone) return LG_OK;  // a capturing stream cannot be synchronised
        e = hipStreamSynchronize(s);
        if (e != hipSuccess) return fail(LG_EHIP, "%s: %s", what, hipGetErrorString(e));
    }
    return LG_OK;
}

// ---- library-owned device buffers, one per (purpose, device, stream)

static std::mutex g_sb_mu;
// (purpose, device, stream handle, host thread): the thread is part of the key only for
// hipStreamPerThread, one handle that names a different stream in each host thread
static std::map<std::tuple<int, int, uintptr_t, size_t>, StreamBuf> g_sb;

static size_t stream_thread(hipStream_t s) {
    return s == hipStreamPerThread ? std::hash<std::thread::id>{}(std::this_thread::get_id()) : 0;
}
static std::vector<void *> g_retired;  // buffers a captured graph may still use: never freed

BufLease::~BufLease() { delete static_cast<std::unique_lock<std::mutex> *>(lock); }

int stream_buffer(int purpose, hipStream_t s, uint64_t need, BufLease &lease, const char *what) {
    int dev = 0;
    LG_HIP_TRY(hipGetDevice(&dev));
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    LG_HIP_TRY(hipStreamIsCapturing(s, &cs));
    const bool capturing = cs != hipStreamCaptureStatusNone;
    auto *lk = new std::unique_lock<std::mutex>(g_sb_mu);
    lease.lock = lk;
    StreamBuf &b = g_sb[std::make_tuple(purpose, dev, reinterpret_cast<uintptr_t>(s), stream_thread(s))];
    if (b.bytes < need) {
        if (capturing)
            return fail(LG_EINVAL,
                        "%s: its device workspace must grow to %llu bytes while the stream is being captured; make "
                        "the same call once on this stream before capturing",
                        what, (unsigned long long)need);
        if (b.ptr) {
            if (b.captured) {
                g_retired.push_back(b.ptr);
            } else {
                LG_HIP_TRY(hipStreamSynchronize(s));  // earlier launches on this stream may still use it
                LG_HIP_TRY(hipFree(b.ptr));
            }
        }
        b = StreamBuf();
        const uint64_t sz = (need + (1u << 20) - 1) & ~(uint64_t)((1u << 20) - 1);
        void *p = nullptr;
        if (hipMalloc(&p, sz) != hipSuccess) {
            (void)hipGetLastError();
            return fail(LG_ENOMEM, "%s: device workspace of %llu bytes", what, (unsigned long long)sz);
        }
        LG_HIP_TRY(hipMemsetAsync(p, 0, sz, s));  // arrival counters start at zero
        b.ptr = p;
        b.bytes = sz;
    }
    if (capturing) b.captured = true;
    lease.buf = &b;
    return LG_OK;
}

// Drops the buffers of stream s on every device (lg_stream_destroy): freed after the
// stream's work, or retired when a captured graph may still use them.
static int release_stream_buffers(hipStream_t s) {
    std::lock_guard<std::mutex> lk(g_sb_mu);
    bool synced = false;
    for (auto it = g_sb.begin(); it != g_sb.end();) {
        if (std::get<2>(it->first) != reinterpret_cast<uintptr_t>(s) || std::get<3>(it->first) != stream_thread(s)) {
            ++it;
            continue;
        }
        StreamBuf &b = it->second;
        if (b.ptr) {
            if (b.captured) {
                g_retired.push_back(b.ptr);
            } else {
                if (!synced) LG_HIP_TRY(hipStreamSynchronize(s));
                synced = true;
                LG_HIP_TRY(hipFree(b.ptr));
            }
        }
        it = g_sb.erase(it);
    }
    return LG_OK;
}

int stream_workspace(hipStream_t s, uint64_t need, void **out) {
    BufLease lease;
    LG_TRY(stream_buffer(BUF_PRODUCT, s, need, lease, "product workspace"));
    *out = lease.buf->ptr;
    return LG_OK;
}

// Plain 16-byte copy (lg_buf_copy).  It is also the known-size kernel that hardware
// traffic counters are calibrated against (bytes read = bytes written = size).
__global__ __launch_bounds__(256) void k_copy16(const uint4 *__restrict__ src, uint4 *__restrict__ dst, uint64_t n16) {
    for (uint64_t i = (uint64_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += (uint64_t)gridDim.x * 256) dst[i] = src[i];
}

}  // namespace lg

using namespace lg;

extern "C" {

const char *lg_last_error(void) { return g_err.c_str(); }

const char *lg_version(void) { return "laguna-hip 0.1 (gfx950)"; }

int lg_device_count(int *count) {
    LG_REQUIRE(count, "lg_device_count: null count");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    (void)hipGetLastError();
    *count = n;
    return LG_OK;
}

int lg_init(int device) {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
        (void)hipGetLastError();
        return fail(LG_ENODEV, "lg_init: no HIP device");
    }
    LG_REQUIRE(device >= 0 && device < n, "lg_init: device %d out of range (%d devices)", device, n);
    LG_HIP_TRY(hipSetDevice(device));
    LG_HIP_TRY(hipFree(nullptr));  // create the context now, not inside the first timed call
    LG_TRY(static_scratch_setup(device));
    clear_error();
    return LG_OK;
}

int lg_set_blocking(int b) {
    g_blocking = b != 0;
    return LG_OK;
}

int lg_buf_alloc(void **dptr, uint64_t bytes) {
    LG_REQUIRE(dptr, "lg_buf_alloc: null dptr");
    LG_REQUIRE(bytes > 0, "lg_buf_alloc: zero bytes");
    void *p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(LG_ENOMEM, "lg_buf_alloc(%llu): %s", (unsigned long long)bytes, hipGetErrorString(e));
    }
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_allocs[reinterpret_cast<uintptr_t>(p)] = bytes;
    }
    *dptr = p;
    return LG_OK;
}

int lg_buf_free(void *dptr) {
    if (!dptr) return LG_OK;
    {
        std::lock_guard<std::mutex> lk(g_mu);
        g_allocs.erase(reinterpret_cast<uintptr_t>(dptr));
    }
    LG_HIP_TRY(hipFree(dptr));
    return LG_OK;
}

int lg_buf_upload(void *dst, const void *src, uint64_t bytes, void *stream) {
    if (bytes == 0) return LG_OK;
    LG_REQUIRE(dst && src, "lg_buf_upload: null pointer");
    LG_EXTENT(dst, bytes, "lg_buf_upload dst");
    LG_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, (hipStream_t)stream));
    LG_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return LG_OK;
}

int lg_buf_download(void *dst, const void *src, uint64_t bytes, void *stream) {
    if (bytes == 0) return LG_OK;
    LG_REQUIRE(dst && src, "lg_buf_download: null pointer");
    LG_EXTENT(src, bytes, "lg_buf_download src");
    LG_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, (hipStream_t)stream));
    LG_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return LG_OK;
}

int lg_buf_memset(void *dst, int value, uint64_t bytes, void *stream) {
    if (bytes == 0) return LG_OK;
    LG_REQUIRE(dst, "lg_buf_memset: null pointer");
    LG_EXTENT(dst, bytes, "lg_buf_memset dst");
    LG_HIP_TRY(hipMemsetAsync(dst, value, bytes, (hipStream_t)stream));
    return after_launch("lg_buf_memset", (hipStream_t)stream);
}

int lg_buf_copy(void *dst, const void *src, uint64_t bytes, void *stream) {
    if (bytes == 0) return LG_OK;
    LG_REQUIRE(dst && src, "lg_buf_copy: null pointer");
    LG_EXTENT(dst, bytes, "lg_buf_copy dst");
    LG_EXTENT(src, bytes, "lg_buf_copy src");
    hipStream_t s = (hipStream_t)stream;
    const bool vec = bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(dst) & 15u) == 0 &&
                     (reinterpret_cast<uintptr_t>(src) & 15u) == 0;
    if (!vec) {
        LG_HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, s));
        return after_launch("lg_buf_copy", s);
    }
    const uint64_t n16 = bytes / 16;
    uint64_t grid = (n16 + 255) / 256;
    grid = grid < 4096 ? grid : 4096;
    hipLaunchKernelGGL(k_copy16, dim3((unsigned)grid), dim3(256), 0, s, static_cast<const uint4 *>(src),
                       static_cast<uint4 *>(dst), n16);
    return after_launch("lg_buf_copy", s);
}

int lg_stream_create(void **stream) {
    LG_REQUIRE(stream, "lg_stream_create: null");
    hipStream_t s = nullptr;
    LG_HIP_TRY(hipStreamCreateWithFlags(&s, hipStreamNonBlocking));
    *stream = s;
    return LG_OK;
}

int lg_stream_destroy(void *stream) {
    if (!stream) return LG_OK;
    LG_TRY(release_stream_buffers((hipStream_t)stream));
    LG_HIP_TRY(hipStreamDestroy((hipStream_t)stream));
    return LG_OK;
}

int lg_sync(void *stream) {
    LG_HIP_TRY(hipStreamSynchronize((hipStream_t)stream));
    return LG_OK;
}

}  // extern "C"
