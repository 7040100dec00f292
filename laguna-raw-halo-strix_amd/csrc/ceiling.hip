// Ceiling kernels for measurement (no counterpart in the reference): an empty
// kernel and a plain streaming read.  Timed next to the projections, they give what
// one launch and one read of the same bytes cost on this device, so that each
// projection's time can be read against both.
#include "lg_common.hpp"

using namespace lg;

// Written only if a read's checksum hits a magic value (never, in practice); external
// linkage keeps the store, and so the loads feeding it, in the kernel.
__device__ uint32_t lg_bench_sink;

namespace {

__global__ __launch_bounds__(256) void k_empty() {}

// Every thread issues its READ_L 16-byte loads at once; workgroup b reads the
// contiguous READ_L * 4 KiB starting at b * READ_L * 4 KiB (the last one re-reads the
// final 16 bytes for its indices past the end).
constexpr int READ_L = 8;

__global__ __launch_bounds__(256) void k_read(const uint4 *__restrict__ p, uint64_t n16) {
    const uint64_t base = (uint64_t)blockIdx.x * READ_L * 256 + threadIdx.x;
    uint4 v[READ_L];
#pragma unroll
    for (int i = 0; i < READ_L; i++) {
        const uint64_t j = base + (uint64_t)i * 256;
        v[i] = p[j < n16 ? j : n16 - 1];
    }
    uint32_t s = 0;
#pragma unroll
    for (int i = 0; i < READ_L; i++) s ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    if (s == 0x9E3779B9u) lg_bench_sink = s;
}

}  // namespace

extern "C" int lg_bench_empty(uint32_t workgroups, void *stream) {
    clear_error();
    LG_REQUIRE(workgroups >= 1 && workgroups <= 65535u, "lg_bench_empty: %u workgroups (1..65535)", workgroups);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_empty, dim3(workgroups), dim3(256), 0, s);
    return after_launch("lg_bench_empty", s);
}

extern "C" int lg_bench_read(const void *buf, uint64_t bytes, void *stream) {
    clear_error();
    LG_REQUIRE(buf, "lg_bench_read: null buffer");
    LG_REQUIRE(bytes >= 16 && bytes % 16 == 0 && (reinterpret_cast<uintptr_t>(buf) & 15u) == 0,
               "lg_bench_read: %llu bytes (a positive multiple of 16, 16-byte aligned)", (unsigned long long)bytes);
    LG_EXTENT(buf, bytes, "lg_bench_read");
    const uint64_t n16 = bytes / 16, per = (uint64_t)READ_L * 256;
    const uint64_t wgs = (n16 + per - 1) / per;
    LG_REQUIRE(wgs <= 0x7FFFFFFFu, "lg_bench_read: %llu bytes is too large", (unsigned long long)bytes);
    hipStream_t s = (hipStream_t)stream;
    hipLaunchKernelGGL(k_read, dim3((uint32_t)wgs), dim3(256), 0, s, static_cast<const uint4 *>(buf), n16);
    return after_launch("lg_bench_read", s);
}
