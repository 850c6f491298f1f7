// Measurement-only kernels for the benchmark (libnq_measure.so): not part of the
// serving library's C ABI and not called by any serving path.
//
// nq_kv_read_probe: read-bandwidth yardstick for the decode attention's access
// pattern.  Every page of `pages` is read whole (page_bytes, a multiple of
// 64 KiB) and folded into one xor per thread, nothing else; ids outside
// [0, num_pages) are skipped.  One workgroup of 256 threads per page at a time,
// 16 x 128-bit loads per thread in flight.  `out` (>= grid words) is written
// only for an impossible xor value, so the loads stay live.  With the pages of
// a permuted pool it bounds the paged gather; with pages 0, 1, 2, ... of the
// same buffer it is a plain contiguous read of the same bytes.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

__global__ void __launch_bounds__(256)
kv_read_probe_kernel(const uint4 *__restrict__ base, int num_pages, const int32_t *__restrict__ pages, int n_pages,
                     int64_t page_vec, uint32_t *__restrict__ out) {
    uint32_t acc = 0;
    for (int p = blockIdx.x; p < n_pages; p += gridDim.x) {
        const int page = pages[p];
        if (static_cast<unsigned>(page) >= static_cast<unsigned>(num_pages)) continue;
        const uint4 *src = base + static_cast<int64_t>(page) * page_vec;
        for (int64_t at = 0; at < page_vec; at += 16 * 256) {
            uint4 v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) v[i] = src[at + i * 256 + threadIdx.x];
#pragma unroll
            for (int i = 0; i < 16; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
        }
    }
    if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;
}

}  // namespace

// Returns 0, -1 for a bad argument, -2 for an unsupported page size or alignment, -3 for a
// launch failure (the serving library's status values).
extern "C" int nq_kv_read_probe(const void *base, int num_pages, int64_t page_bytes, const int32_t *pages,
                                int n_pages, int grid, uint32_t *out, void *stream) {
    if (!base || !pages || !out || n_pages < 1 || num_pages < 1 || grid < 1) return -1;
    if (page_bytes <= 0 || page_bytes % (16 * 16 * 256) != 0 || (reinterpret_cast<uintptr_t>(base) & 15) != 0)
        return -2;
    hipLaunchKernelGGL(kv_read_probe_kernel, dim3(grid), dim3(256), 0, static_cast<hipStream_t>(stream),
                       static_cast<const uint4 *>(base), num_pages, pages, n_pages, page_bytes / 16, out);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}
