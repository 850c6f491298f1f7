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

// The same pages read the way the decode attention reads them: workgroup (group g, kv head h) of a
// grid of groups x heads reads, for pages g, g + groups, g + 2 groups, ..., only head h's rows -- the
// 256-byte K and V rows of every slot, at offset 256 h of each slot row of the [page, 2, slot, head,
// 128] bf16 layout -- sixteen lanes per row, U pages' loads in flight per thread.
template <int U>
__global__ void __launch_bounds__(256)
kv_head_read_probe_kernel(const uint4 *__restrict__ base, int num_pages, const int32_t *__restrict__ pages,
                          int n_pages, int64_t page_vec, int heads, int slots, uint32_t *__restrict__ out) {
    const int h = static_cast<int>(blockIdx.x) % heads, g = static_cast<int>(blockIdx.x) / heads;
    const int groups = static_cast<int>(gridDim.x) / heads;
    const int64_t kind_vec = page_vec / 2, slot_vec = static_cast<int64_t>(heads) * 16;
    // the head's 2 x slots x 16 vectors of a page (512 with 16 slots): thread t takes t and t + 256
    int64_t off[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int idx = static_cast<int>(threadIdx.x) + 256 * j;
        const int kind = idx / (slots * 16), rest = idx - kind * (slots * 16);
        off[j] = kind * kind_vec + (rest / 16) * slot_vec + h * 16 + (rest % 16);
    }
    uint32_t acc = 0;
    for (int p0 = g; p0 < n_pages; p0 += U * groups) {
        uint4 v[2 * U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int p = p0 + u * groups;
            const int page = p < n_pages ? pages[p] : -1;
            const bool ok = static_cast<unsigned>(page) < static_cast<unsigned>(num_pages);
            const uint4 *src = base + static_cast<int64_t>(ok ? page : 0) * page_vec;
            v[2 * u] = ok ? src[off[0]] : make_uint4(0, 0, 0, 0);
            v[2 * u + 1] = ok ? src[off[1]] : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int i = 0; i < 2 * U; ++i) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    }
    if (acc == 0x9e3779b9u) out[blockIdx.x] = acc;
}

}  // namespace

// Per-head reads of the same pages (kv_head_read_probe_kernel): 16 slots of `heads` rows of 256
// bytes per kind, page_bytes == 2 x 16 x heads x 256; grid = groups x heads workgroups; depth = pages
// in flight per thread (8 or 16).  Same status values as nq_kv_read_probe.
extern "C" int nq_kv_head_read_probe(const void *base, int num_pages, int64_t page_bytes, const int32_t *pages,
                                     int n_pages, int heads, int groups, int depth, uint32_t *out, void *stream) {
    if (!base || !pages || !out || n_pages < 1 || num_pages < 1 || heads < 1 || groups < 1) return -1;
    if (depth != 8 && depth != 16) return -1;
    if (page_bytes != 2LL * 16 * heads * 256 || (reinterpret_cast<uintptr_t>(base) & 15) != 0) return -2;
    const dim3 grid(static_cast<unsigned>(groups * heads));
    const uint4 *b = static_cast<const uint4 *>(base);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (depth == 8)
        hipLaunchKernelGGL(kv_head_read_probe_kernel<8>, grid, dim3(256), 0, st, b, num_pages, pages, n_pages,
                           page_bytes / 16, heads, 16, out);
    else
        hipLaunchKernelGGL(kv_head_read_probe_kernel<16>, grid, dim3(256), 0, st, b, num_pages, pages, n_pages,
                           page_bytes / 16, heads, 16, out);
    return hipGetLastError() == hipSuccess ? 0 : -3;
}

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
