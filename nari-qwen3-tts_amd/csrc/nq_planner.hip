// GPU construction of the ragged paged-KV metadata of one capture bucket.
//
// Restates PagedTalkerKV._metadata (executor/talker_kv.py:403-483) and the
// page choice of PagedKVAllocator.reserve (executor/cache.py:135-184) as
// integer kernels.  Every workgroup scans the (few) row descriptors into LDS
// redundantly, so no inter-workgroup synchronisation is needed; the
// O(pages + tokens) output fill is then spread grid-stride over the launch.
#include "nq_common.h"

namespace nq {
namespace {

constexpr int kPlanThreads = 1024;  // also the largest capture bucket supported

// Largest r in [0, n) with off[r] <= x (off non-decreasing, off[0] == 0).
__device__ __forceinline__ int find_row(const int *off, int n, int x) {
    int lo = 0, hi = n;  // invariant: off[lo] <= x, answer in [lo, hi)
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= x) lo = mid; else hi = mid;
    }
    return lo;
}

__global__ void __launch_bounds__(kPlanThreads)
plan_ragged_kernel(const int32_t *__restrict__ seq_len, const int32_t *__restrict__ pos_start,
                   const int32_t *__restrict__ advance, const int32_t *__restrict__ prior_pages,
                   const int32_t *__restrict__ table_row, int n_rows, int capture_rows,
                   int token_capacity, int page_size, int prefill, int32_t *__restrict__ page_table,
                   int64_t table_stride, const int32_t *__restrict__ free_pages, int n_free,
                   const int32_t *__restrict__ expect_pages, const int32_t *__restrict__ scratch_pages,
                   int32_t *__restrict__ qo_indptr,
                   int32_t *__restrict__ kv_indptr, int32_t *__restrict__ kv_indices,
                   int64_t kv_indices_capacity, int32_t *__restrict__ last_page_len,
                   int64_t *__restrict__ position_ids, int64_t *__restrict__ write_pages,
                   int64_t *__restrict__ write_offsets, int32_t *__restrict__ status) {
    __shared__ int s_page_off[kPlanThreads];
    __shared__ int s_tok_off[kPlanThreads];
    __shared__ int s_miss_off[kPlanThreads];
    // the rows' descriptors, read once here for the fill loops below
    __shared__ int s_seq[kPlanThreads], s_prior[kPlanThreads], s_trow[kPlanThreads], s_pos[kPlanThreads];
    __shared__ int s_tmp[5 * (kWave + 1)];

    const int r = threadIdx.x;
    int npages = 0, ntok = 0, miss = 0, adv_real = 0, bad = 0, total = 0;
    if (r < n_rows) {
        const int sl = seq_len[r], adv = advance[r], pr = prior_pages[r];
        s_seq[r] = sl;
        s_prior[r] = pr;
        s_trow[r] = table_row[r];
        s_pos[r] = pos_start[r];
        total = sl + adv;
        const int needed = (total + page_size - 1) / page_size;
        miss = needed - pr;
        if (miss < 0 || adv < 1) bad = 1;
        npages = needed;
        ntok = adv;
        adv_real = adv;
    } else if (r < capture_rows) {
        npages = 1;
        ntok = prefill ? 0 : 1;
    }
    // page, token and new-page offsets, the real advance and the error flag in one scan
    int ex[5], tot[5];
    block_exclusive_scan_n<5>({npages, ntok, miss > 0 ? miss : 0, adv_real, bad}, s_tmp, ex, tot);
    const int page_off = ex[0], tok_off = ex[1], miss_off = ex[2];
    const int total_pages = tot[0], total_tok = tot[1], total_miss = tot[2], sum_adv = tot[3], any_bad = tot[4];
    s_page_off[r] = page_off;
    s_tok_off[r] = tok_off;
    s_miss_off[r] = miss_off;
    __syncthreads();

    int err = NQ_OK;
    if (any_bad || total_pages > kv_indices_capacity || total_tok > token_capacity)
        err = NQ_ERR_INVALID_ARGUMENT;
    else if (total_miss > n_free)
        err = NQ_ERR_CAPACITY;
    if (err != NQ_OK) {
        if (blockIdx.x == 0 && r == 0) {
            status[0] = err;
            status[1] = 0;
        }
        return;
    }
    if (blockIdx.x == 0) {
        // The pages this plan takes (the front of the device free list) must be the ones the host
        // ledger's reservation took: a difference means the two copies of the free list diverged.
        // It is reported, not fatal here: the metadata below is still complete and consistent
        // with the device list, and the step report fails the step on the host.
        int differ = 0;
        if (expect_pages)
            for (int j = r; j < total_miss; j += kPlanThreads) differ |= free_pages[j] != expect_pages[j];
        differ = __syncthreads_or(differ);
        if (r == 0) {
            status[0] = differ ? NQ_ERR_STATE : NQ_OK;
            status[1] = total_miss;
        }
    }

    if (blockIdx.x == 0 && r < capture_rows) {
        kv_indptr[r + 1] = page_off + npages;
        if (r == 0) kv_indptr[0] = 0;
        if (r < n_rows) {
            const int rem = total % page_size;
            last_page_len[r] = rem ? rem : page_size;
        } else {
            last_page_len[r] = 1;
        }
        if (prefill) {
            // padding rows add no queries
            qo_indptr[r + 1] = (r < n_rows) ? tok_off + ntok : sum_adv;
            if (r == 0) qo_indptr[0] = 0;
        }
    }

    const int64_t gstride = static_cast<int64_t>(gridDim.x) * blockDim.x;
    const int64_t gid = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;

    // Page list: prior pages, then the row's slice of the sorted free list.
    for (int64_t j = gid; j < total_pages; j += gstride) {
        const int row = find_row(s_page_off, capture_rows, static_cast<int>(j));
        const int i = static_cast<int>(j) - s_page_off[row];
        int page;
        if (row < n_rows) {
            const int prior = s_prior[row];
            int32_t *trow = page_table + static_cast<int64_t>(s_trow[row]) * table_stride;
            if (i < prior) {
                page = trow[i];
            } else {
                page = free_pages[s_miss_off[row] + (i - prior)];
                trow[i] = page;  // proposed pages; harmless if the publication is discarded
            }
        } else {
            page = scratch_pages[row];
        }
        kv_indices[j] = page;
    }

    // Per-token write slots and positions.
    for (int64_t t = gid; t < token_capacity; t += gstride) {
        int64_t wpage, woff, pos;
        if (t < total_tok) {
            const int row = find_row(s_tok_off, capture_rows, static_cast<int>(t));
            const int o = static_cast<int>(t) - s_tok_off[row];
            if (row < n_rows) {
                const int abs_pos = s_seq[row] + o;
                const int pidx = abs_pos / page_size;
                const int prior = s_prior[row];
                if (pidx < prior)
                    wpage = page_table[static_cast<int64_t>(s_trow[row]) * table_stride + pidx];
                else
                    wpage = free_pages[s_miss_off[row] + (pidx - prior)];
                woff = abs_pos % page_size;
                pos = static_cast<int64_t>(s_pos[row]) + o;
            } else {  // decode padding row: scratch slot 0 of its own page
                wpage = scratch_pages[row];
                woff = 0;
                pos = 0;
            }
        } else {  // padding tokens walk the scratch slots after the real tokens
            const int64_t slot = t - sum_adv;
            wpage = scratch_pages[slot / page_size];
            woff = slot % page_size;
            pos = 0;
        }
        position_ids[t] = pos;
        write_pages[t] = wpage;
        write_offsets[t] = woff;
    }
}

}  // namespace
}  // namespace nq

extern "C" int nq_plan_ragged(const int32_t *seq_len, const int32_t *pos_start,
                              const int32_t *advance, const int32_t *prior_pages,
                              const int32_t *table_row, int n_rows, int capture_rows,
                              int token_capacity, int page_size, int prefill,
                              int32_t *page_table, int64_t table_stride,
                              const int32_t *free_pages, int n_free, const int32_t *expect_pages,
                              const int32_t *scratch_pages, int n_scratch,
                              int32_t *qo_indptr, int32_t *kv_indptr, int32_t *kv_indices,
                              int64_t kv_indices_capacity, int32_t *last_page_len,
                              int64_t *position_ids, int64_t *write_pages,
                              int64_t *write_offsets, int32_t *status, int grid_blocks,
                              void *stream) {
    NQ_CHECK_ARG(n_rows >= 1 && n_rows <= capture_rows);
    if (capture_rows > nq::kPlanThreads) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(page_size >= 1 && token_capacity >= 1 && n_free >= 0);
    // Scratch capacity rule of PagedTalkerKV._validate_scratch_capacity (talker_kv.py:397-401).
    NQ_CHECK_ARG(capture_rows <= n_scratch);
    NQ_CHECK_ARG(static_cast<int64_t>(token_capacity) <= static_cast<int64_t>(n_scratch) * page_size);
    NQ_CHECK_ARG(seq_len && pos_start && advance && prior_pages && table_row && page_table);
    NQ_CHECK_ARG(scratch_pages && kv_indptr && kv_indices && last_page_len && status);
    NQ_CHECK_ARG(position_ids && write_pages && write_offsets && table_stride >= 1);
    NQ_CHECK_ARG(!prefill || qo_indptr);
    NQ_CHECK_ARG(n_free == 0 || free_pages);
    int grid = grid_blocks > 0 ? grid_blocks : 8;
    hipLaunchKernelGGL(nq::plan_ragged_kernel, dim3(grid), dim3(nq::kPlanThreads), 0,
                       static_cast<hipStream_t>(stream), seq_len, pos_start, advance,
                       prior_pages, table_row, n_rows, capture_rows, token_capacity, page_size,
                       prefill, page_table, table_stride, free_pages, n_free, expect_pages, scratch_pages,
                       qo_indptr, kv_indptr, kv_indices, kv_indices_capacity, last_page_len,
                       position_ids, write_pages, write_offsets, status);
    return NQ_LAUNCH_STATUS();
}

namespace nq {
namespace {

constexpr int kMergeThreads = 256;

// Number of elements of the sorted array v[0, n) that are smaller than x.
__device__ __forceinline__ int count_below(const int32_t *v, int n, int32_t x) {
    int lo = 0, hi = n;
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (v[mid] < x) lo = mid + 1; else hi = mid;
    }
    return lo;
}

// out = the sorted union of a[0, na) and b[0, nb) (both sorted, distinct): every element finds
// its output position by one binary search in the other list.  A page present in both lists is
// reported as NQ_ERR_INVALID_ARGUMENT (it would be handed out twice).
__global__ void __launch_bounds__(kMergeThreads)
free_list_merge_kernel(const int32_t *__restrict__ a, int na, const int32_t *__restrict__ b, int nb,
                       int32_t *__restrict__ out, int32_t *__restrict__ status) {
    const int i = blockIdx.x * kMergeThreads + threadIdx.x;
    if (i < na) {
        const int32_t v = a[i];
        out[i + count_below(b, nb, v)] = v;
    } else if (i < na + nb) {
        const int j = i - na;
        const int32_t v = b[j];
        const int below = count_below(a, na, v);
        if (below < na && a[below] == v) {
            if (status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
            return;
        }
        out[j + below] = v;
    }
}

// One decode step's report: the planner status (written by every planner launch), then the
// free-list merge, attention and embedding status words (each read, then cleared for the next
// step), the number of tokens outside [0, vocab), and per row whether the token is the
// end-of-speech id.
__global__ void __launch_bounds__(kMergeThreads)
step_report_kernel(const int32_t *__restrict__ plan_status, int32_t *__restrict__ merge_status,
                   int32_t *__restrict__ attention_status, int32_t *__restrict__ embed_status,
                   const int64_t *__restrict__ tokens, int rows, int64_t eos_id, int64_t vocab,
                   int32_t *__restrict__ report) {
    __shared__ int s_bad;
    if (threadIdx.x == 0) s_bad = 0;
    __syncthreads();
    int bad = 0;
    for (int r = threadIdx.x; r < rows; r += kMergeThreads) {
        const int64_t t = tokens[r];
        bad += (t < 0 || t >= vocab) ? 1 : 0;
        report[NQ_REPORT_HEAD + r] = t == eos_id ? 1 : 0;
    }
    if (bad) atomicAdd(&s_bad, bad);
    __syncthreads();
    if (threadIdx.x == 0) {
        int32_t *cleared[3] = {merge_status, attention_status, embed_status};
        report[0] = plan_status ? plan_status[0] : NQ_OK;
        for (int i = 0; i < 3; ++i) {
            report[1 + i] = cleared[i] ? cleared[i][0] : NQ_OK;
            if (cleared[i]) cleared[i][0] = NQ_OK;
        }
        report[4] = s_bad;
        for (int i = 5; i < NQ_REPORT_HEAD; ++i) report[i] = 0;
    }
}

}  // namespace
}  // namespace nq

extern "C" int nq_free_list_merge(const int32_t *free_pages, int n_free, const int32_t *returned, int n_returned,
                                  int32_t *out, int32_t *status, void *stream) {
    NQ_CHECK_ARG(n_free >= 0 && n_returned >= 0 && out);
    NQ_CHECK_ARG((n_free == 0 || free_pages) && (n_returned == 0 || returned));
    const int n = n_free + n_returned;
    if (n == 0) return NQ_OK;
    hipLaunchKernelGGL(nq::free_list_merge_kernel, dim3((n + nq::kMergeThreads - 1) / nq::kMergeThreads),
                       dim3(nq::kMergeThreads), 0, static_cast<hipStream_t>(stream), free_pages, n_free, returned,
                       n_returned, out, status);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_step_report(const int32_t *plan_status, int32_t *merge_status, int32_t *attention_status,
                              int32_t *embed_status, const int64_t *tokens, int rows, int64_t eos_id, int64_t vocab,
                              int32_t *report, void *stream) {
    NQ_CHECK_ARG(tokens && report && rows >= 1 && vocab >= 1);
    hipLaunchKernelGGL(nq::step_report_kernel, dim3(1), dim3(nq::kMergeThreads), 0,
                       static_cast<hipStream_t>(stream), plan_status, merge_status, attention_status, embed_status,
                       tokens, rows, eos_id, vocab, report);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_abi_version(void) { return NQ_ABI_VERSION; }

extern "C" const char *nq_status_string(int status) {
    switch (status) {
        case NQ_OK: return "ok";
        case NQ_ERR_INVALID_ARGUMENT: return "invalid argument";
        case NQ_ERR_UNSUPPORTED: return "unsupported dtype or size";
        case NQ_ERR_LAUNCH: return "HIP launch failure";
        case NQ_ERR_CAPACITY: return "not enough free KV pages";
        case NQ_ERR_STATE: return "device KV state differs from the host ledger";
        default: return "unknown status";
    }
}
