// Paged GQA attention over the talker's paged KV cache, and the code
// predictor's dense short-cache attention.
//
// Work unit: one (query token, key chunk, kv head) item per workgroup of 4
// waves.  Each wave streams 16-token blocks of K and V straight from HBM with
// 128-bit loads (D/8 lanes cover one 256-byte K or V row, so one load
// instruction moves 1 KiB of a page), keeps an online softmax per lane group
// and, at the end of the chunk, the waves combine through LDS.  Items of the
// same query are merged by the workgroup that finishes last (an arrival
// counter per (query, kv head), reset by that workgroup), so a step needs one
// launch per layer and no separate reduction kernel.
//
// Semantics follow FlashInfer's paged decode/prefill as bound in
// executor/talker_kv.py:140-306 (scale 1/sqrt(D), fp32 softmax and
// accumulation, bf16 output), the bottom-right causal rule of
// BatchPrefillWithPagedKVCacheWrapper(causal=True) (talker_kv.py:218) and the
// short-cache kernel of model/kernels.py:408-463.
#include "nq_common.h"

namespace nq {
namespace {

constexpr int kAttnThreads = 256;
constexpr int kWaves = kAttnThreads / kWave;
constexpr int kBlockTok = 16;        // tokens per wave iteration
constexpr int kTargetItems = 8192;   // preferred upper bound on chunk items per launch
constexpr int kPpcCandidates = 14;   // pages per chunk in {1, 2, ..., 8192}
constexpr int kPlanThreads = 1024;   // rows per plan launch (largest bucket)
constexpr int kMinChunkTokens = 64;

enum MetaSlot { kMetaChunks = 0, kMetaPpc = 1, kMetaStatus = 2, kMetaQueries = 3 };

struct PlanLayout {
    int64_t meta, chunk_indptr, q_row, q_kvlen, counters, part_ml, part_o, total;
    int64_t max_chunks;
};

__host__ __device__ inline int64_t align256(int64_t x) { return (x + 255) & ~int64_t(255); }

__host__ __device__ inline int64_t chunk_capacity(int T, int max_pages, int Hkv) {
    return 2 * static_cast<int64_t>(T) + kTargetItems / Hkv + max_pages / 64 + 64;
}

__host__ __device__ inline PlanLayout plan_layout(int T, int max_pages, int Hq, int Hkv, int D) {
    PlanLayout L;
    L.max_chunks = chunk_capacity(T, max_pages, Hkv);
    int64_t off = 0;
    L.meta = off;         off = align256(off + 8 * 4);
    L.chunk_indptr = off; off = align256(off + (static_cast<int64_t>(T) + 1) * 4);
    L.q_row = off;        off = align256(off + static_cast<int64_t>(T) * 4);
    L.q_kvlen = off;      off = align256(off + static_cast<int64_t>(T) * 4);
    L.counters = off;     off = align256(off + static_cast<int64_t>(T) * Hkv * 4);
    L.part_ml = off;      off = align256(off + L.max_chunks * Hq * 2 * 4);
    L.part_o = off;       off = align256(off + L.max_chunks * Hq * D * 4);
    L.total = off;
    return L;
}

__device__ __forceinline__ int ilog2_exact(int x) { return 31 - __clz(x); }

__device__ int plan_block_scan(int v, int *tmp, int *total) {
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    int incl = v;
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1) {
        int o = __shfl_up(incl, d, kWave);
        if (lane >= d) incl += o;
    }
    if (lane == kWave - 1) tmp[wave] = incl;
    __syncthreads();
    if (wave == 0) {
        const int nw = blockDim.x / kWave;
        int w = lane < nw ? tmp[lane] : 0;
        int wi = w;
#pragma unroll
        for (int d = 1; d < kWave; d <<= 1) {
            int o = __shfl_up(wi, d, kWave);
            if (lane >= d) wi += o;
        }
        if (lane < nw) tmp[lane] = wi - w;
        if (lane == nw - 1) tmp[kWave] = wi;
    }
    __syncthreads();
    const int res = tmp[wave] + incl - v;
    *total = tmp[kWave];
    __syncthreads();
    return res;
}

// One workgroup: per query token its row, causal key count and chunk range.
__global__ void __launch_bounds__(kPlanThreads)
attention_plan_kernel(const int32_t *__restrict__ qo_indptr, const int32_t *__restrict__ kv_indptr,
                      const int32_t *__restrict__ last_page_len, int n_rows, int max_queries,
                      int page_size, int num_kv_heads, int64_t max_chunks, char *__restrict__ ws,
                      PlanLayout L) {
    __shared__ int s_qo[kPlanThreads + 1];
    __shared__ int s_kvlen[kPlanThreads];
    __shared__ unsigned long long s_cand[kPpcCandidates];
    __shared__ int s_tmp[kWave + 1];

    int32_t *meta = reinterpret_cast<int32_t *>(ws + L.meta);
    int32_t *chunk_indptr = reinterpret_cast<int32_t *>(ws + L.chunk_indptr);
    int32_t *q_row = reinterpret_cast<int32_t *>(ws + L.q_row);
    int32_t *q_kvlen = reinterpret_cast<int32_t *>(ws + L.q_kvlen);
    int32_t *counters = reinterpret_cast<int32_t *>(ws + L.counters);

    const int tid = threadIdx.x;
    if (tid < n_rows) {
        const int np = kv_indptr[tid + 1] - kv_indptr[tid];
        int last = last_page_len[tid];
        last = last < 1 ? 1 : (last > page_size ? page_size : last);  // keys stay inside the row's pages
        s_kvlen[tid] = np > 0 ? (np - 1) * page_size + last : 0;
        s_qo[tid] = qo_indptr ? qo_indptr[tid] : tid;
    }
    if (tid == 0) s_qo[n_rows] = qo_indptr ? qo_indptr[n_rows] : n_rows;
    if (tid < kPpcCandidates) s_cand[tid] = 0;
    __syncthreads();
    const int T = s_qo[n_rows];
    if (T < 0 || T > max_queries) {
        if (tid == 0) {
            meta[kMetaChunks] = 0;
            meta[kMetaPpc] = 1;
            meta[kMetaStatus] = NQ_ERR_INVALID_ARGUMENT;
            meta[kMetaQueries] = 0;
        }
        return;
    }

    // Causal pages of query q.
    auto query_pages = [&](int q, int *row_out, int *kvlen_out) {
        int lo = 0, hi = n_rows;
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (s_qo[mid] <= q) lo = mid; else hi = mid;
        }
        const int qo_len = s_qo[lo + 1] - s_qo[lo];
        int kvlen = s_kvlen[lo] - qo_len + (q - s_qo[lo]) + 1;
        kvlen = kvlen < 0 ? 0 : (kvlen > s_kvlen[lo] ? s_kvlen[lo] : kvlen);
        *row_out = lo;
        *kvlen_out = kvlen;
        return (kvlen + page_size - 1) / page_size;
    };

    // Pass 1: chunk totals for every candidate chunk size.
    unsigned long long cand[kPpcCandidates];
#pragma unroll
    for (int c = 0; c < kPpcCandidates; ++c) cand[c] = 0;
    for (int q = tid; q < T; q += blockDim.x) {
        int row, kvlen;
        const int pages = query_pages(q, &row, &kvlen);
#pragma unroll
        for (int c = 0; c < kPpcCandidates; ++c) {
            const int n = (pages + (1 << c) - 1) >> c;
            cand[c] += n > 0 ? n : 1;
        }
    }
#pragma unroll
    for (int c = 0; c < kPpcCandidates; ++c) atomicAdd(&s_cand[c], cand[c]);
    __syncthreads();

    const int min_tokens = kMinChunkTokens > page_size ? kMinChunkTokens : page_size;
    int ppc_log = 0;
    while ((page_size << ppc_log) < min_tokens && ppc_log < kPpcCandidates - 1) ++ppc_log;
    int chosen = -1;
    for (int c = ppc_log; c < kPpcCandidates; ++c)
        if (s_cand[c] * num_kv_heads <= kTargetItems) { chosen = c; break; }
    if (chosen < 0)
        for (int c = ppc_log; c < kPpcCandidates; ++c)
            if (s_cand[c] <= static_cast<unsigned long long>(max_chunks)) { chosen = c; break; }
    if (chosen < 0) {
        if (tid == 0) {
            meta[kMetaChunks] = 0;
            meta[kMetaPpc] = 1;
            meta[kMetaStatus] = NQ_ERR_CAPACITY;
            meta[kMetaQueries] = 0;
        }
        return;
    }

    // Pass 2: chunk prefix per query.
    int carry = 0;
    for (int base = 0; base < T; base += blockDim.x) {
        const int q = base + tid;
        int n = 0, row = 0, kvlen = 0;
        if (q < T) {
            const int pages = query_pages(q, &row, &kvlen);
            n = (pages + (1 << chosen) - 1) >> chosen;
            if (n < 1) n = 1;
        }
        int total;
        const int excl = plan_block_scan(n, s_tmp, &total);
        if (q < T) {
            chunk_indptr[q] = carry + excl;
            q_row[q] = row;
            q_kvlen[q] = kvlen;
        }
        carry += total;
    }
    for (int i = tid; i < T * num_kv_heads; i += blockDim.x) counters[i] = 0;
    if (tid == 0) {
        chunk_indptr[T] = carry;
        meta[kMetaChunks] = carry;
        meta[kMetaPpc] = 1 << chosen;
        meta[kMetaStatus] = NQ_OK;
        meta[kMetaQueries] = T;
    }
}

// Where the keys of one work item live.
struct PagedSource {
    const int32_t *kv_indices;
    int page_base;
    int ps_log2;
    int num_pages;
    __device__ __forceinline__ int page_of(int tok) const {
        return kv_indices[page_base + (tok >> ps_log2)];
    }
    __device__ __forceinline__ int slot_of(int tok) const { return tok & ((1 << ps_log2) - 1); }
};

struct DenseSource {
    int row;
    __device__ __forceinline__ int page_of(int) const { return row; }
    __device__ __forceinline__ int slot_of(int tok) const { return tok; }
};

struct Smem {
    float m[kWaves][8];
    float l[kWaves][8];
    float acc[kWaves][8][128];
    int flag;
};

// Attend one query token (G consecutive query heads of kv head h) to the keys
// [tok_begin, tok_end).  Leaves the combined (m, l, acc) of the workgroup for
// output element t = j*D + d in *m_out/*l_out/*o_out of the calling thread
// (threads t < G*D; larger G*D handled by the caller's loop).
template <int D, int G, typename Src>
__device__ __forceinline__ void attend_chunk(const uint16_t *__restrict__ qptr, int64_t q_s1,
                                             const uint16_t *__restrict__ cache, int64_t c_page,
                                             int64_t c_kind, int64_t c_slot, int64_t c_head,
                                             int h, int tok_begin, int tok_end, int page_limit,
                                             float scale_log2, const Src &src, Smem &sm,
                                             int32_t *status) {
    constexpr int LPT = D / 8;            // lanes per 256/128-byte row
    constexpr int TPL = kWave / LPT;      // tokens per load instruction
    constexpr int NL = kBlockTok / TPL;   // loads per block per K or V
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int g = lane / LPT;
    const int sub = lane % LPT;

    float qv[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const uint4 p = *reinterpret_cast<const uint4 *>(qptr + (h * G + j) * q_s1 + sub * 8);
        unpack8(p, qv[j]);
#pragma unroll
        for (int e = 0; e < 8; ++e) qv[j][e] *= scale_log2;
    }
    float m[G], l[G], acc[G][8];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        m[j] = -INFINITY;
        l[j] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[j][e] = 0.f;
    }

    const uint16_t *head_base = cache + h * c_head + sub * 8;
    const int ntok = tok_end - tok_begin;
    const int nblk = ntok > 0 ? (ntok + kBlockTok - 1) / kBlockTok : 0;
    bool bad_page = false;
    for (int b = wave; b < nblk; b += kWaves) {
        const int tb = tok_begin + b * kBlockTok;
        uint4 kr[NL], vr[NL];
        bool valid[NL];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            const int tok = tb + i * TPL + g;
            valid[i] = tok < tok_end;
            kr[i] = make_uint4(0, 0, 0, 0);
            vr[i] = make_uint4(0, 0, 0, 0);
            if (valid[i]) {
                const int page = src.page_of(tok);
                if (static_cast<unsigned>(page) < static_cast<unsigned>(page_limit)) {
                    const uint16_t *p = head_base + page * c_page + src.slot_of(tok) * c_slot;
                    kr[i] = *reinterpret_cast<const uint4 *>(p);
                    vr[i] = *reinterpret_cast<const uint4 *>(p + c_kind);
                } else {
                    valid[i] = false;
                    bad_page = true;
                }
            }
        }
        float s[NL][G];
#pragma unroll
        for (int i = 0; i < NL; ++i) {
            float kf[8];
            unpack8(kr[i], kf);
#pragma unroll
            for (int j = 0; j < G; ++j) {
                float part = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) part += qv[j][e] * kf[e];
                part = group_sum<LPT>(part);
                s[i][j] = valid[i] ? part : -INFINITY;
            }
        }
#pragma unroll
        for (int j = 0; j < G; ++j) {
            float mb = s[0][j];
#pragma unroll
            for (int i = 1; i < NL; ++i) mb = fmaxf(mb, s[i][j]);
            const float mn = fmaxf(m[j], mb);
            if (mn == -INFINITY) continue;
            const float alpha = exp2f(m[j] - mn);
            m[j] = mn;
            l[j] *= alpha;
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[j][e] *= alpha;
#pragma unroll
            for (int i = 0; i < NL; ++i) {
                const float p = exp2f(s[i][j] - mn);
                l[j] += p;
                float vf[8];
                unpack8(vr[i], vf);
#pragma unroll
                for (int e = 0; e < 8; ++e) acc[j][e] += p * vf[e];
            }
        }
    }
    if (bad_page && status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);

    // Combine the lane groups of the wave (lanes sub, sub+LPT, ...).
#pragma unroll
    for (int mask = LPT; mask < kWave; mask <<= 1) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            const float mo = __shfl_xor(m[j], mask, kWave);
            const float lo = __shfl_xor(l[j], mask, kWave);
            const float mn = fmaxf(m[j], mo);
            const float a = m[j] == -INFINITY ? 0.f : exp2f(m[j] - mn);
            const float bsc = mo == -INFINITY ? 0.f : exp2f(mo - mn);
            l[j] = l[j] * a + lo * bsc;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float ao = __shfl_xor(acc[j][e], mask, kWave);
                acc[j][e] = acc[j][e] * a + ao * bsc;
            }
            m[j] = mn;
        }
    }
    if (g == 0) {
#pragma unroll
        for (int j = 0; j < G; ++j) {
            if (sub == 0) {
                sm.m[wave][j] = m[j];
                sm.l[wave][j] = l[j];
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) sm.acc[wave][j][sub * 8 + e] = acc[j][e];
        }
    }
    __syncthreads();
}

// Combine the per-wave states in shared memory for output element t = j*D+d.
template <int D>
__device__ __forceinline__ void wave_combine(const Smem &sm, int t, float *M, float *Lsum,
                                             float *O) {
    const int j = t / D, d = t % D;
    float mx = -INFINITY;
#pragma unroll
    for (int w = 0; w < kWaves; ++w) mx = fmaxf(mx, sm.m[w][j]);
    float ls = 0.f, os = 0.f;
    if (mx != -INFINITY) {
#pragma unroll
        for (int w = 0; w < kWaves; ++w) {
            const float mw = sm.m[w][j];
            const float sc = mw == -INFINITY ? 0.f : exp2f(mw - mx);
            ls += sm.l[w][j] * sc;
            os += sm.acc[w][j][d] * sc;
        }
    }
    *M = mx;
    *Lsum = ls;
    *O = os;
}

template <int D, int G>
__global__ void __launch_bounds__(kAttnThreads)
paged_decode_kernel(const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1,
                    const uint16_t *__restrict__ cache, int64_t c_page, int64_t c_kind,
                    int64_t c_slot, int64_t c_head, int num_pages,
                    const int32_t *__restrict__ kv_indptr, const int32_t *__restrict__ kv_indices,
                    int num_kv_heads, int ps_log2, float scale_log2, uint16_t *__restrict__ out,
                    int64_t o_s0, int64_t o_s1, char *__restrict__ ws, PlanLayout L,
                    int32_t *status) {
    __shared__ Smem sm;
    const int32_t *meta = reinterpret_cast<const int32_t *>(ws + L.meta);
    const int32_t *chunk_indptr = reinterpret_cast<const int32_t *>(ws + L.chunk_indptr);
    const int32_t *q_row = reinterpret_cast<const int32_t *>(ws + L.q_row);
    const int32_t *q_kvlen = reinterpret_cast<const int32_t *>(ws + L.q_kvlen);
    int32_t *counters = reinterpret_cast<int32_t *>(ws + L.counters);
    float *part_ml = reinterpret_cast<float *>(ws + L.part_ml);
    float *part_o = reinterpret_cast<float *>(ws + L.part_o);
    if (meta[kMetaStatus] != NQ_OK) return;
    const int n_chunks = meta[kMetaChunks];
    const int T = meta[kMetaQueries];
    const int chunk_tok = meta[kMetaPpc] << ps_log2;
    const int Hq = num_kv_heads * G;
    const int64_t n_items = static_cast<int64_t>(n_chunks) * num_kv_heads;

    for (int64_t w = blockIdx.x; w < n_items; w += gridDim.x) {
        const int c = static_cast<int>(w / num_kv_heads);
        const int h = static_cast<int>(w - static_cast<int64_t>(c) * num_kv_heads);
        int lo = 0, hi = T;  // query owning chunk c
        while (hi - lo > 1) {
            const int mid = (lo + hi) >> 1;
            if (chunk_indptr[mid] <= c) lo = mid; else hi = mid;
        }
        const int qi = lo;
        const int c0 = chunk_indptr[qi];
        const int nk = chunk_indptr[qi + 1] - c0;
        const int row = q_row[qi];
        const int kvlen = q_kvlen[qi];
        const int tok_begin = (c - c0) * chunk_tok;
        const int tok_end = min(kvlen, tok_begin + chunk_tok);
        PagedSource src{kv_indices, kv_indptr[row], ps_log2, num_pages};
        attend_chunk<D, G>(q + qi * q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, h,
                           tok_begin, tok_end, num_pages, scale_log2, src, sm, status);
        if (nk == 1) {
            for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
                float M, Ls, O;
                wave_combine<D>(sm, t, &M, &Ls, &O);
                const int j = t / D, d = t % D;
                out[qi * o_s0 + (h * G + j) * o_s1 + d] = f32_to_bf16(Ls > 0.f ? O / Ls : 0.f);
            }
        } else {
            for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
                float M, Ls, O;
                wave_combine<D>(sm, t, &M, &Ls, &O);
                const int j = t / D, d = t % D;
                const int64_t hh = static_cast<int64_t>(c) * Hq + h * G + j;
                part_o[hh * D + d] = O;
                if (d == 0) {
                    part_ml[hh * 2] = M;
                    part_ml[hh * 2 + 1] = Ls;
                }
            }
            __threadfence();
            __syncthreads();
            if (threadIdx.x == 0) {
                const int prev = atomicAdd(&counters[qi * num_kv_heads + h], 1);
                sm.flag = (prev == nk - 1);
            }
            __syncthreads();
            if (sm.flag) {
                __threadfence();
                for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
                    const int j = t / D, d = t % D;
                    float mx = -INFINITY;
                    for (int k = 0; k < nk; ++k)
                        mx = fmaxf(mx, part_ml[(static_cast<int64_t>(c0 + k) * Hq + h * G + j) * 2]);
                    float ls = 0.f, os = 0.f;
                    if (mx != -INFINITY) {
                        for (int k = 0; k < nk; ++k) {
                            const int64_t hh = static_cast<int64_t>(c0 + k) * Hq + h * G + j;
                            const float mk = part_ml[hh * 2];
                            const float sc = mk == -INFINITY ? 0.f : exp2f(mk - mx);
                            ls += part_ml[hh * 2 + 1] * sc;
                            os += part_o[hh * D + d] * sc;
                        }
                    }
                    out[qi * o_s0 + (h * G + j) * o_s1 + d] = f32_to_bf16(ls > 0.f ? os / ls : 0.f);
                }
                if (threadIdx.x == 0) atomicExch(&counters[qi * num_kv_heads + h], 0);
            }
        }
        __syncthreads();
    }
}

template <int D, int G>
__global__ void __launch_bounds__(kAttnThreads)
dense_short_kernel(const uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1,
                   const uint16_t *__restrict__ cache, int64_t c_row, int64_t c_kind, int64_t c_pos,
                   int64_t c_head, int rows, int valid_length, int num_kv_heads, float scale_log2,
                   uint16_t *__restrict__ out, int64_t o_s0, int64_t o_s1) {
    __shared__ Smem sm;
    const int64_t n_items = static_cast<int64_t>(rows) * num_kv_heads;
    for (int64_t w = blockIdx.x; w < n_items; w += gridDim.x) {
        const int row = static_cast<int>(w / num_kv_heads);
        const int h = static_cast<int>(w - static_cast<int64_t>(row) * num_kv_heads);
        DenseSource src{row};
        attend_chunk<D, G>(q + row * q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head, h, 0,
                           valid_length, rows, scale_log2, src, sm, nullptr);
        for (int t = threadIdx.x; t < G * D; t += kAttnThreads) {
            float M, Ls, O;
            wave_combine<D>(sm, t, &M, &Ls, &O);
            const int j = t / D, d = t % D;
            out[row * o_s0 + (h * G + j) * o_s1 + d] = f32_to_bf16(Ls > 0.f ? O / Ls : 0.f);
        }
        __syncthreads();
    }
}

constexpr float kLog2e = 1.4426950408889634f;

template <int D, int G>
int launch_paged(const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                 int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head, int num_pages,
                 const int32_t *kv_indptr, const int32_t *kv_indices, int Hkv, int ps_log2,
                 float scale, uint16_t *out, int64_t o_s0, int64_t o_s1, char *ws,
                 const PlanLayout &L, int32_t *status, hipStream_t stream) {
    int64_t items = L.max_chunks * Hkv;
    int grid = static_cast<int>(items < 4096 ? items : 4096);
    if (grid < 1) grid = 1;
    hipLaunchKernelGGL((paged_decode_kernel<D, G>), dim3(grid), dim3(kAttnThreads), 0, stream, q,
                       q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head, num_pages, kv_indptr,
                       kv_indices, Hkv, ps_log2, scale * kLog2e, out, o_s0, o_s1, ws, L, status);
    return NQ_LAUNCH_STATUS();
}

template <int D, int G>
int launch_dense(const uint16_t *q, int64_t q_s0, int64_t q_s1, const uint16_t *cache,
                 int64_t c_row, int64_t c_kind, int64_t c_pos, int64_t c_head, int rows,
                 int valid_length, int Hkv, float scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                 hipStream_t stream) {
    int64_t items = static_cast<int64_t>(rows) * Hkv;
    int grid = static_cast<int>(items < 8192 ? items : 8192);
    hipLaunchKernelGGL((dense_short_kernel<D, G>), dim3(grid), dim3(kAttnThreads), 0, stream, q,
                       q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head, rows, valid_length, Hkv,
                       scale * kLog2e, out, o_s0, o_s1);
    return NQ_LAUNCH_STATUS();
}

bool aligned16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace nq

using nq::PlanLayout;

extern "C" int64_t nq_attention_workspace_bytes(int max_query_tokens, int max_pages, int page_size,
                                                int num_qo_heads, int num_kv_heads, int head_dim) {
    if (max_query_tokens < 1 || max_pages < 1 || page_size < 1 || num_kv_heads < 1 ||
        num_qo_heads < num_kv_heads || head_dim < 8)
        return NQ_ERR_INVALID_ARGUMENT;
    return nq::plan_layout(max_query_tokens, max_pages, num_qo_heads, num_kv_heads, head_dim).total;
}

extern "C" int nq_attention_plan(const int32_t *qo_indptr, const int32_t *kv_indptr,
                                 const int32_t *last_page_len, int n_rows, int max_query_tokens,
                                 int max_pages, int page_size, int num_qo_heads, int num_kv_heads,
                                 int head_dim, void *workspace, int64_t workspace_bytes,
                                 void *stream) {
    NQ_CHECK_ARG(n_rows >= 1 && max_query_tokens >= 1 && max_pages >= 1);
    if (n_rows > nq::kPlanThreads) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(page_size >= 1 && (page_size & (page_size - 1)) == 0);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    NQ_CHECK_ARG(kv_indptr && last_page_len && workspace);
    NQ_CHECK_ARG(qo_indptr || n_rows <= max_query_tokens);
    const PlanLayout L =
        nq::plan_layout(max_query_tokens, max_pages, num_qo_heads, num_kv_heads, head_dim);
    NQ_CHECK_ARG(workspace_bytes >= L.total);
    hipLaunchKernelGGL(nq::attention_plan_kernel, dim3(1), dim3(nq::kPlanThreads), 0,
                       static_cast<hipStream_t>(stream), qo_indptr, kv_indptr, last_page_len,
                       n_rows, max_query_tokens, page_size, num_kv_heads, L.max_chunks,
                       static_cast<char *>(workspace), L);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_paged_attention(const uint16_t *q, int64_t q_s0, int64_t q_s1,
                                  const uint16_t *cache, int64_t c_page, int64_t c_kind,
                                  int64_t c_slot, int64_t c_head, int num_pages,
                                  const int32_t *kv_indptr, const int32_t *kv_indices,
                                  int page_size, int num_qo_heads, int num_kv_heads, int head_dim,
                                  float sm_scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                                  int max_query_tokens, int max_pages, void *workspace,
                                  int64_t workspace_bytes, int32_t *status, void *stream) {
    NQ_CHECK_ARG(q && cache && kv_indptr && kv_indices && out && workspace);
    NQ_CHECK_ARG(page_size >= 1 && (page_size & (page_size - 1)) == 0 && num_pages >= 1);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    NQ_CHECK_ARG(max_query_tokens >= 1 && max_pages >= 1);
    if (!nq::aligned16(q) || !nq::aligned16(cache) || !nq::aligned16(out)) return NQ_ERR_UNSUPPORTED;
    if ((q_s0 | q_s1 | c_page | c_kind | c_slot | c_head) & 7) return NQ_ERR_UNSUPPORTED;
    const PlanLayout L =
        nq::plan_layout(max_query_tokens, max_pages, num_qo_heads, num_kv_heads, head_dim);
    NQ_CHECK_ARG(workspace_bytes >= L.total);
    int ps_log2 = 0;
    while ((1 << ps_log2) < page_size) ++ps_log2;
    const int G = num_qo_heads / num_kv_heads;
    hipStream_t s = static_cast<hipStream_t>(stream);
    char *ws = static_cast<char *>(workspace);
#define NQ_PAGED(DD, GG)                                                                          \
    if (head_dim == DD && G == GG)                                                                \
        return nq::launch_paged<DD, GG>(q, q_s0, q_s1, cache, c_page, c_kind, c_slot, c_head,     \
                                        num_pages, kv_indptr, kv_indices, num_kv_heads, ps_log2,  \
                                        sm_scale, out, o_s0, o_s1, ws, L, status, s);
    NQ_PAGED(128, 1) NQ_PAGED(128, 2) NQ_PAGED(128, 4) NQ_PAGED(128, 8)
    NQ_PAGED(64, 1) NQ_PAGED(64, 2) NQ_PAGED(64, 4) NQ_PAGED(64, 8)
#undef NQ_PAGED
    return NQ_ERR_UNSUPPORTED;
}

extern "C" int nq_cp_short_attention(const uint16_t *q, int64_t q_s0, int64_t q_s1,
                                     const uint16_t *cache, int64_t c_row, int64_t c_kind,
                                     int64_t c_pos, int64_t c_head, int rows, int valid_length,
                                     int num_qo_heads, int num_kv_heads, int head_dim,
                                     float sm_scale, uint16_t *out, int64_t o_s0, int64_t o_s1,
                                     void *stream) {
    NQ_CHECK_ARG(q && cache && out && rows >= 1 && valid_length >= 1);
    NQ_CHECK_ARG(num_kv_heads >= 1 && num_qo_heads % num_kv_heads == 0);
    if (!nq::aligned16(q) || !nq::aligned16(cache) || !nq::aligned16(out)) return NQ_ERR_UNSUPPORTED;
    if ((q_s0 | q_s1 | c_row | c_kind | c_pos | c_head) & 7) return NQ_ERR_UNSUPPORTED;
    const int G = num_qo_heads / num_kv_heads;
    hipStream_t s = static_cast<hipStream_t>(stream);
#define NQ_DENSE(DD, GG)                                                                         \
    if (head_dim == DD && G == GG)                                                               \
        return nq::launch_dense<DD, GG>(q, q_s0, q_s1, cache, c_row, c_kind, c_pos, c_head, rows, \
                                        valid_length, num_kv_heads, sm_scale, out, o_s0, o_s1, s);
    NQ_DENSE(128, 1) NQ_DENSE(128, 2) NQ_DENSE(128, 4) NQ_DENSE(128, 8)
    NQ_DENSE(64, 1) NQ_DENSE(64, 2) NQ_DENSE(64, 4) NQ_DENSE(64, 8)
#undef NQ_DENSE
    return NQ_ERR_UNSUPPORTED;
}
