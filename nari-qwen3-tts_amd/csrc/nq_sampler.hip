// Fused sampler: logit masks, repetition penalty, temperature, top-k, top-p
// and an inverse-CDF draw from a caller-supplied uniform, one workgroup per
// row; plus Philox-4x32-10 uniforms from (seed, offset) counters.
//
// Arithmetic contract (restated exactly by the numpy oracle, so token ids are
// bit-identical; this translation unit is built with -ffp-contract=off):
//   x_i   = logit_i (fp32; bf16 widened exactly); masked ids -> -inf
//           (executor/talker.py:173-183, 240-243)
//   x_i   = seen_i ? (x_i > 0 ? x_i / r : x_i * r) : x_i   (model/sampling.py:55-65)
//   T == 0: token = argmax_i x_i, lowest id on ties         (model/sampling.py:183-187)
//   s_i   = x_i / T                                         (model/sampling.py:218,
//                                                            executor/sampling.py:267)
//   order : by (s desc, id asc) on the IEEE bit pattern (sortable key), top
//           k_eff = (k > 0 ? min(k, V) : V) ranks           (executor/sampling.py:172-177,268)
//   w_r   = nq_exp(s_r - s_0)                               (executor/sampling.py:272)
//   cum   = segmented wave scan: lane L of 64 owns ranks [L*E, L*E+E), E = ceil(k/64);
//           sequential inclusive sums inside a lane, Kogge-Stone inclusive scan
//           of the lane totals, cum_r = excl_L + local_r
//   keep  = longest rank prefix with (cum_r - w_r) < min(p,1) * cum_{k-1}
//                                                           (executor/sampling.py:275-277)
//   token = id of the first kept rank with cum_r >= u * cum_{last kept}
//           (the last kept rank if none)                    (executor/sampling.py:282-288)
// nq_exp is Cody-Waite range reduction (ln 2 split as in Cephes' expf) with a
// degree-7 Taylor polynomial in Horner form; inputs below -87 give 0.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

constexpr int kSampThreads = 256;
constexpr int kMaxVocab = 4096;
constexpr uint32_t kLog2eBits = 0x3fb8aa3bu;   // 1.44269504f
constexpr uint32_t kLn2HiBits = 0x3f318000u;   // 0.693359375f
constexpr uint32_t kLn2LoBits = 0xb95e8083u;   // -2.12194440e-4f
constexpr uint32_t kExpLowBits = 0xc2ae0000u;  // -87.0f

__device__ __forceinline__ float fbits(uint32_t b) { return __uint_as_float(b); }

__device__ float nq_exp(float x) {
    if (!(x > fbits(kExpLowBits))) return 0.0f;
    const float t = x * fbits(kLog2eBits);
    const float n = floorf(t + 0.5f);
    float r = x - n * fbits(kLn2HiBits);
    r = r - n * fbits(kLn2LoBits);
    float p = 1.0f / 5040.0f;
    p = p * r + 1.0f / 720.0f;
    p = p * r + 1.0f / 120.0f;
    p = p * r + 1.0f / 24.0f;
    p = p * r + 1.0f / 6.0f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    const int ni = static_cast<int>(n);
    return p * __uint_as_float(static_cast<uint32_t>(ni + 127) << 23);
}

__device__ __forceinline__ uint32_t sort_key(float f) {
    const uint32_t u = __float_as_uint(f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

__device__ __forceinline__ uint64_t composite(float f, int id) {
    return (static_cast<uint64_t>(sort_key(f)) << 32) | (0xffffffffu - static_cast<uint32_t>(id));
}

__device__ __forceinline__ uint64_t shfl_xor_u64(uint64_t v, int m) {
    const uint32_t lo = __shfl_xor(static_cast<uint32_t>(v), m, kWave);
    const uint32_t hi = __shfl_xor(static_cast<uint32_t>(v >> 32), m, kWave);
    return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <typename InT>
__device__ __forceinline__ float load_logit(const InT *p);
template <>
__device__ __forceinline__ float load_logit<float>(const float *p) { return *p; }
template <>
__device__ __forceinline__ float load_logit<uint16_t>(const uint16_t *p) { return bf16_to_f32(*p); }

// Eight consecutive logits from a 16- (bf16) or 32-byte (fp32) aligned address.
template <typename InT>
__device__ __forceinline__ void load_logits8(const InT *p, float *x);
template <>
__device__ __forceinline__ void load_logits8<float>(const float *p, float *x) {
    const float4 a = reinterpret_cast<const float4 *>(p)[0], b = reinterpret_cast<const float4 *>(p)[1];
    x[0] = a.x; x[1] = a.y; x[2] = a.z; x[3] = a.w;
    x[4] = b.x; x[5] = b.y; x[6] = b.z; x[7] = b.w;
}
template <>
__device__ __forceinline__ void load_logits8<uint16_t>(const uint16_t *p, float *x) {
    float t[8];
    unpack8(*reinterpret_cast<const uint4 *>(p), t);
#pragma unroll
    for (int e = 0; e < 8; ++e) x[e] = t[e];
}

// Lanes of this wave below the calling lane among those whose bit is set.
__device__ __forceinline__ int lanes_below(uint64_t mask) {
    return static_cast<int>(__builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(mask >> 32),
                                                      __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(mask), 0u)));
}



constexpr int kSampPer = kMaxVocab / kSampThreads;  // elements per thread (8 consecutive, twice)

// Philox-4x32-10 (Salmon, Moraes, Dror, Shaw, SC'11): 10 rounds, key bumped by
// the Weyl constants.  Returns the first output word.
__device__ __forceinline__ uint32_t philox_first(uint32_t c0, uint32_t c1, uint32_t c2, uint32_t c3,
                                                 uint32_t k0, uint32_t k1) {
    constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u;
    constexpr uint32_t W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
    for (int i = 0; i < 10; ++i) {
        const uint64_t p0 = static_cast<uint64_t>(M0) * c0;
        const uint64_t p1 = static_cast<uint64_t>(M1) * c2;
        const uint32_t hi0 = static_cast<uint32_t>(p0 >> 32), lo0 = static_cast<uint32_t>(p0);
        const uint32_t hi1 = static_cast<uint32_t>(p1 >> 32), lo1 = static_cast<uint32_t>(p1);
        const uint32_t n0 = hi1 ^ c1 ^ k0;
        const uint32_t n1 = lo1;
        const uint32_t n2 = hi0 ^ c3 ^ k1;
        const uint32_t n3 = lo0;
        c0 = n0; c1 = n1; c2 = n2; c3 = n3;
        k0 += W0;
        k1 += W1;
    }
    return c0;
}

// The uniform of a (seed, offset) counter: the top 24 bits of the first Philox word.
__device__ __forceinline__ float counter_uniform(int64_t seed, int64_t offset) {
    const uint64_t sd = static_cast<uint64_t>(seed), o = static_cast<uint64_t>(offset);
    const uint32_t x = philox_first(static_cast<uint32_t>(o), static_cast<uint32_t>(o >> 32), 0u, 0u,
                                    static_cast<uint32_t>(sd), static_cast<uint32_t>(sd >> 32));
    return static_cast<float>(x >> 8) * (1.0f / 16777216.0f);
}

// kPlanes: `logits` is `splits` fp32 split-K planes of a projection, `plane`
// elements apart; each logit is their sum in plane order rounded to bf16 (the
// value the projection's reduction would store), also written to logits_out
// (bf16, row stride out_s0) when that is given.
template <typename InT, bool kPlanes>
__global__ void __launch_bounds__(kSampThreads)
sample_kernel(const InT *__restrict__ logits, int64_t logits_s0, int vocab,
              const float *__restrict__ temperature, const int32_t *__restrict__ top_k,
              const float *__restrict__ top_p, const float *__restrict__ penalty,
              uint8_t *__restrict__ seen, int64_t seen_s0, const float *__restrict__ uniforms,
              const int64_t *__restrict__ seed, int64_t seed_stride, const int64_t *__restrict__ offset,
              int64_t offset_stride, int mask_from, int eos_id, const uint8_t *__restrict__ suppress_eos,
              int update_seen, int64_t *__restrict__ tokens, int splits, int64_t plane,
              uint16_t *__restrict__ logits_out, int64_t out_s0) {
    __shared__ float s_val[kMaxVocab];
    __shared__ uint64_t s_sort[kMaxVocab];
    __shared__ uint32_t s_hist[2][256];
    __shared__ int s_bin, s_above, s_count, s_whole;
    __shared__ uint64_t s_red[kSampThreads / kWave];

    const int row = blockIdx.x;
    const int tid = threadIdx.x;
    const int lane = tid & (kWave - 1);
    const int wave = tid / kWave;
    const InT *lrow = logits + row * logits_s0;
    const float T = temperature[row];
    const float r = penalty ? penalty[row] : 1.0f;
    const bool greedy = T == 0.0f;
    const bool sup_eos = suppress_eos && suppress_eos[row];
    uint8_t *srow = seen ? seen + row * seen_s0 : nullptr;

    // 1. masks, penalty, temperature: thread t owns ids 8t .. 8t + 7 and
    // 8 (t + 256) .. + 7, loaded in one round trip; values go to LDS and stay in
    // registers with their sortable keys (ids past the vocabulary get key 0,
    // below every value)
    float val[kSampPer];
    uint32_t key[kSampPer];
    {
        // whole 8-id groups as one vector load each when the rows allow it
        const bool vec = vocab % 8 == 0 && reinterpret_cast<uintptr_t>(lrow) % (8 * sizeof(InT)) == 0 &&
                         (!srow || reinterpret_cast<uintptr_t>(srow) % 8 == 0) &&
                         (!kPlanes || (plane % 8 == 0 && (!logits_out || (out_s0 % 8 == 0 &&
                                                          reinterpret_cast<uintptr_t>(logits_out) % 16 == 0))));
        float x[kSampPer];
        uint8_t sn[kSampPer];
#pragma unroll
        for (int h = 0; h < kSampPer / 8; ++h) {
            const int id0 = (tid + h * kSampThreads) * 8;
            if (vec) {
                if (id0 < vocab) {
                    if constexpr (kPlanes) {
                        float t[8];
                        sum_partials8<4>(reinterpret_cast<const float *>(lrow) + id0, splits, plane, t);
                        uint4 o;
                        o.x = pack2_bf16(t[0], t[1]);
                        o.y = pack2_bf16(t[2], t[3]);
                        o.z = pack2_bf16(t[4], t[5]);
                        o.w = pack2_bf16(t[6], t[7]);
                        if (logits_out) *reinterpret_cast<uint4 *>(logits_out + row * out_s0 + id0) = o;
                        unpack8(o, t);
#pragma unroll
                        for (int e = 0; e < 8; ++e) x[h * 8 + e] = t[e];
                    } else {
                        load_logits8<InT>(lrow + id0, &x[h * 8]);
                    }
                    const uint2 m = srow ? *reinterpret_cast<const uint2 *>(srow + id0) : make_uint2(0u, 0u);
#pragma unroll
                    for (int e = 0; e < 8; ++e) sn[h * 8 + e] = static_cast<uint8_t>((e < 4 ? m.x : m.y) >> (8 * (e % 4)));
                } else {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        x[h * 8 + e] = 0.f;
                        sn[h * 8 + e] = 0;
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int id = id0 + e;
                    if constexpr (kPlanes) {
                        float acc = 0.f;
                        if (id < vocab) {
                            for (int sp = 0; sp < splits; ++sp)
                                acc += reinterpret_cast<const float *>(lrow)[sp * plane + id];
                            const uint16_t b = f32_to_bf16(acc);
                            if (logits_out) logits_out[row * out_s0 + id] = b;
                            acc = bf16_to_f32(b);
                        }
                        x[h * 8 + e] = acc;
                    } else {
                        x[h * 8 + e] = id < vocab ? load_logit<InT>(lrow + id) : 0.f;
                    }
                    sn[h * 8 + e] = (srow && id < vocab) ? srow[id] : 0;
                }
            }
        }
#pragma unroll
        for (int i = 0; i < kSampPer; ++i) {
            const int id = (tid + (i / 8) * kSampThreads) * 8 + i % 8;
            float xv = x[i];
            if ((id >= mask_from && id != eos_id) || (id == eos_id && sup_eos)) xv = -INFINITY;
            if (sn[i]) xv = xv > 0.0f ? xv / r : xv * r;
            val[i] = greedy ? xv : xv / T;
            key[i] = id < vocab ? sort_key(val[i]) : 0u;
            if (id < vocab) s_val[id] = val[i];
        }
    }
    for (int i = tid; i < 2 * 256; i += kSampThreads) (&s_hist[0][0])[i] = 0u;
    if (tid == 0) s_count = 0;
    __syncthreads();

    int token;
    if (greedy) {
        uint64_t best = 0;
#pragma unroll
        for (int i = 0; i < kSampPer; ++i) {
            const int id = (tid + (i / 8) * kSampThreads) * 8 + i % 8;
            if (id < vocab) {
                const uint64_t c = composite(val[i], id);
                best = c > best ? c : best;
            }
        }
#pragma unroll
        for (int m = 1; m < kWave; m <<= 1) {
            const uint64_t o = shfl_xor_u64(best, m);
            best = o > best ? o : best;
        }
        if (lane == 0) s_red[wave] = best;
        __syncthreads();
        best = s_red[0];
        for (int w = 1; w < kSampThreads / kWave; ++w) best = s_red[w] > best ? s_red[w] : best;
        token = static_cast<int>(0xffffffffu - static_cast<uint32_t>(best));
    } else {
        const int kq = top_k[row];
        const int k_eff = (kq > 0 && kq < vocab) ? kq : vocab;
        float p = top_p[row];
        p = p < 1.0f ? p : 1.0f;

        // 2. radix select of the k_eff-th largest sortable key, 8 bits a pass from
        // the top; wave 0 locates each pass's digit (lane L scans bins
        // 255 - 4L .. 252 - 4L) and clears the other histogram for the next pass
        uint32_t prefix = 0, pmask = 0;
        int remaining = k_eff;
        // once the bin holding the k_eff-th key is needed whole, the keys at or
        // above its lowest key are exactly the selection: the select stops there
        if (tid == 0) s_whole = 0;
        for (int pass = 0; pass < 4; ++pass) {
            const int shift = 24 - 8 * pass;
            uint32_t *hist = s_hist[pass & 1];
#pragma unroll
            for (int i = 0; i < kSampPer; ++i)
                if (key[i] != 0u && (key[i] & pmask) == prefix) atomicAdd(&hist[(key[i] >> shift) & 255u], 1u);
            __syncthreads();
            if (wave == 0) {
                uint32_t c[4];
                uint32_t tot = 0;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    c[j] = hist[255 - 4 * lane - j];
                    tot += c[j];
                }
                uint32_t incl = tot;
#pragma unroll
                for (int d = 1; d < kWave; d <<= 1) {
                    const uint32_t o = static_cast<uint32_t>(__shfl_up(static_cast<int>(incl), d, kWave));
                    if (lane >= d) incl += o;
                }
                uint32_t above = incl - tot;  // count in the bins above this lane's
                const int rem = remaining;
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    if (static_cast<int>(above) < rem && rem <= static_cast<int>(above + c[j])) {
                        s_bin = 255 - 4 * lane - j;
                        s_above = static_cast<int>(above);
                        s_whole = rem == static_cast<int>(above + c[j]) ? 1 : 0;
                    }
                    above += c[j];
                }
#pragma unroll
                for (int j = 0; j < 4; ++j) s_hist[(pass + 1) & 1][lane * 4 + j] = 0u;
            }
            __syncthreads();
            prefix |= static_cast<uint32_t>(s_bin) << shift;
            pmask |= 255u << shift;
            remaining -= s_above;
            if (s_whole) break;  // uniform: every thread read the same flag
        }
        const uint32_t thr = prefix;

        // 3. every entry at or above the threshold (ties included), in any order:
        // the sort below puts them in (value desc, id asc) order and the first
        // k_eff are the selection
#pragma unroll
        for (int i = 0; i < kSampPer; ++i) {
            const bool sel = key[i] != 0u && key[i] >= thr;
            const uint64_t m = __ballot(sel);
            if (m) {
                int base = 0;
                const int leader = __ffsll(static_cast<long long>(m)) - 1;
                if (lane == leader) base = atomicAdd(&s_count, __popcll(m));
                base = __shfl(base, leader, kWave);
                const int id = (tid + (i / 8) * kSampThreads) * 8 + i % 8;
                if (sel) s_sort[base + lanes_below(m)] = composite(val[i], id);
            }
        }
        __syncthreads();
        const int n_c = s_count;

        // 4. sort the n_c collected entries by (value desc, id asc).
        if (n_c <= kWave) {
            if (wave == 0) {
                uint64_t kv = lane < n_c ? s_sort[lane] : 0ull;
#pragma unroll
                for (int kk = 2; kk <= kWave; kk <<= 1) {
#pragma unroll
                    for (int j = kk >> 1; j > 0; j >>= 1) {
                        const uint64_t other = shfl_xor_u64(kv, j);
                        const bool lower = (lane & j) == 0;
                        const bool asc = (lane & kk) == 0;
                        const bool take_max = lower == asc;
                        kv = take_max ? (kv > other ? kv : other) : (kv < other ? kv : other);
                    }
                }
                if (lane < n_c) s_sort[lane] = kv;
            }
        } else {
            int n2 = 1;
            while (n2 < n_c) n2 <<= 1;
            for (int i = n_c + tid; i < n2; i += kSampThreads) s_sort[i] = 0ull;
            __syncthreads();
            for (int kk = 2; kk <= n2; kk <<= 1) {
                for (int j = kk >> 1; j > 0; j >>= 1) {
                    for (int idx = tid; idx < n2 / 2; idx += kSampThreads) {
                        const int i = 2 * j * (idx / j) + (idx % j);
                        const int pr = i + j;
                        const bool asc = (i & kk) == 0;
                        const uint64_t a = s_sort[i], b = s_sort[pr];
                        const bool swap = asc ? (a < b) : (a > b);
                        if (swap) {
                            s_sort[i] = b;
                            s_sort[pr] = a;
                        }
                    }
                    __syncthreads();
                }
            }
        }
        __syncthreads();

        // 5. weights (rank order), stored as (w bits << 32 | id).
        const float v0 = s_val[static_cast<int>(0xffffffffu - static_cast<uint32_t>(s_sort[0]))];
        __syncthreads();
        for (int rr = tid; rr < k_eff; rr += kSampThreads) {
            const int id = static_cast<int>(0xffffffffu - static_cast<uint32_t>(s_sort[rr]));
            const float w = nq_exp(s_val[id] - v0);
            s_sort[rr] = (static_cast<uint64_t>(__float_as_uint(w)) << 32) | static_cast<uint32_t>(id);
        }
        __syncthreads();

        // 6. segmented wave scan, nucleus and draw (wave 0).
        if (wave == 0) {
            const int E = (k_eff + kWave - 1) / kWave;
            const int r0 = lane * E;
            const int r1 = min(k_eff, r0 + E);
            float loc = 0.0f;
            for (int rr = r0; rr < r1; ++rr) {
                loc = loc + __uint_as_float(static_cast<uint32_t>(s_sort[rr] >> 32));
                s_val[rr] = loc;  // local inclusive sums, rank-indexed (ids are no longer needed)
            }
            float S = loc;
#pragma unroll
            for (int d = 1; d < kWave; d <<= 1) {
                const float o = __shfl_up(S, d, kWave);
                if (lane >= d) S = S + o;
            }
            float excl = __shfl_up(S, 1, kWave);
            if (lane == 0) excl = 0.0f;
            for (int rr = r0; rr < r1; ++rr) s_val[rr] = excl + s_val[rr];
        }
        __syncthreads();
        if (wave == 0) {
            const float total = s_val[k_eff - 1];
            const float pt = p * total;
            const int E = (k_eff + kWave - 1) / kWave;
            const int r0 = lane * E;
            const int r1 = min(k_eff, r0 + E);
            int first_drop = k_eff;
            for (int rr = r0; rr < r1; ++rr) {
                const float w = __uint_as_float(static_cast<uint32_t>(s_sort[rr] >> 32));
                if (!((s_val[rr] - w) < pt)) { first_drop = rr; break; }
            }
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) first_drop = min(first_drop, __shfl_xor(first_drop, m, kWave));
            const int kept = first_drop > 0 ? first_drop : 1;
            const float mass = s_val[kept - 1];
            // the row's uniform: given, or drawn here from its (seed, offset) counter
            const float u = uniforms ? uniforms[row] : counter_uniform(seed[row * seed_stride], offset[row * offset_stride]);
            const float um = u * mass;
            int pick = kept - 1;
            for (int rr = r0; rr < min(r1, kept); ++rr)
                if (s_val[rr] >= um) { pick = rr; break; }
#pragma unroll
            for (int m = 1; m < kWave; m <<= 1) pick = min(pick, __shfl_xor(pick, m, kWave));
            if (v0 == -INFINITY) pick = 0;
            if (lane == 0) s_bin = static_cast<int>(static_cast<uint32_t>(s_sort[pick]));
        }
        __syncthreads();
        token = s_bin;
    }
    if (tid == 0) {
        tokens[row] = token;
        if (update_seen && srow) srow[token] = 1;
    }
}

__global__ void uniforms_kernel(const int64_t *__restrict__ seed, int64_t seed_stride,
                                const int64_t *__restrict__ offset, int64_t offset_stride, int rows,
                                float *__restrict__ out) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= rows) return;
    out[i] = counter_uniform(seed[i * seed_stride], offset[i * offset_stride]);
}

}  // namespace
}  // namespace nq

namespace {

int launch_sample(const void *logits, int logits_dtype, int64_t logits_s0, int rows, int vocab,
                  const float *temperature, const int32_t *top_k, const float *top_p,
                  const float *repetition_penalty, uint8_t *seen, int64_t seen_s0, const float *uniforms,
                  const int64_t *seed, int64_t seed_stride, const int64_t *offset, int64_t offset_stride,
                  int mask_from, int eos_id, const uint8_t *suppress_eos, int update_seen, int64_t *tokens,
                  void *stream, int splits = 0, uint16_t *logits_out = nullptr, int64_t out_s0 = 0) {
    NQ_CHECK_ARG(logits && temperature && top_k && top_p && tokens);
    NQ_CHECK_ARG(uniforms || (seed && offset));
    NQ_CHECK_ARG(rows >= 0 && vocab >= 1);
    NQ_CHECK_ARG(!update_seen || seen);
    if (vocab > nq::kMaxVocab) return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    hipStream_t s = static_cast<hipStream_t>(stream);
    const dim3 grid(rows), block(nq::kSampThreads);
    if (splits > 0) {
        // fp32 planes [splits][rows][logits_s0]
        const int64_t plane = static_cast<int64_t>(rows) * logits_s0;
        hipLaunchKernelGGL((nq::sample_kernel<float, true>), grid, block, 0, s, static_cast<const float *>(logits),
                           logits_s0, vocab, temperature, top_k, top_p, repetition_penalty, seen, seen_s0, uniforms,
                           seed, seed_stride, offset, offset_stride, mask_from, eos_id, suppress_eos, update_seen,
                           tokens, splits, plane, logits_out, out_s0);
    } else if (logits_dtype == NQ_F32) {
        hipLaunchKernelGGL((nq::sample_kernel<float, false>), grid, block, 0, s, static_cast<const float *>(logits),
                           logits_s0, vocab, temperature, top_k, top_p, repetition_penalty, seen, seen_s0, uniforms,
                           seed, seed_stride, offset, offset_stride, mask_from, eos_id, suppress_eos, update_seen,
                           tokens, 0, int64_t{0}, static_cast<uint16_t *>(nullptr), int64_t{0});
    } else if (logits_dtype == NQ_BF16) {
        hipLaunchKernelGGL((nq::sample_kernel<uint16_t, false>), grid, block, 0, s,
                           static_cast<const uint16_t *>(logits), logits_s0, vocab, temperature, top_k, top_p,
                           repetition_penalty, seen, seen_s0, uniforms, seed, seed_stride, offset, offset_stride,
                           mask_from, eos_id, suppress_eos, update_seen, tokens, 0, int64_t{0},
                           static_cast<uint16_t *>(nullptr), int64_t{0});
    } else {
        return NQ_ERR_UNSUPPORTED;
    }
    return NQ_LAUNCH_STATUS();
}

}  // namespace

extern "C" int nq_sample(const void *logits, int logits_dtype, int64_t logits_s0, int rows,
                         int vocab, const float *temperature, const int32_t *top_k,
                         const float *top_p, const float *repetition_penalty, uint8_t *seen,
                         int64_t seen_s0, const float *uniforms, int mask_from, int eos_id,
                         const uint8_t *suppress_eos, int update_seen, int64_t *tokens,
                         void *stream) {
    NQ_CHECK_ARG(uniforms);
    return launch_sample(logits, logits_dtype, logits_s0, rows, vocab, temperature, top_k, top_p,
                         repetition_penalty, seen, seen_s0, uniforms, nullptr, 0, nullptr, 0, mask_from, eos_id,
                         suppress_eos, update_seen, tokens, stream);
}

extern "C" int nq_sample_counter(const void *logits, int logits_dtype, int64_t logits_s0, int rows, int vocab,
                                 const float *temperature, const int32_t *top_k, const float *top_p,
                                 const float *repetition_penalty, uint8_t *seen, int64_t seen_s0,
                                 const int64_t *seed, int64_t seed_stride, const int64_t *offset,
                                 int64_t offset_stride, int mask_from, int eos_id, const uint8_t *suppress_eos,
                                 int update_seen, int64_t *tokens, void *stream) {
    NQ_CHECK_ARG(seed && offset);
    return launch_sample(logits, logits_dtype, logits_s0, rows, vocab, temperature, top_k, top_p,
                         repetition_penalty, seen, seen_s0, nullptr, seed, seed_stride, offset, offset_stride,
                         mask_from, eos_id, suppress_eos, update_seen, tokens, stream);
}

extern "C" int nq_sample_counter_planes(const float *planes, int splits, int64_t row_stride, int rows, int vocab,
                                        const float *temperature, const int32_t *top_k, const float *top_p,
                                        const float *repetition_penalty, uint8_t *seen, int64_t seen_s0,
                                        const int64_t *seed, int64_t seed_stride, const int64_t *offset,
                                        int64_t offset_stride, int mask_from, int eos_id, const uint8_t *suppress_eos,
                                        int update_seen, uint16_t *logits_out, int64_t out_s0, int64_t *tokens,
                                        void *stream) {
    NQ_CHECK_ARG(seed && offset && planes && splits >= 1 && splits <= 64 && row_stride >= vocab);
    NQ_CHECK_ARG(!logits_out || out_s0 >= vocab);
    return launch_sample(planes, NQ_F32, row_stride, rows, vocab, temperature, top_k, top_p, repetition_penalty,
                         seen, seen_s0, nullptr, seed, seed_stride, offset, offset_stride, mask_from, eos_id,
                         suppress_eos, update_seen, tokens, stream, splits, logits_out, out_s0);
}

extern "C" int nq_uniforms_from_counter(const int64_t *seed, int64_t seed_stride,
                                        const int64_t *offset, int64_t offset_stride, int rows,
                                        float *uniforms, void *stream) {
    NQ_CHECK_ARG(seed && offset && uniforms && rows >= 0);
    if (rows == 0) return NQ_OK;
    hipLaunchKernelGGL(nq::uniforms_kernel, dim3((rows + 255) / 256), dim3(256), 0,
                       static_cast<hipStream_t>(stream), seed, seed_stride, offset, offset_stride,
                       rows, uniforms);
    return NQ_LAUNCH_STATUS();
}
