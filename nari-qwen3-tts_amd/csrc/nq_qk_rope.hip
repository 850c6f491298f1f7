// Fused per-head q/k RMSNorm + rotate-half RoPE with the paged (or dense)
// K/V cache write.
//
// Restates _paired_qk_norm_rope_paged_cache_kernel (model/kernels.py:15-91)
// and _paired_qk_norm_rope_dense_kernel (model/kernels.py:163-248): fp32
// RMSNorm with weight, optional bf16 rounding before the rotation,
// inv_freq = exp(-ln(theta) * 2i/D), angle = position * inv_freq, and the
// rotate-half pair (i, i + D/2).
//
// Work split: one wave per (token, unit), where the units of a token are its
// query heads, its key heads and its value heads (the value units only copy
// V into the cache), so a decode batch of 64 tokens runs 64 x 32 waves
// instead of 64 serial workgroups.  Lane i of a q/k unit holds the pair
// (i, i + D/2): the rotation needs no data exchange and the sum of squares is
// one reduction over D/2 lanes.  The q/k/v values come either from bf16
// tensors (rotated in place, the reference's contract) or straight from the
// fp32 split-K partial planes of the packed QKV projection, summed in plane
// order and rounded to bf16 -- the value the bf16 projection output would
// hold -- so the projection needs no separate reduction pass.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

constexpr int kRopeThreads = 256;
constexpr int kRopeWaves = kRopeThreads / kWave;

enum Unit { kUnitQ = 0, kUnitK = 1, kUnitV = 2 };

struct Bf16Heads {
    const uint16_t *q, *k, *v;
    int64_t q_s0, q_s1, k_s0, k_s1, v_s0, v_s1;
    __device__ __forceinline__ float load(int kind, int64_t tok, int head, int d) const {
        const uint16_t *p = kind == kUnitQ ? q + tok * q_s0 + head * q_s1
                          : kind == kUnitK ? k + tok * k_s0 + head * k_s1
                                           : v + tok * v_s0 + head * v_s1;
        return bf16_to_f32(p[d]);
    }
};

struct PartialHeads {
    const float *p;
    int S;
    int64_t plane, row;  // plane = tokens * row, row = (Hq + 2 Hkv) * D
    int Hq, Hkv, D;
    __device__ __forceinline__ float load(int kind, int64_t tok, int head, int d) const {
        const int col = (kind == kUnitQ ? head : kind == kUnitK ? Hq + head : Hq + Hkv + head) * D + d;
        const float *e = p + tok * row + col;
        float s = 0.f;
        // four planes in flight at a time, added in plane order
        for (int i0 = 0; i0 < S; i0 += 4) {
            float a[4];
#pragma unroll
            for (int v = 0; v < 4; ++v) a[v] = i0 + v < S ? e[(i0 + v) * plane] : 0.f;
#pragma unroll
            for (int v = 0; v < 4; ++v)
                if (i0 + v < S) s += a[v];
        }
        return bf16_to_f32(f32_to_bf16(s));
    }
};

struct RopeOut {
    uint16_t *q;  // rotated q (in place for bf16 sources)
    int64_t q_s0, q_s1;
    uint16_t *k;  // rotated k, or null
    int64_t k_s0, k_s1;
};

template <int D, typename Src>
__global__ void __launch_bounds__(kRopeThreads)
qk_norm_rope_kernel(Src src, RopeOut dst, const uint16_t *__restrict__ q_weight,
                    const uint16_t *__restrict__ k_weight, const int64_t *__restrict__ positions,
                    int64_t pos_stride, int num_qo_heads, int num_kv_heads, int units, float eps,
                    float log_theta, int round_to_input, uint16_t *__restrict__ cache, int64_t c_page,
                    int64_t c_kind, int64_t c_slot, int64_t c_head, const int64_t *__restrict__ write_pages,
                    const int64_t *__restrict__ write_offsets, int cache_position) {
    constexpr int HALF = D / 2;
    const int lane = threadIdx.x & (kWave - 1);
    const int64_t tok = blockIdx.x;
    const int unit = blockIdx.y * kRopeWaves + threadIdx.x / kWave;
    if (unit >= units) return;  // whole waves leave; no barriers follow
    int kind, head;
    if (unit < num_qo_heads) {
        kind = kUnitQ;
        head = unit;
    } else if (unit < num_qo_heads + num_kv_heads) {
        kind = kUnitK;
        head = unit - num_qo_heads;
    } else {
        kind = kUnitV;
        head = unit - num_qo_heads - num_kv_heads;
    }
    int64_t page = 0, slot = 0;
    if (cache) {
        page = write_pages ? write_pages[tok] : tok;
        slot = write_offsets ? write_offsets[tok] : cache_position;
    }
    if (kind == kUnitV) {
        uint16_t *dstv = cache + page * c_page + c_kind + slot * c_slot + head * c_head;
        for (int d = lane; d < D; d += kWave) dstv[d] = f32_to_bf16(src.load(kUnitV, tok, head, d));
        return;
    }
    const bool on = lane < HALF;
    float x1 = 0.f, x2 = 0.f, w1 = 0.f, w2 = 0.f;
    if (on) {
        // the norm weights are loaded with the inputs, not after their reduction
        const uint16_t *wt = kind == kUnitQ ? q_weight : k_weight;
        w1 = bf16_to_f32(wt[lane]);
        w2 = bf16_to_f32(wt[lane + HALF]);
        x1 = src.load(kind, tok, head, lane);
        x2 = src.load(kind, tok, head, lane + HALF);
    }
    uint16_t o1 = 0, o2 = 0;
    norm_rope_pair<D>(x1, x2, on, w1, w2, lane, eps, log_theta, static_cast<float>(positions[tok * pos_stride]),
                      round_to_input, o1, o2);
    if (!on) return;
    if (kind == kUnitQ) {
        uint16_t *qo = dst.q + tok * dst.q_s0 + head * dst.q_s1;
        qo[lane] = o1;
        qo[lane + HALF] = o2;
        return;
    }
    if (dst.k) {
        uint16_t *ko = dst.k + tok * dst.k_s0 + head * dst.k_s1;
        ko[lane] = o1;
        ko[lane + HALF] = o2;
    }
    if (cache) {
        uint16_t *dk = cache + page * c_page + slot * c_slot + head * c_head;
        dk[lane] = o1;
        dk[lane + HALF] = o2;
    }
}

template <typename Src>
int launch_rope(const Src &src, const RopeOut &dst, const uint16_t *q_weight, const uint16_t *k_weight,
                const int64_t *positions, int64_t pos_stride, int tokens, int Hq, int Hkv, int D, float eps,
                float rope_theta, int round_to_input, uint16_t *cache, int64_t c_page, int64_t c_kind,
                int64_t c_slot, int64_t c_head, const int64_t *write_pages, const int64_t *write_offsets,
                int cache_position, bool has_v, hipStream_t s) {
    const float log_theta = logf(rope_theta);
    const int units = Hq + Hkv + ((cache && has_v) ? Hkv : 0);
    const dim3 grid(static_cast<unsigned>(tokens), static_cast<unsigned>((units + kRopeWaves - 1) / kRopeWaves));
#define NQ_ROPE(DD)                                                                                        \
    if (D == DD) {                                                                                         \
        hipLaunchKernelGGL((qk_norm_rope_kernel<DD, Src>), grid, dim3(kRopeThreads), 0, s, src, dst, q_weight, \
                           k_weight, positions, pos_stride, Hq, Hkv, units, eps, log_theta, round_to_input,    \
                           cache, c_page, c_kind, c_slot, c_head, write_pages, write_offsets, cache_position); \
        return NQ_LAUNCH_STATUS();                                                                         \
    }
    NQ_ROPE(128) NQ_ROPE(64) NQ_ROPE(32)
#undef NQ_ROPE
    return NQ_ERR_UNSUPPORTED;
}

}  // namespace
}  // namespace nq

extern "C" int nq_qk_norm_rope_kv_write(uint16_t *q, int64_t q_s0, int64_t q_s1, uint16_t *k,
                                        int64_t k_s0, int64_t k_s1, const uint16_t *v,
                                        int64_t v_s0, int64_t v_s1, const uint16_t *q_weight,
                                        const uint16_t *k_weight, const int64_t *positions,
                                        int64_t pos_stride, int tokens, int num_qo_heads,
                                        int num_kv_heads, int head_dim, float eps,
                                        float rope_theta, int round_to_input, uint16_t *cache,
                                        int64_t c_page, int64_t c_kind, int64_t c_slot,
                                        int64_t c_head, const int64_t *write_pages,
                                        const int64_t *write_offsets, int cache_position,
                                        void *stream) {
    NQ_CHECK_ARG(q && k && q_weight && k_weight && positions && tokens >= 0);
    NQ_CHECK_ARG(num_qo_heads >= 1 && num_kv_heads >= 1 && rope_theta > 0.f);
    NQ_CHECK_ARG(!cache || v);
    NQ_CHECK_ARG((write_pages == nullptr) == (write_offsets == nullptr));
    if (tokens == 0) return NQ_OK;
    const nq::Bf16Heads src{q, k, v, q_s0, q_s1, k_s0, k_s1, v_s0, v_s1};
    const nq::RopeOut dst{q, q_s0, q_s1, k, k_s0, k_s1};
    return nq::launch_rope(src, dst, q_weight, k_weight, positions, pos_stride, tokens, num_qo_heads, num_kv_heads,
                           head_dim, eps, rope_theta, round_to_input, cache, c_page, c_kind, c_slot, c_head,
                           write_pages, write_offsets, cache_position, v != nullptr,
                           static_cast<hipStream_t>(stream));
}

extern "C" int nq_qkv_partials_norm_rope_kv_write(const float *partials, int splits, int tokens, uint16_t *q_out,
                                                  int64_t q_s0, int64_t q_s1, uint16_t *k_out, int64_t k_s0,
                                                  int64_t k_s1, const uint16_t *q_weight, const uint16_t *k_weight,
                                                  const int64_t *positions, int64_t pos_stride, int num_qo_heads,
                                                  int num_kv_heads, int head_dim, float eps, float rope_theta,
                                                  int round_to_input, uint16_t *cache, int64_t c_page,
                                                  int64_t c_kind, int64_t c_slot, int64_t c_head,
                                                  const int64_t *write_pages, const int64_t *write_offsets,
                                                  int cache_position, void *stream) {
    NQ_CHECK_ARG(partials && splits >= 1 && q_out && q_weight && k_weight && positions && tokens >= 0);
    NQ_CHECK_ARG(num_qo_heads >= 1 && num_kv_heads >= 1 && rope_theta > 0.f && cache);
    NQ_CHECK_ARG((write_pages == nullptr) == (write_offsets == nullptr));
    if (tokens == 0) return NQ_OK;
    const int64_t row = static_cast<int64_t>(num_qo_heads + 2 * num_kv_heads) * head_dim;
    const nq::PartialHeads src{partials, splits, static_cast<int64_t>(tokens) * row, row, num_qo_heads, num_kv_heads,
                               head_dim};
    const nq::RopeOut dst{q_out, q_s0, q_s1, k_out, k_s0, k_s1};
    return nq::launch_rope(src, dst, q_weight, k_weight, positions, pos_stride, tokens, num_qo_heads, num_kv_heads,
                           head_dim, eps, rope_theta, round_to_input, cache, c_page, c_kind, c_slot, c_head,
                           write_pages, write_offsets, cache_position, true, static_cast<hipStream_t>(stream));
}
