// Fused per-head q/k RMSNorm + rotate-half RoPE with the paged (or dense)
// K/V cache write, one workgroup per token.
//
// Restates _paired_qk_norm_rope_paged_cache_kernel (model/kernels.py:15-91)
// and _paired_qk_norm_rope_dense_kernel (model/kernels.py:163-248): fp32
// RMSNorm with weight, optional bf16 rounding before the rotation,
// inv_freq = exp(-ln(theta) * 2i/D), angle = position * inv_freq, and the
// rotate-half pair (i, i + D/2).  Lane i of a head holds exactly that pair,
// so the rotation needs no data exchange; the sum of squares is a wave
// reduction over D/2 lanes.
#include "nq_common.h"

namespace nq {
namespace {

constexpr int kRopeThreads = 256;

template <int D>
__global__ void __launch_bounds__(kRopeThreads)
qk_norm_rope_kernel(uint16_t *__restrict__ q, int64_t q_s0, int64_t q_s1, uint16_t *__restrict__ k,
                    int64_t k_s0, int64_t k_s1, const uint16_t *__restrict__ v, int64_t v_s0,
                    int64_t v_s1, const uint16_t *__restrict__ q_weight,
                    const uint16_t *__restrict__ k_weight, const int64_t *__restrict__ positions,
                    int64_t pos_stride, int num_qo_heads, int num_kv_heads, float eps,
                    float log_theta, int round_to_input, uint16_t *__restrict__ cache,
                    int64_t c_page, int64_t c_kind, int64_t c_slot, int64_t c_head,
                    const int64_t *__restrict__ write_pages, const int64_t *__restrict__ write_offsets,
                    int cache_position) {
    constexpr int HALF = D / 2;
    constexpr int HPW = kWave / HALF;  // heads per wave pass
    const int tok = blockIdx.x;
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int i = lane % HALF;
    const int sub_head = lane / HALF;
    const int total_heads = num_qo_heads + num_kv_heads;

    int64_t page = 0, slot = 0;
    if (cache) {
        page = write_pages ? write_pages[tok] : tok;
        slot = write_offsets ? write_offsets[tok] : cache_position;
    }
    const float position = static_cast<float>(positions[tok * pos_stride]);
    const float inv_freq = expf(-log_theta * (static_cast<float>(i) * 2.0f / static_cast<float>(D)));
    const float angle = position * inv_freq;
    float sn, cs;
    sincosf(angle, &sn, &cs);

    for (int hb = wave * HPW; hb < total_heads; hb += (kRopeThreads / kWave) * HPW) {
        const int head = hb + sub_head;
        const bool active = head < total_heads;
        const bool is_q = head < num_qo_heads;
        uint16_t *base = nullptr;
        const uint16_t *w = nullptr;
        if (active) {
            base = is_q ? q + tok * q_s0 + head * q_s1 : k + tok * k_s0 + (head - num_qo_heads) * k_s1;
            w = is_q ? q_weight : k_weight;
        }
        float x1 = 0.f, x2 = 0.f;
        if (active) {
            x1 = bf16_to_f32(base[i]);
            x2 = bf16_to_f32(base[i + HALF]);
        }
        const float ss = group_sum<HALF>(x1 * x1 + x2 * x2);
        if (!active) continue;
        const float inv_rms = 1.0f / sqrtf(ss / static_cast<float>(D) + eps);
        float f = x1 * inv_rms * bf16_to_f32(w[i]);
        float s = x2 * inv_rms * bf16_to_f32(w[i + HALF]);
        if (round_to_input) {
            f = bf16_to_f32(f32_to_bf16(f));
            s = bf16_to_f32(f32_to_bf16(s));
        }
        const uint16_t o1 = f32_to_bf16(f * cs - s * sn);
        const uint16_t o2 = f32_to_bf16(s * cs + f * sn);
        base[i] = o1;
        base[i + HALF] = o2;
        if (!is_q && cache) {
            uint16_t *dst = cache + page * c_page + slot * c_slot + (head - num_qo_heads) * c_head;
            dst[i] = o1;
            dst[i + HALF] = o2;
        }
    }
    if (cache) {
        for (int e = threadIdx.x; e < num_kv_heads * D; e += kRopeThreads) {
            const int h = e / D, d = e % D;
            cache[page * c_page + c_kind + slot * c_slot + h * c_head + d] =
                v[tok * v_s0 + h * v_s1 + d];
        }
    }
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
    const float log_theta = logf(rope_theta);
    hipStream_t s = static_cast<hipStream_t>(stream);
#define NQ_ROPE(DD)                                                                               \
    if (head_dim == DD) {                                                                         \
        hipLaunchKernelGGL(nq::qk_norm_rope_kernel<DD>, dim3(tokens), dim3(nq::kRopeThreads), 0, \
                           s, q, q_s0, q_s1, k, k_s0, k_s1, v, v_s0, v_s1, q_weight, k_weight,    \
                           positions, pos_stride, num_qo_heads, num_kv_heads, eps, log_theta,     \
                           round_to_input, cache, c_page, c_kind, c_slot, c_head, write_pages,    \
                           write_offsets, cache_position);                                        \
        return NQ_LAUNCH_STATUS();                                                                \
    }
    NQ_ROPE(128) NQ_ROPE(64) NQ_ROPE(32)
#undef NQ_ROPE
    return NQ_ERR_UNSUPPORTED;
}
