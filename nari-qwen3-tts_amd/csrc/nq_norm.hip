// Row-wise residual-add + RMSNorm, RMSNorm and SwiGLU pointwise kernels of the
// talker decode step (model/layers.py:28-115), bf16 in and out, fp32 math.
// One workgroup per row; each thread keeps its 8-element slices in registers
// between the sum-of-squares reduction and the scaled store, so a row is read
// and written exactly once.  The add-RMSNorm that feeds the FP8 gate/up
// projection can instead store its bf16 result quantized to e4m3fn codes with
// one scale per 128 columns (max |y| / 448), the activation quantization of the
// block-scaled FP8 GEMM, so that GEMM reads one byte per activation.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

constexpr int kNormThreads = 256;
constexpr int kMaxVec = 4;  // width <= 256 * 8 * 4 = 8192

__device__ float norm_block_sum(float v, float *tmp) {
    v = group_sum<kWave>(v);
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    if (lane == 0) tmp[wave] = v;
    __syncthreads();
    float s = 0.f;
#pragma unroll
    for (int w = 0; w < kNormThreads / kWave; ++w) s += tmp[w];
    __syncthreads();
    return s;
}

// Source of the "hidden" operand: a bf16 tensor, or the fp32 split-K partial
// planes of a projection, summed in plane order and rounded to bf16 (exactly
// the value the bf16 projection output would hold).
struct Bf16Src {
    const uint16_t *p;
    int64_t s0;
    __device__ __forceinline__ void load8(int64_t row, int col, float (&x)[8]) const {
        unpack8(*reinterpret_cast<const uint4 *>(p + row * s0 + col), x);
    }
};

struct PartialSrc {
    const float *p;
    int S;
    int64_t plane;  // elements per partial plane
    int64_t s0;     // row stride of a plane
    __device__ __forceinline__ void load8(int64_t row, int col, float (&x)[8]) const {
        // every plane of the projection in flight at once (up to 16): the norm
        // runs one workgroup per row, so each round trip is paid in full
        sum_partials8<16>(p + row * s0 + col, S, plane, x);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = bf16_to_f32(f32_to_bf16(x[e]));
    }
};

// Source of the "hidden" operand gathered from an embedding table by token
// id: row r reads table[ids[r]]; an id outside [0, n) reads row 0 and reports
// NQ_ERR_INVALID_ARGUMENT in *status (when given), where nn.Embedding raises.
struct GatherSrc {
    const uint16_t *table;
    int64_t s0;
    const int64_t *ids;
    int64_t n;
    int32_t *status;
    __device__ __forceinline__ void load8(int64_t row, int col, float (&x)[8]) const {
        int64_t id = ids[row];
        if (id < 0 || id >= n) {
            if (status && col == 0) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
            id = 0;
        }
        unpack8(*reinterpret_cast<const uint4 *>(table + id * s0 + col), x);
    }
};

// Prefill input embedding (materialize_prefill, executor/talker.py:246-254): row r is
// text[text_ids[r]] + codec[codec_ids[r]] added in bf16 where mask[r], else text[text_ids[r]]
// exactly.  Ids outside their tables read row 0 and report NQ_ERR_INVALID_ARGUMENT.
struct MaskedPairSrc {
    GatherSrc text;
    GatherSrc codec;
    const uint8_t *mask;
    __device__ __forceinline__ void load8(int64_t row, int col, float (&x)[8]) const {
        text.load8(row, col, x);
        if (!mask[row]) return;
        float c[8];
        codec.load8(row, col, c);
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = bf16_to_f32(f32_to_bf16(x[e] + c[e]));
    }
};

// Quantized output of the normalised row: codes [rows, width] and scales
// [rows, width / 128].
struct Fp8Out {
    uint8_t *q;
    int64_t q_s0;
    float *s;
    int64_t s_s0;
};

// kAdd false: the residual row is the hidden operand itself (a gathered
// embedding row, copied exactly), nothing is added.
template <typename Src, bool kFp8, int kVec, bool kAdd = true>
__global__ void __launch_bounds__(kNormThreads)
add_rmsnorm_kernel(Src hidden, uint16_t *__restrict__ hidden_out, int64_t ho_s0,
                   uint16_t *__restrict__ residual, const uint16_t *__restrict__ residual_in, int64_t ri_s0,
                   const uint16_t *__restrict__ weight, int width, float eps, Fp8Out fp8) {
    __shared__ float tmp[kNormThreads / kWave];
    const int64_t row = blockIdx.x;
    const int nvec = width / 8;
    float x[kVec][8], w[kVec][8];
    float ss = 0.f;
    // every load of the row first (residual and weight as raw words, then the
    // hidden operand, whose split-K source waits for its planes), then the math
    float a[kVec][8], b[kVec][8];
    uint4 rb[kVec], rw[kVec];
    // the residual is read from residual_in when given (then only written to residual)
    const uint16_t *rin = residual_in ? residual_in + row * ri_s0 : residual + row * width;
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
        const int vi = threadIdx.x + i * kNormThreads;
        if (vi < nvec) {
            if constexpr (kAdd) rb[i] = *reinterpret_cast<const uint4 *>(rin + vi * 8);
            rw[i] = *reinterpret_cast<const uint4 *>(weight + vi * 8);
        }
    }
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
        const int vi = threadIdx.x + i * kNormThreads;
        if (vi < nvec) {
            hidden.load8(row, vi * 8, a[i]);
            if constexpr (kAdd) unpack8(rb[i], b[i]);
            unpack8(rw[i], w[i]);
        }
    }
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
        const int vi = threadIdx.x + i * kNormThreads;
        if (vi < nvec) {
            uint4 packed;
            uint32_t *pw = reinterpret_cast<uint32_t *>(&packed);
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                if constexpr (kAdd)
                    pw[e / 2] = pack2_bf16(a[i][e] + b[i][e], a[i][e + 1] + b[i][e + 1]);
                else
                    pw[e / 2] = pack2_bf16(a[i][e], a[i][e + 1]);  // bf16 values: exact
            }
            *reinterpret_cast<uint4 *>(residual + row * width + vi * 8) = packed;
            unpack8(packed, x[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += x[i][e] * x[i][e];
        }
    }
    const float inv = rsqrtf(norm_block_sum(ss, tmp) / static_cast<float>(width) + eps);
#pragma unroll
    for (int i = 0; i < kVec; ++i) {
        const int vi = threadIdx.x + i * kNormThreads;
        if (vi < nvec) {
            if constexpr (kFp8) {
                // the 16 threads of a 128-column group are consecutive and all inside the row
                float y[8];
                float amax = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    y[e] = bf16_to_f32(f32_to_bf16(x[i][e] * inv * w[i][e]));
                    amax = fmaxf(amax, fabsf(y[e]));
                }
                const float sc = row_group_scale(group_max<16>(amax));
                *reinterpret_cast<uint2 *>(fp8.q + row * fp8.q_s0 + vi * 8) = e4m3_pack8(y, sc);
                if ((vi & 15) == 0) fp8.s[row * fp8.s_s0 + vi / 16] = sc;
            } else {
                uint4 packed;
                uint32_t *pw = reinterpret_cast<uint32_t *>(&packed);
#pragma unroll
                for (int e = 0; e < 8; e += 2)
                    pw[e / 2] = pack2_bf16(x[i][e] * inv * w[i][e], x[i][e + 1] * inv * w[i][e + 1]);
                *reinterpret_cast<uint4 *>(hidden_out + row * ho_s0 + vi * 8) = packed;
            }
        }
    }
}

__global__ void __launch_bounds__(kNormThreads)
rmsnorm_kernel(const uint16_t *__restrict__ xin, const uint16_t *__restrict__ weight,
               uint16_t *__restrict__ out, int width, float eps) {
    __shared__ float tmp[kNormThreads / kWave];
    const int64_t base = static_cast<int64_t>(blockIdx.x) * width;
    const int nvec = width / 8;
    float x[kMaxVec][8];
    float ss = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const int vi = threadIdx.x + i * kNormThreads;
        if (vi < nvec) {
            unpack8(*reinterpret_cast<const uint4 *>(xin + base + vi * 8), x[i]);
#pragma unroll
            for (int e = 0; e < 8; ++e) ss += x[i][e] * x[i][e];
        }
    }
    const float inv = rsqrtf(norm_block_sum(ss, tmp) / static_cast<float>(width) + eps);
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const int vi = threadIdx.x + i * kNormThreads;
        if (vi < nvec) {
            float w[8];
            unpack8(*reinterpret_cast<const uint4 *>(weight + vi * 8), w);
            uint4 packed;
            uint32_t *pw = reinterpret_cast<uint32_t *>(&packed);
#pragma unroll
            for (int e = 0; e < 8; e += 2)
                pw[e / 2] = pack2_bf16(x[i][e] * inv * w[e], x[i][e + 1] * inv * w[e + 1]);
            *reinterpret_cast<uint4 *>(out + base + vi * 8) = packed;
        }
    }
}

template <typename Src>
__global__ void __launch_bounds__(256)
silu_mul_kernel(Src gate_up, uint16_t *__restrict__ out, int64_t o_s0, int rows, int width) {
    const int nvec = width / 8;
    const int64_t total = static_cast<int64_t>(rows) * nvec;
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * blockDim.x) {
        const int64_t r = i / nvec;
        const int v = static_cast<int>(i - r * nvec);
        float g[8], u[8];
        gate_up.load8(r, v * 8, g);
        gate_up.load8(r, width + v * 8, u);
        uint4 packed;
        uint32_t *pw = reinterpret_cast<uint32_t *>(&packed);
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const float a = g[e] / (1.0f + expf(-g[e])) * u[e];
            const float b = g[e + 1] / (1.0f + expf(-g[e + 1])) * u[e + 1];
            pw[e / 2] = pack2_bf16(a, b);
        }
        *reinterpret_cast<uint4 *>(out + r * o_s0 + v * 8) = packed;
    }
}

// Launch with the fewest 8-column vectors per thread that cover the row, so
// that a narrow row keeps no registers for vectors it does not have.
template <typename Src, bool kFp8, bool kAdd = true, typename... Args>
void launch_add_rmsnorm(int rows, int width, hipStream_t st, Src src, Args... args) {
    const int nv = (width / 8 + kNormThreads - 1) / kNormThreads;
    const dim3 grid(rows), block(kNormThreads);
    if (nv <= 1)
        hipLaunchKernelGGL((add_rmsnorm_kernel<Src, kFp8, 1, kAdd>), grid, block, 0, st, src, args...);
    else if (nv <= 2)
        hipLaunchKernelGGL((add_rmsnorm_kernel<Src, kFp8, 2, kAdd>), grid, block, 0, st, src, args...);
    else
        hipLaunchKernelGGL((add_rmsnorm_kernel<Src, kFp8, kMaxVec, kAdd>), grid, block, 0, st, src, args...);
}

int silu_grid(int rows, int width) {
    const int64_t total = static_cast<int64_t>(rows) * (width / 8);
    int64_t grid = (total + 255) / 256;
    return static_cast<int>(grid > 4096 ? 4096 : grid);
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }


// out[r] = t0[first_ids[r]] + t[0][ids[0][r]] + ... + t[G-1][ids[G-1][r]], the
// adds in group order with each partial sum rounded to bf16 (the value of
// adding the rows one launch at a time in bf16).  One thread per 8 columns of
// a row; an id outside its table reads row 0 and reports in *status.
__global__ void __launch_bounds__(256)
gather_sum_rows_kernel(const int64_t *__restrict__ first_ids, const uint16_t *__restrict__ first_table,
                       int64_t first_s0, int64_t first_rows, const int64_t *__restrict__ ids, int64_t ids_s0,
                       int64_t ids_s1, const uint16_t *__restrict__ tables, int64_t table_s0, int64_t table_s1,
                       int64_t table_rows, int groups, int rows, int width, uint16_t *__restrict__ out,
                       int64_t out_s0, int32_t *status) {
    const int nvec = width / 8;
    const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= static_cast<int64_t>(rows) * nvec) return;
    const int r = static_cast<int>(i / nvec), col = static_cast<int>(i % nvec) * 8;
    bool bad = false;
    int64_t id = first_ids[r];
    if (id < 0 || id >= first_rows) {
        bad = true;
        id = 0;
    }
    float acc[8];
    unpack8(*reinterpret_cast<const uint4 *>(first_table + id * first_s0 + col), acc);
    // up to 16 groups per round: every id, then every row, in flight together
    // (indexes past the last group repeat it, so that no load is conditional;
    // their rows are not added)
    constexpr int kRound = 16;
    for (int g0 = 0; g0 < groups; g0 += kRound) {
        int64_t t[kRound];
#pragma unroll
        for (int u = 0; u < kRound; ++u) {
            const int gi = g0 + u < groups ? g0 + u : groups - 1;
            t[u] = ids[gi * ids_s0 + r * ids_s1];
        }
        uint4 rowv[kRound];
#pragma unroll
        for (int u = 0; u < kRound; ++u) {
            const int gi = g0 + u < groups ? g0 + u : groups - 1;
            const bool in = t[u] >= 0 && t[u] < table_rows;
            bad = bad || !in;
            rowv[u] = *reinterpret_cast<const uint4 *>(tables + gi * table_s0 + (in ? t[u] : 0) * table_s1 + col);
        }
#pragma unroll
        for (int u = 0; u < kRound; ++u) {
            float e[8];
            unpack8(rowv[u], e);
            const bool use = g0 + u < groups;
#pragma unroll
            for (int k = 0; k < 8; ++k) acc[k] = use ? bf16_to_f32(f32_to_bf16(acc[k] + e[k])) : acc[k];
        }
    }
    uint4 o;
    o.x = pack2_bf16(acc[0], acc[1]);
    o.y = pack2_bf16(acc[2], acc[3]);
    o.z = pack2_bf16(acc[4], acc[5]);
    o.w = pack2_bf16(acc[6], acc[7]);
    *reinterpret_cast<uint4 *>(out + r * out_s0 + col) = o;
    if (bad && status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
}
}  // namespace

int launch_add_rmsnorm_partials(const float *part, int S, int rows, int width, uint16_t *hidden_out,
                                int64_t ho_s0, uint16_t *residual, const uint16_t *weight, float eps,
                                hipStream_t st) {
    if (width % 8 || width > kNormThreads * 8 * kMaxVec) return NQ_ERR_UNSUPPORTED;
    const PartialSrc src{part, S, static_cast<int64_t>(rows) * width, width};
    launch_add_rmsnorm<PartialSrc, false>(rows, width, st, src, hidden_out, ho_s0, residual, nullptr, 0, weight,
                                          width, eps, Fp8Out{});
    return NQ_LAUNCH_STATUS();
}

int launch_add_rmsnorm_partials_fp8(const float *part, int S, int rows, int width, uint16_t *residual,
                                    const uint16_t *weight, float eps, uint8_t *xq, int64_t xq_s0, float *sx,
                                    int64_t sx_s0, hipStream_t st) {
    if (width % 128 || width > kNormThreads * 8 * kMaxVec) return NQ_ERR_UNSUPPORTED;
    const PartialSrc src{part, S, static_cast<int64_t>(rows) * width, width};
    launch_add_rmsnorm<PartialSrc, true>(rows, width, st, src, nullptr, 0, residual, nullptr, 0, weight, width,
                                         eps, Fp8Out{xq, xq_s0, sx, sx_s0});
    return NQ_LAUNCH_STATUS();
}

int launch_silu_mul_partials(const float *part, int S, int rows, int width, uint16_t *out, int64_t o_s0,
                             hipStream_t st) {
    const PartialSrc src{part, S, static_cast<int64_t>(rows) * 2 * width, 2 * width};
    hipLaunchKernelGGL(silu_mul_kernel<PartialSrc>, dim3(silu_grid(rows, width)), dim3(256), 0, st, src, out,
                       o_s0, rows, width);
    return NQ_LAUNCH_STATUS();
}

}  // namespace nq

extern "C" int nq_add_rmsnorm(uint16_t *hidden, uint16_t *residual, const uint16_t *weight,
                              int rows, int width, float eps, void *stream) {
    NQ_CHECK_ARG(hidden && residual && weight && rows >= 0 && width >= 8);
    if (width % 8 || width > nq::kNormThreads * 8 * nq::kMaxVec) return NQ_ERR_UNSUPPORTED;
    if (!nq::al16(hidden) || !nq::al16(residual) || !nq::al16(weight)) return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    const nq::Bf16Src src{hidden, width};
    nq::launch_add_rmsnorm<nq::Bf16Src, false>(rows, width, static_cast<hipStream_t>(stream), src, hidden,
                                               static_cast<int64_t>(width), residual, nullptr, 0, weight, width,
                                               eps, nq::Fp8Out{});
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_add_rmsnorm_fp8(const uint16_t *hidden, uint16_t *residual, const uint16_t *weight, int rows,
                                  int width, float eps, uint8_t *xq, int64_t xq_s0, float *sx, int64_t sx_s0,
                                  void *stream) {
    NQ_CHECK_ARG(hidden && residual && weight && xq && sx && rows >= 0 && width >= 128);
    if (width % 128 || width > nq::kNormThreads * 8 * nq::kMaxVec) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(xq_s0 >= width && xq_s0 % 8 == 0 && sx_s0 >= width / 128);
    if (!nq::al16(hidden) || !nq::al16(residual) || !nq::al16(weight) || reinterpret_cast<uintptr_t>(xq) % 8)
        return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    const nq::Bf16Src src{hidden, width};
    nq::launch_add_rmsnorm<nq::Bf16Src, true>(rows, width, static_cast<hipStream_t>(stream), src, nullptr, 0,
                                              residual, nullptr, 0, weight, width, eps,
                                              nq::Fp8Out{xq, xq_s0, sx, sx_s0});
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_rmsnorm(const uint16_t *x, const uint16_t *weight, uint16_t *out, int rows,
                          int width, float eps, void *stream) {
    NQ_CHECK_ARG(x && weight && out && rows >= 0 && width >= 8);
    if (width % 8 || width > nq::kNormThreads * 8 * nq::kMaxVec) return NQ_ERR_UNSUPPORTED;
    if (!nq::al16(x) || !nq::al16(weight) || !nq::al16(out)) return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    hipLaunchKernelGGL(nq::rmsnorm_kernel, dim3(rows), dim3(nq::kNormThreads), 0,
                       static_cast<hipStream_t>(stream), x, weight, out, width, eps);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_silu_mul(const uint16_t *gate_up, uint16_t *out, int rows, int width,
                           void *stream) {
    NQ_CHECK_ARG(gate_up && out && rows >= 0 && width >= 8);
    if (width % 8) return NQ_ERR_UNSUPPORTED;
    if (!nq::al16(gate_up) || !nq::al16(out)) return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    const nq::Bf16Src src{gate_up, 2 * static_cast<int64_t>(width)};
    hipLaunchKernelGGL(nq::silu_mul_kernel<nq::Bf16Src>, dim3(nq::silu_grid(rows, width)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), src, out, static_cast<int64_t>(width), rows, width);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_embed_add_rmsnorm(const int64_t *ids, const uint16_t *table, int64_t table_s0, int64_t num_embeddings,
                                    const uint16_t *addend, int64_t addend_s0, const uint16_t *weight, int rows,
                                    int width, float eps, uint16_t *residual, uint16_t *out, int32_t *status,
                                    void *stream) {
    NQ_CHECK_ARG(ids && table && weight && residual && out && rows >= 0 && width >= 8);
    NQ_CHECK_ARG(num_embeddings >= 1 && table_s0 >= width && (!addend || addend_s0 >= width));
    if (width % 8 || width > nq::kNormThreads * 8 * nq::kMaxVec) return NQ_ERR_UNSUPPORTED;
    if (!nq::al16(table) || (addend && !nq::al16(addend)) || !nq::al16(weight) || !nq::al16(residual) ||
        !nq::al16(out) || table_s0 % 8 || (addend && addend_s0 % 8))
        return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    const nq::GatherSrc src{table, table_s0, ids, num_embeddings, status};
    if (!addend) {  // residual = the gathered row
        nq::launch_add_rmsnorm<nq::GatherSrc, false, false>(rows, width, static_cast<hipStream_t>(stream), src, out,
                                                            static_cast<int64_t>(width), residual, nullptr, 0,
                                                            weight, width, eps, nq::Fp8Out{});
        return NQ_LAUNCH_STATUS();
    }
    nq::launch_add_rmsnorm<nq::GatherSrc, false>(rows, width, static_cast<hipStream_t>(stream), src, out,
                                                 static_cast<int64_t>(width), residual, addend, addend_s0, weight,
                                                 width, eps, nq::Fp8Out{});
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_prefill_embed_rmsnorm(const int64_t *text_ids, const uint16_t *text_table, int64_t text_s0,
                                        int64_t text_rows, const int64_t *codec_ids, const uint16_t *codec_table,
                                        int64_t codec_s0, int64_t codec_rows, const uint8_t *mask,
                                        const uint16_t *weight, int rows, int width, float eps, uint16_t *residual,
                                        uint16_t *out, int32_t *status, void *stream) {
    NQ_CHECK_ARG(text_ids && text_table && codec_ids && codec_table && mask && weight && residual && out);
    NQ_CHECK_ARG(rows >= 0 && width >= 8 && text_rows >= 1 && codec_rows >= 1 && text_s0 >= width &&
                 codec_s0 >= width);
    if (width % 8 || width > nq::kNormThreads * 8 * nq::kMaxVec || text_s0 % 8 || codec_s0 % 8 ||
        !nq::al16(text_table) || !nq::al16(codec_table) || !nq::al16(residual) || !nq::al16(out))
        return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    const nq::MaskedPairSrc src{nq::GatherSrc{text_table, text_s0, text_ids, text_rows, status},
                                nq::GatherSrc{codec_table, codec_s0, codec_ids, codec_rows, status}, mask};
    nq::launch_add_rmsnorm<nq::MaskedPairSrc, false, false>(rows, width, static_cast<hipStream_t>(stream), src, out,
                                                             static_cast<int64_t>(width), residual, nullptr, 0,
                                                             weight, width, eps, nq::Fp8Out{});
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_gather_sum_rows(const int64_t *first_ids, const uint16_t *first_table, int64_t first_s0,
                                  int64_t first_rows, const int64_t *ids, int64_t ids_s0, int64_t ids_s1,
                                  const uint16_t *tables, int64_t table_s0, int64_t table_s1, int64_t table_rows,
                                  int groups, int rows, int width, uint16_t *out, int64_t out_s0, int32_t *status,
                                  void *stream) {
    NQ_CHECK_ARG(first_ids && first_table && out && rows >= 0 && width >= 8 && groups >= 0);
    NQ_CHECK_ARG(first_rows >= 1 && first_s0 >= width && out_s0 >= width);
    NQ_CHECK_ARG(groups == 0 || (ids && tables && table_rows >= 1 && table_s1 >= width));
    if (width % 8 || first_s0 % 8 || out_s0 % 8 || (groups && (table_s1 % 8 || table_s0 % 8)) ||
        !nq::al16(first_table) || !nq::al16(out) || (groups && !nq::al16(tables)))
        return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    const int64_t threads = static_cast<int64_t>(rows) * (width / 8);
    hipLaunchKernelGGL(nq::gather_sum_rows_kernel, dim3(static_cast<unsigned>((threads + 255) / 256)), dim3(256), 0,
                       static_cast<hipStream_t>(stream), first_ids, first_table, first_s0, first_rows, ids, ids_s0,
                       ids_s1, tables, table_s0, table_s1, table_rows, groups, rows, width, out, out_s0, status);
    return NQ_LAUNCH_STATUS();
}
