// fp32 GEMM with fused epilogues for the incremental codec decoder (which runs
// in fp32, executor/build.py:91-95): the transformer's linear layers
// (model/incremental_codec.py:193-381), the ConvNeXt pointwise layers and the
// im2col forms of the causal convolutions and transposed convolutions.
//
//   out[m, n] = res[m, n] + scale[n] * act(sum_k X[row(m), k] W[n, k] + bias[n])
//
// with each of res, scale, bias optional, act none or GELU (erf form, as
// torch.nn.functional.gelu), and row(m) = m or x_rows[m] (a row gather).
//
// Two product precisions, torch's float32 matmul precisions by name:
// - "highest": v_mfma_f32_16x16x4_f32, full fp32 products and sums.
// - "high" (the reference's serving policy, model/checkpoint.py:46-49 sets
//   torch.set_float32_matmul_precision("high")): each fp32 operand is the sum
//   of two bf16, v = hi + lo + e with hi = bf16(v), lo = bf16(v - hi) and
//   |e| <= 2^-16 |v|, and a product is hi*hi + hi*lo + lo*hi on
//   v_mfma_f32_16x16x32_bf16 (each bf16 product exact in fp32, fp32 sums), so
//   each product is within 3 * 2^-16 of x*w -- the "sum of two bfloat16"
//   form torch documents for that precision.  The three MFMAs of a 32-k step
//   cost about a fifth of the eight fp32 MFMAs of the same step.
//
// A workgroup owns a BM x BN tile, its WM x WN waves a (16 MT) x (16 NT) block
// each; 32-wide K slices of the X and W tiles are staged through LDS, double
// buffered, with two slices of global loads in flight (a K tail reads as zero,
// columns past N are not stored).  Both operands are K-contiguous.  fp32
// stages: a lane's 16-byte LDS read holds 4 consecutive k of one row, which
// feed the 4 MFMAs of a 16-k group (MFMA t sums k = 4 q + t over the lane
// groups q), so A and B take the same k.  Split stages: the fp32 slice is
// split while it is written to LDS, a row holding its 32 hi then its 32 lo
// values, and a lane's 16-byte read is the 8 consecutive k of one 32-k MFMA
// operand.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float floatx2_t __attribute__((ext_vector_type(2)));

// LDS row of a stage of KS k: KS fp32, or KS hi then KS lo bf16, then 32 bytes of padding (a row offset of
// 32 bytes modulo 128 spreads a 16-byte read of 16 rows over the banks)
template <int KS>
constexpr int sg_row_bytes() {
    return KS * 4 + 32;
}

bool sg_al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The thread's vectors of one stage: every vector of a thread has the same 4-float chunk of its row,
// so one test covers the K tail (chunks at or past K read as zero; K % 4 == 0).
template <int KS, int XV, int WV>
__device__ __forceinline__ void sg_load(floatx4_t (&xr)[XV], floatx4_t (&wr)[WV], const float *const (&xp)[XV],
                                        const float *const (&wp)[WV], int stage, int k_left) {
    const int k0 = stage * KS;
    const bool in = k0 < k_left;
#pragma unroll
    for (int q = 0; q < WV; ++q)
        wr[q] = in ? *reinterpret_cast<const floatx4_t *>(wp[q] + k0) : floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < XV; ++q)
        xr[q] = in ? *reinterpret_cast<const floatx4_t *>(xp[q] + k0) : floatx4_t{0.f, 0.f, 0.f, 0.f};
}

// v = hi + lo + e: hi = bf16(v), lo = bf16(v - hi) (round to nearest even, v_cvt_pk_bf16_f32; v - hi is
// exact in fp32), |e| <= 2^-16 |v|
__device__ __forceinline__ uint32_t sg_pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((floatx2_t){a, b}, bf16x2_t));
}
__device__ __forceinline__ void sg_split(const floatx4_t &v, uint2 &hi, uint2 &lo) {
    hi.x = sg_pack(v[0], v[1]);
    hi.y = sg_pack(v[2], v[3]);
    lo.x = sg_pack(v[0] - __uint_as_float(hi.x << 16), v[1] - __uint_as_float(hi.x & 0xffff0000u));
    lo.y = sg_pack(v[2] - __uint_as_float(hi.y << 16), v[3] - __uint_as_float(hi.y & 0xffff0000u));
}

// One register set into LDS.  Vector i = threadIdx.x + T q: tile row i / (KS / 4), 4-float chunk
// c = i % (KS / 4) (k = 4c .. 4c + 3 of the stage): fp32 at byte 16 c of the row, or split, hi at byte
// 8 c and lo at byte 2 KS + 8 c.
template <int KS, int V, int T, bool kSplit>
__device__ __forceinline__ void sg_store_rows(const floatx4_t (&r)[V], char *buf) {
    constexpr int C = KS / 4;
#pragma unroll
    for (int q = 0; q < V; ++q) {
        const int i = threadIdx.x + q * T;
        char *row = buf + (i / C) * sg_row_bytes<KS>();
        if constexpr (kSplit) {
            uint2 hi, lo;
            sg_split(r[q], hi, lo);
            *reinterpret_cast<uint2 *>(row + (i % C) * 8) = hi;
            *reinterpret_cast<uint2 *>(row + 2 * KS + (i % C) * 8) = lo;
        } else {
            *reinterpret_cast<floatx4_t *>(row + (i % C) * 16) = r[q];
        }
    }
}

// The MFMAs of one staged slice on the wave's (16 MT) x (16 NT) block; xt / wt point at the lane's row
// (r16) of the wave's first tile, plus 16 kq bytes.
template <int MT, int NT, int KS, bool kSplit>
__device__ __forceinline__ void sg_compute(floatx4_t (&acc)[MT][NT], const char *xt, const char *wt) {
    constexpr int RB = sg_row_bytes<KS>();
    if constexpr (kSplit) {
        // lane (r16, kq): k = 32 j + 8 kq .. + 7 of 32-k step j, the same k in A (W rows) and B (X rows)
#pragma unroll
        for (int j = 0; j < KS / 32; ++j) {
            bf16x8_t ah[NT], al[NT], bh[MT], bl[MT];
#pragma unroll
            for (int n = 0; n < NT; ++n) {
                ah[n] = *reinterpret_cast<const bf16x8_t *>(wt + n * 16 * RB + j * 64);
                al[n] = *reinterpret_cast<const bf16x8_t *>(wt + n * 16 * RB + 2 * KS + j * 64);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m) {
                bh[m] = *reinterpret_cast<const bf16x8_t *>(xt + m * 16 * RB + j * 64);
                bl[m] = *reinterpret_cast<const bf16x8_t *>(xt + m * 16 * RB + 2 * KS + j * 64);
            }
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int n = 0; n < NT; ++n) {
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[n], bh[m], acc[m][n], 0, 0, 0);
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[n], bl[m], acc[m][n], 0, 0, 0);
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[n], bh[m], acc[m][n], 0, 0, 0);
                }
        }
    } else {
        // lane (r16, kq): k = 16 g + 4 kq + t feeds MFMA t of 16-k group g
#pragma unroll
        for (int g = 0; g < KS / 16; ++g) {
            floatx4_t a[NT], b[MT];
#pragma unroll
            for (int n = 0; n < NT; ++n)
                a[n] = *reinterpret_cast<const floatx4_t *>(wt + n * 16 * RB + g * 64);
#pragma unroll
            for (int m = 0; m < MT; ++m)
                b[m] = *reinterpret_cast<const floatx4_t *>(xt + m * 16 * RB + g * 64);
#pragma unroll
            for (int t = 0; t < 4; ++t)
#pragma unroll
                for (int m = 0; m < MT; ++m)
#pragma unroll
                    for (int n = 0; n < NT; ++n)
                        acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[n][t], b[m][t], acc[m][n], 0, 0, 0);
        }
    }
}

__device__ __forceinline__ float sg_gelu(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f)); }

template <int MT, int NT, int WM, int WN, int KS, bool kSplit>
__global__ void __launch_bounds__(WM * WN * kWave)
sgemm_kernel(const float *__restrict__ x, int64_t x_s0, const int32_t *__restrict__ x_rows, int M,
             const float *__restrict__ w, int64_t w_s0, int N, int K, const float *__restrict__ bias, int act,
             const float *res, int64_t r_s0, const float *__restrict__ scale, float *out, int64_t o_s0, int tiles_m,
             int units) {
    constexpr int T = WM * WN * kWave;
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    constexpr int C = KS / 4;  // 16-byte chunks per row and stage
    constexpr int RB = sg_row_bytes<KS>();
    constexpr int XV = BM * C / T;  // 16-byte vectors per thread and stage
    constexpr int WV = BN * C / T;
    static_assert(XV >= 1 && WV >= 1 && XV * T == BM * C && WV * T == BN * C && T % C == 0,
                  "stage splits evenly over the threads, one chunk column per thread");
    __shared__ __attribute__((aligned(16))) char xs[2][BM * RB];
    __shared__ __attribute__((aligned(16))) char ws[2][BN * RB];

    // tile of this workgroup: XCD b % 8 takes tiles (b % 8) * per .. + per - 1, m fastest
    const int per = (units + 7) / 8;
    const int t = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (t >= units) return;
    const int m0 = (t % tiles_m) * BM, n0 = (t / tiles_m) * BN;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15, kq = lane >> 4;
    const int wm = wave % WM, wn = wave / WM;

    const float *xp[XV];
    const float *wp[WV];
#pragma unroll
    for (int q = 0; q < XV; ++q) {
        const int i = threadIdx.x + q * T;
        int row = m0 + i / C;
        row = row < M ? row : M - 1;
        if (x_rows) row = x_rows[row];
        xp[q] = x + static_cast<int64_t>(row) * x_s0 + (i % C) * 4;
    }
#pragma unroll
    for (int q = 0; q < WV; ++q) {
        const int i = threadIdx.x + q * T;
        const int n = n0 + i / C;  // rows past N repeat row N - 1; their columns are not stored
        wp[q] = w + static_cast<int64_t>(n < N ? n : N - 1) * w_s0 + (i % C) * 4;
    }
    const int k_left = K - (threadIdx.x % C) * 4;  // stage k0 is inside K for this thread while k0 < k_left

    floatx4_t acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[m][n] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    const int x_off = (wm * 16 * MT + r16) * RB + kq * 16;
    const int w_off = (wn * 16 * NT + r16) * RB + kq * 16;
    auto store = [&](const floatx4_t (&xr)[XV], const floatx4_t (&wr)[WV], int buf) __attribute__((always_inline)) {
        sg_store_rows<KS, XV, T, kSplit>(xr, xs[buf]);
        sg_store_rows<KS, WV, T, kSplit>(wr, ws[buf]);
    };

    // stage j sits in register set j % 2 (a, b) and LDS buffer j % 2.  Step k: MFMAs on buffer
    // k % 2, stage k + 1 to LDS, then the loads of stage k + 3 into the set stage k + 1 left free.
    floatx4_t xa[XV], wa[WV], xb[XV], wb[WV];
    const int stages = (K + KS - 1) / KS;
    sg_load<KS, XV, WV>(xa, wa, xp, wp, 0, k_left);
    store(xa, wa, 0);
    if (stages > 1) sg_load<KS, XV, WV>(xb, wb, xp, wp, 1, k_left);
    if (stages > 2) sg_load<KS, XV, WV>(xa, wa, xp, wp, 2, k_left);
    __syncthreads();
    for (int k = 0;; k += 2) {
        sg_compute<MT, NT, KS, kSplit>(acc, xs[0] + x_off, ws[0] + w_off);
        if (k + 1 < stages) store(xb, wb, 1);
        if (k + 3 < stages) sg_load<KS, XV, WV>(xb, wb, xp, wp, k + 3, k_left);
        __syncthreads();
        if (k + 1 >= stages) break;
        sg_compute<MT, NT, KS, kSplit>(acc, xs[1] + x_off, ws[1] + w_off);
        if (k + 2 < stages) store(xa, wa, 0);
        if (k + 4 < stages) sg_load<KS, XV, WV>(xa, wa, xp, wp, k + 4, k_left);
        __syncthreads();
        if (k + 2 >= stages) break;
    }

    // the lane holds Y[m0 + wm 16 MT + 16 m + r16][n0 + wn 16 NT + 16 n + 4 kq + e]
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        const int col = n0 + wn * 16 * NT + n * 16 + kq * 4;
        if (col >= N) continue;
        floatx4_t bv = floatx4_t{0.f, 0.f, 0.f, 0.f}, sv = floatx4_t{1.f, 1.f, 1.f, 1.f};
        if (bias) bv = *reinterpret_cast<const floatx4_t *>(bias + col);
        if (scale) sv = *reinterpret_cast<const floatx4_t *>(scale + col);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int row = m0 + wm * 16 * MT + m * 16 + r16;
            if (row >= M) continue;
            floatx4_t v;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float y = acc[m][n][e] + bv[e];
                if (act) y = sg_gelu(y);
                v[e] = y * sv[e];
            }
            if (res) {
                const floatx4_t r = *reinterpret_cast<const floatx4_t *>(res + static_cast<int64_t>(row) * r_s0 + col);
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = r[e] + v[e];
            }
            *reinterpret_cast<floatx4_t *>(out + static_cast<int64_t>(row) * o_s0 + col) = v;
        }
    }
}

template <int MT, int NT, int WM, int WN, int KS, bool kSplit>
int launch_sgemm(const float *x, int64_t x_s0, const int32_t *x_rows, int M, const float *w, int64_t w_s0, int N,
                 int K, const float *bias, int act, const float *res, int64_t r_s0, const float *scale, float *out,
                 int64_t o_s0, hipStream_t st) {
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    const int tiles_m = (M + BM - 1) / BM, units = tiles_m * ((N + BN - 1) / BN);
    hipLaunchKernelGGL((sgemm_kernel<MT, NT, WM, WN, KS, kSplit>), dim3((units + 7) / 8 * 8), dim3(WM * WN * kWave), 0,
                       st, x, x_s0, x_rows, M, w, w_s0, N, K, bias, act, res, r_s0, scale, out, o_s0, tiles_m, units);
    return NQ_LAUNCH_STATUS();
}

// Row-parallel RMSNorm / LayerNorm of fp32 rows (one wave per row, width % 4 == 0, width <= 1024):
// RMS: x * rsqrt(mean(x^2) + eps) * w;  LayerNorm: (x - mean) * rsqrt(var + eps) * w + b.
template <bool kLayer>
__global__ void __launch_bounds__(256)
row_norm_kernel(const float *__restrict__ x, int64_t x_s0, int rows, int width, const float *__restrict__ w,
                const float *__restrict__ b, float eps, float *__restrict__ out, int64_t o_s0) {
    const int row = blockIdx.x * 4 + threadIdx.x / kWave;
    const int lane = threadIdx.x & (kWave - 1);
    if (row >= rows) return;
    const float *xr = x + static_cast<int64_t>(row) * x_s0;
    constexpr int kMaxVec = 4;  // 4 float4 per lane: width <= 1024
    float4 v[kMaxVec];
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const int c = (lane + i * kWave) * 4;
        v[i] = c < width ? *reinterpret_cast<const float4 *>(xr + c) : make_float4(0.f, 0.f, 0.f, 0.f);
        s += kLayer ? (v[i].x + v[i].y) + (v[i].z + v[i].w)
                    : (v[i].x * v[i].x + v[i].y * v[i].y) + (v[i].z * v[i].z + v[i].w * v[i].w);
    }
    s = group_sum<kWave>(s);
    float mean = 0.f, inv;
    if constexpr (kLayer) {
        mean = s / static_cast<float>(width);
        float q = 0.f;
#pragma unroll
        for (int i = 0; i < kMaxVec; ++i) {
            const int c = (lane + i * kWave) * 4;
            if (c < width) {
                const float a = v[i].x - mean, bb = v[i].y - mean, cc = v[i].z - mean, d = v[i].w - mean;
                q += (a * a + bb * bb) + (cc * cc + d * d);
            }
        }
        q = group_sum<kWave>(q);
        inv = rsqrtf(q / static_cast<float>(width) + eps);
    } else {
        inv = rsqrtf(s / static_cast<float>(width) + eps);
    }
    float *orow = out + static_cast<int64_t>(row) * o_s0;
#pragma unroll
    for (int i = 0; i < kMaxVec; ++i) {
        const int c = (lane + i * kWave) * 4;
        if (c >= width) continue;
        const float4 wv = *reinterpret_cast<const float4 *>(w + c);
        float4 o;
        if constexpr (kLayer) {
            const float4 bv = *reinterpret_cast<const float4 *>(b + c);
            o = make_float4((v[i].x - mean) * inv * wv.x + bv.x, (v[i].y - mean) * inv * wv.y + bv.y,
                            (v[i].z - mean) * inv * wv.z + bv.z, (v[i].w - mean) * inv * wv.w + bv.w);
        } else {
            o = make_float4(v[i].x * inv * wv.x, v[i].y * inv * wv.y, v[i].z * inv * wv.z, v[i].w * inv * wv.w);
        }
        *reinterpret_cast<float4 *>(orow + c) = o;
    }
}

// Row index of each stream's last fresh frame at the stage with u rows per frame:
// rows[b] = max(off[b + 1] * u - 1, 0).
__global__ void last_rows_kernel(const int32_t *__restrict__ off, int B, int u, int32_t *__restrict__ rows) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b < B) {
        const int r = off[b + 1] * u - 1;
        rows[b] = r > 0 ? r : 0;
    }
}

}  // namespace
}  // namespace nq

using namespace nq;

// K columns per stage of each tile shape (smaller tiles take deeper stages)
constexpr int kSgKs64x128 = 32, kSgKs64x64 = 64, kSgKs32x64 = 64, kSgKs32x32 = 128;

extern "C" int nq_sgemm(const float *x, int64_t x_s0, const int32_t *x_rows, const float *w, int64_t w_s0, int M,
                        int N, int K, const float *bias, int act, const float *res, int64_t r_s0, const float *scale,
                        float *out, int64_t o_s0, int precision, void *stream) {
    NQ_CHECK_ARG(x && w && out && M >= 0 && N > 0 && K > 0 && (act == 0 || act == 1));
    NQ_CHECK_ARG(precision == NQ_MATMUL_HIGHEST || precision == NQ_MATMUL_HIGH);
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K && o_s0 >= N && (!res || r_s0 >= N));
    if (K % 4 || N % 4 || x_s0 % 4 || w_s0 % 4 || o_s0 % 4 || (res && r_s0 % 4) || !sg_al16(x) ||
        !sg_al16(w) || !sg_al16(out) || (res && !sg_al16(res)) || (bias && !sg_al16(bias)) ||
        (scale && !sg_al16(scale)))
        return NQ_ERR_UNSUPPORTED;
    if (M == 0) return NQ_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // the largest tile that still gives every CU a workgroup (MFMA work per staged byte is high, so
    // small tiles lose little and idle CUs lose much)
    auto units = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
#define NQ_SG(MT, NT, WM, WN, KS, SPLIT)                                                                          \
    launch_sgemm<MT, NT, WM, WN, KS, SPLIT>(x, x_s0, x_rows, M, w, w_s0, N, K, bias, act, res, r_s0, scale, out, \
                                            o_s0, st)
    // 128 x 128 and 64 x 128 tiles over 16 and 8 waves of 32 x 32, 64 x 64 over 8 waves of 16 x 32: more
    // waves per CU hide the stage latency (the codec step's fp32 GEMMs 1.30 -> 1.21 ms against 4 waves per
    // tile).  The smaller tiles take more k per stage (fewer barriers and more bytes in flight per wave).
#define NQ_SG_PICK(SPLIT)                                                                \
    if (units(128, 128) >= 256) return NQ_SG(2, 2, 4, 4, 32, SPLIT);                    \
    if (units(64, 128) >= 256) return NQ_SG(2, 2, 2, 4, kSgKs64x128, SPLIT);        \
    if (units(64, 64) >= 256) return NQ_SG(1, 2, 4, 2, kSgKs64x64, SPLIT);          \
    if (units(32, 64) >= 256) return NQ_SG(1, 2, 2, 2, kSgKs32x64, SPLIT);          \
    return NQ_SG(1, 1, 2, 2, kSgKs32x32, SPLIT);
    if (precision == NQ_MATMUL_HIGH) {
        NQ_SG_PICK(true)
    }
    NQ_SG_PICK(false)
#undef NQ_SG_PICK
#undef NQ_SG
}

extern "C" int nq_row_norm(const float *x, int64_t x_s0, int rows, int width, const float *w, const float *b,
                           float eps, float *out, int64_t o_s0, void *stream) {
    NQ_CHECK_ARG(x && w && out && rows >= 0 && width > 0 && x_s0 >= width && o_s0 >= width);
    if (width % 4 || width > 1024 || x_s0 % 4 || o_s0 % 4 || !sg_al16(x) || !sg_al16(w) || !sg_al16(out) ||
        (b && !sg_al16(b)))
        return NQ_ERR_UNSUPPORTED;
    if (rows == 0) return NQ_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const dim3 grid((rows + 3) / 4);
    if (b) {
        hipLaunchKernelGGL(row_norm_kernel<true>, grid, dim3(256), 0, st, x, x_s0, rows, width, w, b, eps, out, o_s0);
    } else {
        hipLaunchKernelGGL(row_norm_kernel<false>, grid, dim3(256), 0, st, x, x_s0, rows, width, w, nullptr, eps, out,
                           o_s0);
    }
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_last_rows(const int32_t *off, int B, int u, int32_t *rows, void *stream) {
    NQ_CHECK_ARG(off && rows && B >= 0 && u >= 1);
    if (B == 0) return NQ_OK;
    hipLaunchKernelGGL(last_rows_kernel, dim3((B + 255) / 256), dim3(256), 0, static_cast<hipStream_t>(stream), off,
                       B, u, rows);
    return NQ_LAUNCH_STATUS();
}
