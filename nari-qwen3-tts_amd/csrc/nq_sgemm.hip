// fp32 GEMM with fused epilogues for the incremental codec decoder (which runs
// in fp32, executor/build.py:91-95): the transformer's linear layers
// (model/incremental_codec.py:193-381), the ConvNeXt pointwise layers and the
// im2col forms of the causal convolutions and transposed convolutions.
//
//   out[m, n] = res[m, n] + scale[n] * act(sum_k X[row(m), k] W[n, k] + bias[n])
//
// with each of res, scale, bias optional, act none or GELU (erf form, as
// torch.nn.functional.gelu), and row(m) = m or x_rows[m] (a row gather).  The
// products run on v_mfma_f32_16x16x4_f32 (full fp32 products and sums, no
// reduced-precision inputs).  A workgroup owns a BM x BN tile, its WM x WN
// waves a (16 MT) x (16 NT) block each; 32-wide K slices of the X and W
// tiles are staged through LDS, double buffered, with two slices of global
// loads in flight (a K tail reads as zero, columns past N are not stored).
// Both operands are K-contiguous: a lane's 16-byte LDS read holds 4
// consecutive k of one row, which feed the 4 MFMAs of a 16-k group
// (MFMA t sums k = 4 q + t over the lane groups q), so A and B take the same k.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kSgK = 32;            // K floats per stage
constexpr int kSgPitch = kSgK + 8;  // LDS row pitch in floats (32 bytes of padding)

bool sg_al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

// The thread's vectors of one stage: every vector of a thread has the same 4-float chunk of its row,
// so one test covers the K tail (chunks at or past K read as zero; K % 4 == 0).
template <int XV, int WV>
__device__ __forceinline__ void sg_load(floatx4_t (&xr)[XV], floatx4_t (&wr)[WV], const float *const (&xp)[XV],
                                        const float *const (&wp)[WV], int stage, int k_left) {
    const int k0 = stage * kSgK;
    const bool in = k0 < k_left;
#pragma unroll
    for (int q = 0; q < WV; ++q)
        wr[q] = in ? *reinterpret_cast<const floatx4_t *>(wp[q] + k0) : floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int q = 0; q < XV; ++q)
        xr[q] = in ? *reinterpret_cast<const floatx4_t *>(xp[q] + k0) : floatx4_t{0.f, 0.f, 0.f, 0.f};
}

// vector i = threadIdx.x + T q: tile row i / 8, 4-float chunk i % 8
template <int XV, int WV, int T>
__device__ __forceinline__ void sg_store(const floatx4_t (&xr)[XV], const floatx4_t (&wr)[WV], float *xbuf,
                                         float *wbuf) {
#pragma unroll
    for (int q = 0; q < XV; ++q) {
        const int i = threadIdx.x + q * T;
        *reinterpret_cast<floatx4_t *>(xbuf + (i >> 3) * kSgPitch + (i & 7) * 4) = xr[q];
    }
#pragma unroll
    for (int q = 0; q < WV; ++q) {
        const int i = threadIdx.x + q * T;
        *reinterpret_cast<floatx4_t *>(wbuf + (i >> 3) * kSgPitch + (i & 7) * 4) = wr[q];
    }
}

template <int MT, int NT>
__device__ __forceinline__ void sg_compute(floatx4_t (&acc)[MT][NT], const float *xt, const float *wt) {
#pragma unroll
    for (int g = 0; g < kSgK / 16; ++g) {
        floatx4_t a[NT], b[MT];
#pragma unroll
        for (int n = 0; n < NT; ++n) a[n] = *reinterpret_cast<const floatx4_t *>(wt + n * 16 * kSgPitch + g * 16);
#pragma unroll
        for (int m = 0; m < MT; ++m) b[m] = *reinterpret_cast<const floatx4_t *>(xt + m * 16 * kSgPitch + g * 16);
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int m = 0; m < MT; ++m)
#pragma unroll
                for (int n = 0; n < NT; ++n)
                    acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[n][t], b[m][t], acc[m][n], 0, 0, 0);
    }
}

__device__ __forceinline__ float sg_gelu(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f)); }

template <int MT, int NT, int WM, int WN>
__global__ void __launch_bounds__(WM * WN * kWave)
sgemm_kernel(const float *__restrict__ x, int64_t x_s0, const int32_t *__restrict__ x_rows, int M,
             const float *__restrict__ w, int64_t w_s0, int N, int K, const float *__restrict__ bias, int act,
             const float *res, int64_t r_s0, const float *__restrict__ scale, float *out, int64_t o_s0, int tiles_m,
             int units) {
    constexpr int T = WM * WN * kWave;
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    constexpr int XV = BM * (kSgK / 4) / T;  // 16-byte vectors per thread and stage
    constexpr int WV = BN * (kSgK / 4) / T;
    static_assert(XV >= 1 && WV >= 1 && XV * T == BM * kSgK / 4 && WV * T == BN * kSgK / 4,
                  "stage splits evenly over the threads");
    __shared__ __attribute__((aligned(16))) float xs[2][BM * kSgPitch];
    __shared__ __attribute__((aligned(16))) float ws[2][BN * kSgPitch];

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
        int row = m0 + (i >> 3);
        row = row < M ? row : M - 1;
        if (x_rows) row = x_rows[row];
        xp[q] = x + static_cast<int64_t>(row) * x_s0 + (i & 7) * 4;
    }
#pragma unroll
    for (int q = 0; q < WV; ++q) {
        const int i = threadIdx.x + q * T;
        const int n = n0 + (i >> 3);  // rows past N repeat row N - 1; their columns are not stored
        wp[q] = w + static_cast<int64_t>(n < N ? n : N - 1) * w_s0 + (i & 7) * 4;
    }
    const int k_left = K - (threadIdx.x & 7) * 4;  // stage k0 is inside K for this thread while k0 < k_left

    floatx4_t acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[m][n] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    const float *xt0 = xs[0] + (wm * 16 * MT + r16) * kSgPitch + kq * 4;
    const float *wt0 = ws[0] + (wn * 16 * NT + r16) * kSgPitch + kq * 4;
    const float *xt1 = xs[1] + (wm * 16 * MT + r16) * kSgPitch + kq * 4;
    const float *wt1 = ws[1] + (wn * 16 * NT + r16) * kSgPitch + kq * 4;

    // stage j sits in register set j % 2 (a, b) and LDS buffer j % 2.  Step k: MFMAs on buffer
    // k % 2, stage k + 1 to LDS, then the loads of stage k + 3 into the set stage k + 1 left free.
    floatx4_t xa[XV], wa[WV], xb[XV], wb[WV];
    const int stages = (K + kSgK - 1) / kSgK;
    sg_load<XV, WV>(xa, wa, xp, wp, 0, k_left);
    sg_store<XV, WV, T>(xa, wa, xs[0], ws[0]);
    if (stages > 1) sg_load<XV, WV>(xb, wb, xp, wp, 1, k_left);
    if (stages > 2) sg_load<XV, WV>(xa, wa, xp, wp, 2, k_left);
    __syncthreads();
    for (int k = 0;; k += 2) {
        sg_compute<MT, NT>(acc, xt0, wt0);
        if (k + 1 < stages) sg_store<XV, WV, T>(xb, wb, xs[1], ws[1]);
        if (k + 3 < stages) sg_load<XV, WV>(xb, wb, xp, wp, k + 3, k_left);
        __syncthreads();
        if (k + 1 >= stages) break;
        sg_compute<MT, NT>(acc, xt1, wt1);
        if (k + 2 < stages) sg_store<XV, WV, T>(xa, wa, xs[0], ws[0]);
        if (k + 4 < stages) sg_load<XV, WV>(xa, wa, xp, wp, k + 4, k_left);
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

template <int MT, int NT, int WM, int WN>
int launch_sgemm(const float *x, int64_t x_s0, const int32_t *x_rows, int M, const float *w, int64_t w_s0, int N,
                 int K, const float *bias, int act, const float *res, int64_t r_s0, const float *scale, float *out,
                 int64_t o_s0, hipStream_t st) {
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    const int tiles_m = (M + BM - 1) / BM, units = tiles_m * ((N + BN - 1) / BN);
    hipLaunchKernelGGL((sgemm_kernel<MT, NT, WM, WN>), dim3((units + 7) / 8 * 8), dim3(WM * WN * kWave), 0, st, x,
                       x_s0,
                       x_rows, M, w, w_s0, N, K, bias, act, res, r_s0, scale, out, o_s0, tiles_m, units);
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

extern "C" int nq_sgemm(const float *x, int64_t x_s0, const int32_t *x_rows, const float *w, int64_t w_s0, int M,
                        int N, int K, const float *bias, int act, const float *res, int64_t r_s0, const float *scale,
                        float *out, int64_t o_s0, void *stream) {
    NQ_CHECK_ARG(x && w && out && M >= 0 && N > 0 && K > 0 && (act == 0 || act == 1));
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K && o_s0 >= N && (!res || r_s0 >= N));
    if (K % 4 || N % 4 || x_s0 % 4 || w_s0 % 4 || o_s0 % 4 || (res && r_s0 % 4) || !sg_al16(x) ||
        !sg_al16(w) || !sg_al16(out) || (res && !sg_al16(res)) || (bias && !sg_al16(bias)) ||
        (scale && !sg_al16(scale)))
        return NQ_ERR_UNSUPPORTED;
    if (M == 0) return NQ_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    // the largest tile that still gives every CU a workgroup (fp32 MFMA work per staged byte is high,
    // so small tiles lose little and idle CUs lose much)
    auto units = [&](int bm, int bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn); };
#define NQ_SG(MT, NT, WM, WN) \
    launch_sgemm<MT, NT, WM, WN>(x, x_s0, x_rows, M, w, w_s0, N, K, bias, act, res, r_s0, scale, out, o_s0, st)
    // 128 x 128 and 64 x 128 tiles over 16 and 8 waves of 32 x 32, 64 x 64 over 8 waves of 16 x 32: more
    // waves per CU hide the stage latency (the codec step's GEMMs 1.30 -> 1.21 ms against 4 waves per tile)
    if (units(128, 128) >= 256) return NQ_SG(2, 2, 4, 4);
    if (units(64, 128) >= 256) return NQ_SG(2, 2, 2, 4);
    if (units(64, 64) >= 256) return NQ_SG(1, 2, 4, 2);
    if (units(32, 64) >= 256) return NQ_SG(1, 2, 2, 2);
    return NQ_SG(1, 1, 2, 2);
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
