// Skinny bf16 GEMM for the decode step: Y[M, N] = X[M, K] . W[N, K]^T with
// M <= 128 activation rows and a weight matrix W that is read from HBM exactly
// once.  Replaces the torch/hipBLASLt projections of the talker layer
// (model/layers.py:195-270 QKV / o / gate_up / down, the codec head).
//
// At decode sizes the projection is a weight stream: 64 rows x 2 flops per
// weight byte is far below the MFMA ridge, so the design maximises bytes in
// flight rather than reuse.  A workgroup (4 waves) owns a K slice of KS
// columns and a band of 64 * NTW output columns.  Each wave issues every
// 128-bit load of its 16 * NTW weight rows over the slice at once (one-shot:
// KS / 32 * NTW loads per lane), while the workgroup stages the matching
// X[:, slice] block in LDS.  Then each wave runs the v_mfma_f32_16x16x32_bf16
// chain with W as the A operand (16 output columns x 32 k) and X^T from LDS as
// the B operand (32 k x 16 rows), so a lane ends with four consecutive output
// columns of one row.  Slices of one band write fp32 partials [S, M, N] that a
// second kernel reduces in a fixed order (deterministic, no atomics); with a
// single slice the bf16 result is written directly.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kGemmWaves = kGemmThreads / kWave;

__device__ __forceinline__ bf16x8_t as_bf16x8(const uint4 &v) {
    bf16x8_t r;
    __builtin_memcpy(&r, &v, sizeof(r));
    return r;
}

// LDS row pitch of the staged X block: KS bf16 + 16 bf16 (32 bytes) of
// padding.  gfx950 serves a ds_read_b128 in lane groups that pair rows of
// different 16-byte k chunks; with a 32-byte row offset those groups cover
// every bank once (a 16-byte offset measured 4 conflict cycles per read).
template <int KS>
constexpr int x_pitch() {
    return KS + 16;
}

// Weights of one wave: its 16 rows over the K slice, one 32-k MFMA step per load:
// lane (r16, kq) reads row n_row at k0 + 32 j + 8 kq, 64 bytes of each of 16 rows per load.
template <int KS>
__device__ __forceinline__ void gemm_load_w(uint4 (&wr)[KS / 32], const uint16_t *__restrict__ w, int64_t w_s0,
                                            int n_row, int k0, int kq) {
    const uint16_t *row = w + static_cast<int64_t>(n_row) * w_s0 + k0 + kq * 8;
#pragma unroll
    for (int j = 0; j < KS / 32; ++j) wr[j] = *reinterpret_cast<const uint4 *>(row + j * 32);
}

// MFMA chain of one 16-column tile over the staged slice, then its store:
// the lane holds Y[m*16 + r16][col + kq*4 + 0..3].
template <int MT, int KS>
__device__ __forceinline__ void gemm_tile(const uint4 (&wr)[KS / 32], const uint16_t *xs, int r16, int kq, int M,
                                          int row0, int mr, int N, int col, int slice, uint16_t *__restrict__ out,
                                          int64_t o_s0, float *__restrict__ part, const uint16_t *__restrict__ bias) {
    floatx4_t acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS / 32; ++j) {
        const bf16x8_t a = as_bf16x8(wr[j]);
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const bf16x8_t bx =
                as_bf16x8(*reinterpret_cast<const uint4 *>(xs + (m * 16 + r16) * x_pitch<KS>() + j * 32 + kq * 8));
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, bx, acc[m], 0, 0, 0);
        }
        // bound how far the scheduler hoists LDS reads (register pressure)
        if (j % 2 == 1) __builtin_amdgcn_sched_barrier(0);
    }
    col += kq * 4;
    float b4[4] = {0.f, 0.f, 0.f, 0.f};
    if (bias && !part) {
#pragma unroll
        for (int e = 0; e < 4; ++e) b4[e] = bf16_to_f32(bias[col + e]);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int lr = m * 16 + r16;  // row within the block
        if (lr >= mr) continue;
        const int row = row0 + lr;
        if (part) {
            float *p = part + (static_cast<int64_t>(slice) * M + row) * N + col;
            *reinterpret_cast<float4 *>(p) = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
        } else {
            uint2 o;
            o.x = pack2_bf16(acc[m][0] + b4[0], acc[m][1] + b4[1]);
            o.y = pack2_bf16(acc[m][2] + b4[2], acc[m][3] + b4[3]);
            *reinterpret_cast<uint2 *>(out + static_cast<int64_t>(row) * o_s0 + col) = o;
        }
    }
}

// Workgroup (bx, by, bz): K slice by, 64-column bands bx*nb .. bx*nb + nb - 1,
// rows bz*16*MT .. (a row block; more than 64 rows run as several blocks, so
// that twice the workgroups share the weights through L2 instead of one
// workgroup staging 128 rows).  The X slice is staged once; wave w computes
// columns band*64 + w*16 + 0..15 of each band while the next band's weights
// are already in flight.
template <int MT, int KS>
__global__ void __launch_bounds__(kGemmThreads) __attribute__((amdgpu_waves_per_eu(KS > 512 ? 1 : 2, 2)))
gemm_kernel(const uint16_t *__restrict__ x, int64_t x_s0, int M, const uint16_t *__restrict__ w,
            int64_t w_s0, int N, int nb, uint16_t *__restrict__ out, int64_t o_s0,
            float *__restrict__ part, const uint16_t *__restrict__ bias) {
    constexpr int kSteps = KS / 32;
    constexpr int kRows = 16 * MT;
    __shared__ __attribute__((aligned(16))) uint16_t xs[kRows * x_pitch<KS>()];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15;
    const int kq = lane >> 4;  // which 8-wide k group of the 32-k step
    const int band0 = blockIdx.x * nb;
    const int k0 = blockIdx.y * KS;
    const int row0 = blockIdx.z * kRows;
    const int mr = M - row0 < kRows ? M - row0 : kRows;  // rows of this block
    x += static_cast<int64_t>(row0) * x_s0;

    // 1. X[:, k0 : k0 + KS] into registers (rows >= M are zero): issued first,
    // so that waiting for them does not wait for the weights
    constexpr int kVecPerRow = KS / 8;
    constexpr int kXVec = kRows * kVecPerRow / kGemmThreads;
    static_assert(kRows * kVecPerRow % kGemmThreads == 0, "X block splits evenly over the threads");
    // The workgroups of one K slice all read this block: each starts at its own
    // rotation of it, so that they do not ask the same L2 lines at once.
    constexpr int kXTotal = kRows * kVecPerRow;
    const int rot = static_cast<int>((blockIdx.x * 66u) % kXTotal);
    auto rot_of = [&](int i) { return i + rot < kXTotal ? i + rot : i + rot - kXTotal; };
    uint4 xr[kXVec];
#pragma unroll
    for (int q = 0; q < kXVec; ++q) {
        const int v = rot_of(threadIdx.x + q * kGemmThreads);
        const int row = v / kVecPerRow, col = v % kVecPerRow;
        // unconditional load (rows past the block read its row 0, mr >= 1) so that
        // no branch splits the prologue: the weight loads below must stay ahead of
        // the barrier, and the compiler only keeps them there in straight-line code
        const uint4 t = *reinterpret_cast<const uint4 *>(x + (row < mr ? row : 0) * x_s0 + k0 + col * 8);
        xr[q] = row < mr ? t : make_uint4(0, 0, 0, 0);
    }

    // 2. the first band's weights, all in flight together
    uint4 wa[kSteps], wb[kSteps];
    gemm_load_w<KS>(wa, w, w_s0, band0 * 64 + wave * 16 + r16, k0, kq);
    // keep every weight load ahead of the wait for the X block
    __builtin_amdgcn_sched_barrier(0);

#pragma unroll
    for (int q = 0; q < kXVec; ++q) {
        const int v = rot_of(threadIdx.x + q * kGemmThreads);
        const int row = v / kVecPerRow, col = v % kVecPerRow;
        *reinterpret_cast<uint4 *>(xs + row * x_pitch<KS>() + col * 8) = xr[q];
    }
    __syncthreads();

    // 3. bands in pairs: the loads of one buffer fly while the other is used.
    // The body runs at least once (nb >= 1): with a loop that might run zero
    // times the compiler sinks the first band's loads into the loop guard,
    // after the barrier, and the weight stream then waits for the X block.
    for (int b = 0;; b += 2) {
        const int col_a = (band0 + b) * 64 + wave * 16;
        if (b + 1 < nb) gemm_load_w<KS>(wb, w, w_s0, col_a + 64 + r16, k0, kq);
        gemm_tile<MT, KS>(wa, xs, r16, kq, M, row0, mr, N, col_a, blockIdx.y, out, o_s0, part, bias);
        if (b + 1 >= nb) break;
        if (b + 2 < nb) gemm_load_w<KS>(wa, w, w_s0, col_a + 128 + r16, k0, kq);
        gemm_tile<MT, KS>(wb, xs, r16, kq, M, row0, mr, N, col_a + 64, blockIdx.y, out, o_s0, part, bias);
        if (b + 2 >= nb) break;
    }
}

// Y = bf16(sum over slices of part), eight columns per thread, slices added
// in index order (the same order the fused epilogues use).
__global__ void __launch_bounds__(kGemmThreads)
gemm_reduce_kernel(const float *__restrict__ part, int S, int M, int N, uint16_t *__restrict__ out,
                   int64_t o_s0, const uint16_t *__restrict__ bias) {
    const int64_t total = static_cast<int64_t>(M) * N / 8;
    const int64_t plane = static_cast<int64_t>(M) * N;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kGemmThreads) + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * kGemmThreads) {
        float v[8];
        sum_partials8(part + i * 8, S, plane, v);
        const int64_t e = i * 8;
        const int row = static_cast<int>(e / N), col = static_cast<int>(e % N);
        if (bias) {
            float bv[8];
            unpack8(*reinterpret_cast<const uint4 *>(bias + col), bv);
#pragma unroll
            for (int k = 0; k < 8; ++k) v[k] += bv[k];
        }
        uint4 o;
        o.x = pack2_bf16(v[0], v[1]);
        o.y = pack2_bf16(v[2], v[3]);
        o.z = pack2_bf16(v[4], v[5]);
        o.w = pack2_bf16(v[6], v[7]);
        *reinterpret_cast<uint4 *>(out + row * o_s0 + col) = o;
    }
}

// More than 64 rows: 768-column K slices (a third of the planes) where K allows
// them and the grid still has a workgroup for every CU, else the 256-column
// slices of a 128-row block (whose sums the fused bf16 gate/up + SwiGLU kernel
// reproduces), in row blocks of 64, else of 32 (32-row blocks of 256-column
// slices when neither fills the CUs).
struct RowsPlan {
    int ks, rows;
};
RowsPlan rows_plan(int M, int N, int K) {
    const int bands = N / 64;
    for (const int ks : {768, 256}) {
        if (K % ks) continue;
        for (const int rb : {64, 32})
            if (static_cast<int64_t>(bands) * (K / ks) * ((M + rb - 1) / rb) >= 256) return {ks, rb};
    }
    return {256, 32};
}

// K slice per workgroup (rows_plan above 64 rows).  Every slice is one fp32
// partial plane.
int slice_of(int M, int N, int K) {
    // 512 K columns per workgroup for up to 64 rows; a projection
    // whose grid would still fit one workgroup per CU with 256-column slices
    // (bands x slices <= 256) takes those, so that every CU streams weights.
    // 768-column slices where they make the grid whole multiples of 256
    // workgroups: with 512 the 2048 x 6144 `down` projection launches 384
    // workgroups, so half the CUs stream twice the weights of the others
    // (measured 10.8 us against 10.2 us for 256 even workgroups, which also
    // leave 8 partial planes instead of 12).
    if (M > 64) return rows_plan(M, N, K).ks;
    if (N % 64 != 0) return 512;
    const int bands = N / 64;
    if (K % 256 == 0 && bands * (K / 256) <= 256) return 256;
    if (K % 768 == 0 && (bands * (K / 768)) % 256 == 0) return 768;
    return 512;
}


template <int MT, int KS>
void launch_gemm(const uint16_t *x, int64_t x_s0, int M, const uint16_t *w, int64_t w_s0, int N, int K,
                 uint16_t *out, int64_t o_s0, float *part, const uint16_t *bias, hipStream_t st) {
    const int bands = N / 64, S = K / KS;
    const int blocks = (M + 16 * MT - 1) / (16 * MT);  // row blocks
    const int nb = bands_per_wg(bands, S * blocks);
    dim3 grid(bands / nb, S, blocks);
    hipLaunchKernelGGL((gemm_kernel<MT, KS>), grid, dim3(kGemmThreads), 0, st, x, x_s0, M, w, w_s0, N, nb, out,
                       o_s0, part, bias);
}

// The launch for M rows with the K slice slice_of picks.
void dispatch_gemm(const uint16_t *x, int64_t x_s0, int M, const uint16_t *w, int64_t w_s0, int N, int K,
                   uint16_t *out, int64_t o_s0, float *part, const uint16_t *bias, hipStream_t st) {
    const int ks = slice_of(M, N, K);
    // more than 64 rows run as the row blocks rows_plan picks (the code predictor's 128-row o
    // projection: 32-row blocks, 256 workgroups instead of 64 for one 128-row block)
    int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
    if (M > 64 && N % 64 == 0) mt = rows_plan(M, N, K).rows / 16;
#define NQ_GEMM_SLICES(MT)                                                                   \
    ks == 256   ? launch_gemm<MT, 256>(x, x_s0, M, w, w_s0, N, K, out, o_s0, part, bias, st) \
    : ks == 768 ? launch_gemm<MT, 768>(x, x_s0, M, w, w_s0, N, K, out, o_s0, part, bias, st) \
                : launch_gemm<MT, 512>(x, x_s0, M, w, w_s0, N, K, out, o_s0, part, bias, st)
    switch (mt) {
        case 1: NQ_GEMM_SLICES(1); break;
        case 2: NQ_GEMM_SLICES(2); break;
        default: NQ_GEMM_SLICES(4); break;
    }
#undef NQ_GEMM_SLICES
}

// ---------------------------------------------------------------------------
// Gate/up with the SwiGLU fused, bf16, for rows in blocks of 64 and K = 1024
// (the code predictor's MLP).  The activation block [64, K] is 128 KiB, so one
// workgroup per CU stages all of it in LDS and computes whole dot products:
// no split-K planes and no second kernel.  The weight rows are interleaved
// (nq_fp8_pack_swiglu on the bf16 rows): 16-row tile t holds, for q = 0..3,
// gate rows 8t + 2q, 8t + 2q + 1 then up rows 8t + 2q, 8t + 2q + 1, so MFMA
// lane group q ends with two gate/up pairs of the same act columns
// 8t + 2q + {0, 1}.  A workgroup owns kBsTiles tiles of one 64-row block; its
// kBsTiles * kBsQuarters waves each take one tile over one quarter of K, the
// chain of each quarter runs in k order from zero (the MFMA operands and
// order of a K slice of the split-K kernel), the quarters are summed in
// order through LDS, and the epilogue rounds gate and up to bf16 and stores
// bf16(silu(g) * u) -- the bits of the split-K projection with four 256-wide
// slices (its choice at 128 rows) followed by the SiLU-mul kernel.

constexpr int kBsTiles = 3;
constexpr int kBsQuarters = 4;
constexpr int kBsThreads = kBsTiles * kBsQuarters * kWave;
constexpr int kBsRows = 64;
constexpr int kBsK = 1024;
static_assert(kBsRows / 16 == kBsQuarters, "the wave of quarter q finishes 16-row block q");

template <int K>
__global__ void __launch_bounds__(kBsThreads)
bf16_swiglu_kernel(const uint16_t *__restrict__ x, int64_t x_s0, int M, const uint16_t *__restrict__ w,
                   int64_t w_s0, uint16_t *__restrict__ out, int64_t o_s0) {
    constexpr int XP = x_pitch<K>();   // LDS row pitch (bf16)
    constexpr int QK = K / kBsQuarters;
    constexpr int QS = QK / 32;         // MFMA steps per quarter
    __shared__ __attribute__((aligned(16))) uint16_t xs[kBsRows * XP];
    static_assert(kBsQuarters * kBsTiles * 4 * kWave * 4 * 4 <= kBsRows * XP * 2, "reduction fits the X area");

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const int tl = wave % kBsTiles;
    const int quarter = wave / kBsTiles;
    const int tile = blockIdx.x * kBsTiles + tl;
    const int row0 = blockIdx.y * kBsRows;
    const int rows = M - row0 < kBsRows ? M - row0 : kBsRows;

    // 1. the activation block (rows past M zero), issued first: loads complete in
    // issue order, so the wait for them below leaves the weights in flight.  Each
    // workgroup starts at its own rotation of the block, so the CUs of an XCD do
    // not all ask the same L2 lines at the same moment.
    constexpr int kVec = kBsRows * (K / 8);
    constexpr int kPer = (kVec + kBsThreads - 1) / kBsThreads;
    const int rot = (blockIdx.x * 258) % kVec;
    auto rot_of = [&](int i) { return i + rot < kVec ? i + rot : i + rot - kVec; };
    uint4 xr[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = threadIdx.x + u * kBsThreads;
        const int v = rot_of(i);
        const int row = v / (K / 8), c = v % (K / 8);
        xr[u] = (i < kVec && row < rows) ? *reinterpret_cast<const uint4 *>(x + (row0 + row) * x_s0 + c * 8)
                                         : make_uint4(0, 0, 0, 0);
    }
    // 2. the wave's weights: 16 packed rows over its K quarter
    uint4 wr[QS];
    {
        const uint16_t *wrow = w + static_cast<int64_t>(tile * 16 + r16) * w_s0 + quarter * QK + kq * 8;
#pragma unroll
        for (int j = 0; j < QS; ++j) wr[j] = *reinterpret_cast<const uint4 *>(wrow + j * 32);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = threadIdx.x + u * kBsThreads;
        const int v = rot_of(i);
        if (i < kVec) *reinterpret_cast<uint4 *>(xs + (v / (K / 8)) * XP + (v % (K / 8)) * 8) = xr[u];
    }
    __syncthreads();

    // 3. the quarter's MFMA chains (W as the A operand, X^T from LDS as the B operand)
    floatx4_t acc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < QS; ++j) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const uint4 b = *reinterpret_cast<const uint4 *>(xs + (m * 16 + r16) * XP + quarter * QK + j * 32 + kq * 8);
            acc[m] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(wr[j]), as_bf16x8(b), acc[m], 0, 0, 0);
        }
    }

    // 4. every quarter wave hands its sums over through the (now free) X area; the
    // wave of quarter q then finishes 16-row block m = q of its tile, adding the
    // quarters in order 0, 1, 2, 3
    __syncthreads();
    float *red = reinterpret_cast<float *>(xs);
    {
        float *dst = red + ((quarter * kBsTiles + tl) * 4 * kWave + lane) * 4;
#pragma unroll
        for (int m = 0; m < 4; ++m)
            *reinterpret_cast<float4 *>(dst + m * kWave * 4) = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
    }
    __syncthreads();
    const int m = quarter;
    float sum[4];
    {
        const float4 v0 = *reinterpret_cast<const float4 *>(red + ((tl * 4 + m) * kWave + lane) * 4);
        sum[0] = v0.x;
        sum[1] = v0.y;
        sum[2] = v0.z;
        sum[3] = v0.w;
    }
#pragma unroll
    for (int q = 1; q < kBsQuarters; ++q) {
        const float4 v = *reinterpret_cast<const float4 *>(red + (((q * kBsTiles + tl) * 4 + m) * kWave + lane) * 4);
        sum[0] += v.x;
        sum[1] += v.y;
        sum[2] += v.z;
        sum[3] += v.w;
    }
    // 5. SwiGLU of the bf16 projection values: act columns 8t + 2kq + {0, 1}
    const int row = m * 16 + r16;
    if (row >= rows) return;
    float a[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
        const float g = bf16_to_f32(f32_to_bf16(sum[e]));
        const float u = bf16_to_f32(f32_to_bf16(sum[2 + e]));
        a[e] = g / (1.0f + expf(-g)) * u;
    }
    *reinterpret_cast<uint32_t *>(out + (row0 + row) * o_s0 + tile * 8 + kq * 2) = pack2_bf16(a[0], a[1]);
}

}  // namespace

// Bands per workgroup: the largest divisor of the band count that still
// leaves at least one workgroup per CU; more bands per workgroup share one
// staged X slice.
int bands_per_wg(int bands, int splits) {
    constexpr int kTargetWgs = 256;
    int best = 1;
    for (int nb = 2; nb <= 8; ++nb)
        if (bands % nb == 0 && (bands / nb) * splits >= kTargetWgs) best = nb;
    return best;
}

int launch_reduce_partials(const float *part, int S, int M, int N, uint16_t *out, int64_t o_s0,
                           const uint16_t *bias, hipStream_t st) {
    const int64_t vec = static_cast<int64_t>(M) * N / 8;
    int blocks = static_cast<int>((vec + kGemmThreads - 1) / kGemmThreads);
    hipLaunchKernelGGL(gemm_reduce_kernel, dim3(blocks > 2048 ? 2048 : blocks), dim3(kGemmThreads), 0, st, part, S,
                       M, N, out, o_s0, bias);
    return NQ_LAUNCH_STATUS();
}

}  // namespace nq

using namespace nq;

extern "C" int nq_linear_splits(int M, int N, int K) {
    if (M <= 0 || M > 128 || N <= 0 || N % 64 != 0 || K <= 0 || K % slice_of(M, N, K) != 0) return -1;
    return K / slice_of(M, N, K);
}

extern "C" int64_t nq_linear_workspace_bytes(int M, int N, int K, int epilogue) {
    const int S = nq_linear_splits(M, N, K);
    if (S < 0 || epilogue < NQ_EPI_NONE || epilogue > NQ_EPI_PARTIALS) return -1;
    if (S == 1 && epilogue == NQ_EPI_NONE) return 0;
    return static_cast<int64_t>(S) * M * N * 4;
}

extern "C" int nq_linear(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M, int N, int K,
                         int epilogue, const uint16_t *bias, uint16_t *out, int64_t o_s0,
                         uint16_t *residual, const uint16_t *norm_weight, float eps, void *workspace,
                         int64_t workspace_bytes, void *stream) {
    NQ_CHECK_ARG(x && w && M > 0 && N > 0 && K > 0);
    NQ_CHECK_ARG(epilogue >= NQ_EPI_NONE && epilogue <= NQ_EPI_PARTIALS);
    const int S = nq_linear_splits(M, N, K);
    if (S < 0) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && x_s0 % 8 == 0 && w_s0 >= K && w_s0 % 8 == 0);
    NQ_CHECK_ARG((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 == 0);
    const int out_width = epilogue == NQ_EPI_SILU_MUL ? N / 2 : N;
    if (epilogue != NQ_EPI_PARTIALS) {
        NQ_CHECK_ARG(out && o_s0 >= out_width && o_s0 % 8 == 0 && reinterpret_cast<uintptr_t>(out) % 16 == 0);
    }
    if (epilogue == NQ_EPI_ADD_RMSNORM) {
        NQ_CHECK_ARG(residual && norm_weight);
        NQ_CHECK_ARG((reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(norm_weight)) % 16 == 0);
        if (N > 8192) return NQ_ERR_UNSUPPORTED;
    }
    if (epilogue == NQ_EPI_SILU_MUL) NQ_CHECK_ARG(N % 16 == 0);
    NQ_CHECK_ARG(!bias || (epilogue == NQ_EPI_NONE && reinterpret_cast<uintptr_t>(bias) % 16 == 0));
    const int64_t need = nq_linear_workspace_bytes(M, N, K, epilogue);
    NQ_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need &&
                               reinterpret_cast<uintptr_t>(workspace) % 16 == 0));
    float *part = need ? static_cast<float *>(workspace) : nullptr;
    hipStream_t st = static_cast<hipStream_t>(stream);
    dispatch_gemm(x, x_s0, M, w, w_s0, N, K, out, o_s0, part, bias, st);
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    switch (epilogue) {
        case NQ_EPI_NONE:
            return S > 1 ? launch_reduce_partials(part, S, M, N, out, o_s0, bias, st) : NQ_LAUNCH_STATUS();
        case NQ_EPI_ADD_RMSNORM:
            return launch_add_rmsnorm_partials(part, S, M, N, out, o_s0, residual, norm_weight, eps, st);
        case NQ_EPI_SILU_MUL:
            return launch_silu_mul_partials(part, S, M, N / 2, out, o_s0, st);
        default:
            return NQ_OK;  // partials stay in the workspace for the caller's consumer
    }
}

extern "C" int nq_linear_add_rmsnorm_fp8(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M,
                                         int N, int K, uint16_t *residual, const uint16_t *norm_weight, float eps,
                                         uint8_t *xq, int64_t xq_s0, float *sx, int64_t sx_s0, void *workspace,
                                         int64_t workspace_bytes, void *stream) {
    NQ_CHECK_ARG(x && w && residual && norm_weight && xq && sx && M > 0 && N > 0 && K > 0);
    const int S = nq_linear_splits(M, N, K);
    if (S < 0 || N % 128 != 0 || N > 8192) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && x_s0 % 8 == 0 && w_s0 >= K && w_s0 % 8 == 0);
    NQ_CHECK_ARG((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 == 0);
    NQ_CHECK_ARG((reinterpret_cast<uintptr_t>(residual) | reinterpret_cast<uintptr_t>(norm_weight)) % 16 == 0);
    NQ_CHECK_ARG(xq_s0 >= N && xq_s0 % 8 == 0 && reinterpret_cast<uintptr_t>(xq) % 8 == 0 && sx_s0 >= N / 128);
    const int64_t need = nq_linear_workspace_bytes(M, N, K, NQ_EPI_ADD_RMSNORM);
    NQ_CHECK_ARG(workspace && workspace_bytes >= need && reinterpret_cast<uintptr_t>(workspace) % 16 == 0);
    float *part = static_cast<float *>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
    dispatch_gemm(x, x_s0, M, w, w_s0, N, K, nullptr, 0, part, nullptr, st);
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    return launch_add_rmsnorm_partials_fp8(part, S, M, N, residual, norm_weight, eps, xq, xq_s0, sx, sx_s0, st);
}

extern "C" int nq_linear_swiglu(const uint16_t *x, int64_t x_s0, int M, const uint16_t *packed, int64_t w_s0, int I,
                                int K, uint16_t *out, int64_t o_s0, void *stream) {
    NQ_CHECK_ARG(x && packed && out && M > 0 && I > 0 && K > 0);
    if (K != nq::kBsK || I % (8 * nq::kBsTiles) != 0) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K && x_s0 % 8 == 0 && w_s0 % 8 == 0);
    NQ_CHECK_ARG((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(packed)) % 16 == 0);
    NQ_CHECK_ARG(o_s0 >= I && o_s0 % 2 == 0 && reinterpret_cast<uintptr_t>(out) % 4 == 0);
    const dim3 grid(static_cast<unsigned>(2 * I / (16 * nq::kBsTiles)),
                    static_cast<unsigned>((M + nq::kBsRows - 1) / nq::kBsRows));
    hipLaunchKernelGGL((nq::bf16_swiglu_kernel<nq::kBsK>), grid, dim3(nq::kBsThreads), 0,
                       static_cast<hipStream_t>(stream), x, x_s0, M, packed, w_s0, out, o_s0);
    return NQ_LAUNCH_STATUS();
}
