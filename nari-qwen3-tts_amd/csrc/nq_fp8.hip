// FP8 (OCP e4m3fn) gate/up projection of the talker decode step.
//
// Weights: the 128 x 128 block quantization of model/layers.py:10-25 -- per
// block, max |w| clamped to >= 1e-4, a power-of-two scale 2^ceil(log2(max /
// 448)) and e4m3fn codes of w / scale rounded to nearest even.
//
// GEMM: the block-scaled FP8 product that model/layers.py:241-262 runs through
// flashinfer's fp8_blockscale_gemm_sm90 (the DeepGEMM fine-grained scheme):
// activations quantized per row and 128 columns (scale = max |x| / 448, codes
// of x / scale), fp32 accumulation with both scales applied per 128-wide K
// block, y[m, n] = sum_kb sx[m, kb] sw[n / 128, kb] (qx[m, kb] . qw[n, kb]).
//
// The GEMM keeps the bf16 skinny GEMM's plan -- each weight byte read from
// HBM once with one-shot 128-bit loads, the X slice staged in LDS, split-K
// fp32 partial planes summed in plane order by the consumer -- and runs the
// gfx950 MFMA v_mfma_scale_f32_16x16x128_f8f6f4 (formats e4m3 x e4m3, unit
// E8M0 scales): one instruction covers exactly one 128-wide K block of a
// 16-column tile, so the block's scale product is applied once to each
// instruction result.  An FP8 weight row slice of 1024 bytes carries the same
// 64 KiB per workgroup in flight as the bf16 GEMM's 512-element slice, with
// half the K splits.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {

namespace {

constexpr int kFp8Threads = 256;
constexpr int kFp8Waves = kFp8Threads / kWave;

// Smallest power of two >= v for a positive normal v.
__device__ __forceinline__ float pow2_ceil(float v) {
    const uint32_t u = __float_as_uint(v);
    return (u & 0x7fffffu) == 0 ? v : __uint_as_float((u & 0x7f800000u) + 0x00800000u);
}

// One workgroup per 128 x 128 block: thread t holds rows t/16 + 16 i (i < 8),
// columns (t % 16) * 8 .. + 7 of the block.
__global__ void __launch_bounds__(kFp8Threads)
quantize_blocks_kernel(const uint16_t *__restrict__ w, int64_t w_s0, uint8_t *__restrict__ q, int64_t q_s0,
                       float *__restrict__ scales, int64_t s_s0) {
    __shared__ float wmax[kFp8Waves];
    const int64_t r0 = static_cast<int64_t>(blockIdx.y) * 128 + threadIdx.x / 16;
    const int c0 = blockIdx.x * 128 + (threadIdx.x & 15) * 8;
    float v[8][8];
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        unpack8(*reinterpret_cast<const uint4 *>(w + (r0 + 16 * i) * w_s0 + c0), v[i]);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[i][e]));
    }
    amax = group_max<kWave>(amax);
    if ((threadIdx.x & (kWave - 1)) == 0) wmax[threadIdx.x / kWave] = amax;
    __syncthreads();
#pragma unroll
    for (int k = 0; k < kFp8Waves; ++k) amax = fmaxf(amax, wmax[k]);
    const float s = pow2_ceil(fmaxf(amax, 1e-4f) / 448.0f);
#pragma unroll
    for (int i = 0; i < 8; ++i) *reinterpret_cast<uint2 *>(q + (r0 + 16 * i) * q_s0 + c0) = e4m3_pack8(v[i], s);
    if (threadIdx.x == 0) scales[blockIdx.y * s_s0 + blockIdx.x] = s;
}

// Thread per 8 columns; the 16 threads of a 128-column group share its scale.
__global__ void __launch_bounds__(kFp8Threads)
quantize_rows_kernel(const uint16_t *__restrict__ x, int64_t x_s0, int M, int K, uint8_t *__restrict__ q,
                     int64_t q_s0, float *__restrict__ scales, int64_t s_s0) {
    const int vecs = K / 8;
    const int64_t total = static_cast<int64_t>(M) * vecs;
    // whole 16-thread groups stay together: total and the stride are multiples of 16
    for (int64_t i = static_cast<int64_t>(blockIdx.x) * kFp8Threads + threadIdx.x; i < total;
         i += static_cast<int64_t>(gridDim.x) * kFp8Threads) {
        const int64_t row = i / vecs;
        const int col = static_cast<int>(i - row * vecs) * 8;
        float v[8];
        unpack8(*reinterpret_cast<const uint4 *>(x + row * x_s0 + col), v);
        float amax = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(v[e]));
        const float s = row_group_scale(group_max<16>(amax));
        *reinterpret_cast<uint2 *>(q + row * q_s0 + col) = e4m3_pack8(v, s);
        if ((col & 127) == 0) scales[row * s_s0 + col / 128] = s;
    }
}

typedef int int8v_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));

// LDS layout of a staged FP8 X slice of R rows x KS bytes.  A lane group takes
// 32 bytes per 128-wide K block (bytes kq*32 .. +31), read as two 16-byte
// halves; the halves live in two planes [half][row][64 bytes per K block] with
// a row pitch of KS/2 + 32 bytes, so each ds_read_b128 reads 16-byte chunks at
// a 32-byte row offset -- the conflict-free pattern on gfx950 (the unsplit
// layout's 32-byte chunks conflict at every padding tried).
template <int R, int KS>
struct Fp8Lds {
    static constexpr int kPitch = KS / 2 + 32;
    static constexpr int kBytes = 2 * R * kPitch;
    // LDS offset of the 16-byte vector c (bytes 16c .. 16c + 15) of staged row `row`
    __device__ static __forceinline__ int stage_offset(int row, int c) {
        const int kb = c >> 3, w = c & 7;
        return (w & 1) * (R * kPitch) + row * kPitch + kb * 64 + (w >> 1) * 16;
    }
    // the 32 bytes of K block j for lane group kq of staged row `row`
    __device__ static __forceinline__ int8v_t read(const uint8_t *xs, int row, int j, int kq) {
        const uint8_t *p = xs + row * kPitch + j * 64 + kq * 16;
        const uint4 lo = *reinterpret_cast<const uint4 *>(p);
        const uint4 hi = *reinterpret_cast<const uint4 *>(p + R * kPitch);
        int8v_t r;
        r[0] = static_cast<int>(lo.x);
        r[1] = static_cast<int>(lo.y);
        r[2] = static_cast<int>(lo.z);
        r[3] = static_cast<int>(lo.w);
        r[4] = static_cast<int>(hi.x);
        r[5] = static_cast<int>(hi.y);
        r[6] = static_cast<int>(hi.z);
        r[7] = static_cast<int>(hi.w);
        return r;
    }
};

// Lane (r16, kq) of a wave holds, for every 128-wide K block j of the slice,
// bytes j*128 + kq*32 .. +31 of weight row n_row: the same K positions the
// B operand takes from the staged X rows, so each MFMA sums matching products.
template <int KS>
__device__ __forceinline__ void fp8_load_w(int8v_t (&wr)[KS / 128], const uint8_t *__restrict__ w, int64_t w_s0,
                                           int n_row, int k0, int kq) {
    const uint8_t *row = w + static_cast<int64_t>(n_row) * w_s0 + k0 + kq * 32;
#pragma unroll
    for (int j = 0; j < KS / 128; ++j) wr[j] = *reinterpret_cast<const int8v_t *>(row + j * 128);
}

// One 16-column tile over the slice: per K block an MFMA from zero, scaled by
// sx[row, kb] * sw[col / 128, kb] into the fp32 sum; then the store (the lane
// holds Y[m*16 + r16][col + kq*4 + 0..3]).
template <int MT, int KS>
__device__ __forceinline__ void fp8_tile(const int8v_t (&wr)[KS / 128], const uint8_t *xs, const float *sxs,
                                         const float (&swv)[KS / 128], int r16, int kq, int M, int N, int col,
                                         int slice, uint16_t *__restrict__ out, int64_t o_s0, float *__restrict__ part) {
    constexpr int kSteps = KS / 128;
    floatx4_t acc[MT];
#pragma unroll
    for (int m = 0; m < MT; ++m) acc[m] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < kSteps; ++j) {
        const float swj = swv[j];
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const int8v_t b = Fp8Lds<16 * MT, KS>::read(xs, m * 16 + r16, j, kq);
            const floatx4_t t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                wr[j], b, floatx4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
            const float s = sxs[j * (16 * MT) + m * 16 + r16] * swj;
#pragma unroll
            for (int e = 0; e < 4; ++e) acc[m][e] = fmaf(t[e], s, acc[m][e]);
        }
        // one K block's B operands (8 VGPRs per row tile) live at a time: the
        // instruction selector may otherwise sink every MFMA (they start from zero
        // and touch no memory) below all LDS reads, so each block's sums are pinned
        // here before the next block's reads
#pragma unroll
        for (int m = 0; m < MT; ++m) asm volatile("" : "+v"(acc[m]));
        __builtin_amdgcn_sched_barrier(0);
    }
    col += kq * 4;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int row = m * 16 + r16;
        if (row >= M) continue;
        if (part) {
            float *p = part + (static_cast<int64_t>(slice) * M + row) * N + col;
            *reinterpret_cast<float4 *>(p) = make_float4(acc[m][0], acc[m][1], acc[m][2], acc[m][3]);
        } else {
            uint2 o;
            o.x = pack2_bf16(acc[m][0], acc[m][1]);
            o.y = pack2_bf16(acc[m][2], acc[m][3]);
            *reinterpret_cast<uint2 *>(out + row * o_s0 + col) = o;
        }
    }
}

// Workgroup (bx, by): K slice by of KS bytes, 64-column band bx (wave w owns
// columns bx*64 + w*16 .. + 15).  One band per workgroup: at KS = 1024 the
// band's weights already fill 64 VGPRs per lane, and the talker's gate/up
// shape gives 384 workgroups.
template <int MT, int KS>
__global__ void __launch_bounds__(kFp8Threads) __attribute__((amdgpu_waves_per_eu(2, 2)))
gemm_fp8_kernel(const uint8_t *__restrict__ x, int64_t x_s0, const float *__restrict__ sx, int64_t sx_s0, int M,
                const uint8_t *__restrict__ w, int64_t w_s0, const float *__restrict__ sw, int64_t sw_s0, int N,
                uint16_t *__restrict__ out, int64_t o_s0, float *__restrict__ part) {
    constexpr int kSteps = KS / 128;
    constexpr int kRows = 16 * MT;
    __shared__ __attribute__((aligned(16))) uint8_t xs[Fp8Lds<kRows, KS>::kBytes];
    __shared__ float sxs[kSteps * kRows];  // activation scales [K block][row] (a wave's rows on distinct banks)

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const int col = blockIdx.x * 64 + wave * 16;
    const int k0 = blockIdx.y * KS;
    const int kb0 = k0 / 128;

    // 1. the band's weight scales (one per K block, wave-uniform), the X slice
    // (rows >= M are zero) and the activation scales
    float swv[kSteps];
    const float *sw_row = sw + (col / 128) * sw_s0 + kb0;
#pragma unroll
    for (int j = 0; j < kSteps; ++j) swv[j] = sw_row[j];
    constexpr int kVecPerRow = KS / 16;
    constexpr int kXVec = kRows * kVecPerRow / kFp8Threads;
    static_assert(kRows * kVecPerRow % kFp8Threads == 0, "X block splits evenly over the threads");
    uint4 xr[kXVec];
#pragma unroll
    for (int q = 0; q < kXVec; ++q) {
        const int i = threadIdx.x + q * kFp8Threads;
        const int row = i / kVecPerRow, c = i % kVecPerRow;
        xr[q] = row < M ? *reinterpret_cast<const uint4 *>(x + row * x_s0 + k0 + c * 16) : make_uint4(0, 0, 0, 0);
    }
    for (int i = threadIdx.x; i < kRows * kSteps; i += kFp8Threads) {
        const int row = i / kSteps, j = i % kSteps;
        sxs[j * kRows + row] = row < M ? sx[row * sx_s0 + kb0 + j] : 0.f;
    }

    // 2. the band's weights, all in flight together
    int8v_t wa[kSteps];
    fp8_load_w<KS>(wa, w, w_s0, col + r16, k0, kq);
    __builtin_amdgcn_sched_barrier(0);

    // one LDS plane per store (adjacent vectors belong to the two planes, whose starts share banks)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
#pragma unroll
        for (int q = 0; q < kXVec; ++q) {
            const int i = threadIdx.x + q * kFp8Threads;
            const int row = i / kVecPerRow, c = i % kVecPerRow;
            if ((c & 1) == h) *reinterpret_cast<uint4 *>(xs + Fp8Lds<kRows, KS>::stage_offset(row, c)) = xr[q];
        }
    }
    __syncthreads();

    fp8_tile<MT, KS>(wa, xs, sxs, swv, r16, kq, M, N, col, blockIdx.y, out, o_s0, part);
}

// ---------------------------------------------------------------------------
// Gate/up with the SwiGLU fused, for <= 64 rows and K = 2048 (the talker's
// MLP).  The FP8 activation block [64, K] is 128 KiB, so one workgroup per CU
// stages all of it in LDS and computes whole dot products: no split-K planes
// and no second kernel.  The gate/up weight rows are held interleaved
// (nq_fp8_pack_swiglu): 16-row tile t holds, for q = 0..3, gate rows
// 8t + 2q, 8t + 2q + 1 then up rows 8t + 2q, 8t + 2q + 1, so MFMA lane group q
// ends with two gate/up pairs of the same act columns 8t + 2q + {0, 1}.  The
// workgroup owns kSwTiles tiles; its kSwTiles * kSwQuarters waves each take
// one tile over one quarter of K (twelve waves keep three per SIMD to hide
// the load and MFMA latencies), and the quarters are summed in order through
// LDS before the epilogue rounds gate and up to bf16 and stores
// bf16(silu(g) * u).

constexpr int kSwTiles = 3;
constexpr int kSwQuarters = 4;
constexpr int kSwThreads = kSwTiles * kSwQuarters * kWave;
constexpr int kSwK = 2048;
constexpr int kSwRows = 64;
static_assert(kSwRows / 16 == kSwQuarters, "the wave of quarter q finishes 16-row tile q");

template <int K>
__global__ void __launch_bounds__(kSwThreads)
fp8_swiglu_kernel(const uint8_t *__restrict__ x, int64_t x_s0, const float *__restrict__ sx, int64_t sx_s0, int M,
                  const uint8_t *__restrict__ w, int64_t w_s0, const float *__restrict__ sw, int64_t sw_s0, int I,
                  uint16_t *__restrict__ out, int64_t o_s0) {
    constexpr int KB = K / 128;                    // K blocks
    constexpr int QS = K / kSwQuarters / 128;      // K blocks per quarter
    using Lds = Fp8Lds<kSwRows, K>;
    __shared__ __attribute__((aligned(16))) uint8_t xs[Lds::kBytes];
    __shared__ float sxs[KB * kSwRows];  // [K block][row]: a wave's 16 rows hit 16 banks
    static_assert(kSwQuarters * kSwTiles * kWave * 16 * 4 <= Lds::kBytes, "reduction fits the X area");

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15;
    const int kq = lane >> 4;
    const int tl = wave % kSwTiles;
    const int quarter = wave / kSwTiles;
    const int tile = blockIdx.x * kSwTiles + tl;
    const int kb0 = quarter * QS;

    // 1. the activation block and its scales (rows >= M zero), issued first:
    // loads complete in issue order, so the wait for them below leaves the
    // weights in flight and the X block reaches LDS long before the weights
    constexpr int kVec = kSwRows * (K / 16);
    constexpr int kPer = (kVec + kSwThreads - 1) / kSwThreads;
    constexpr int kSx = kSwRows * KB;
    constexpr int kSxPer = (kSx + kSwThreads - 1) / kSwThreads;
    // Every workgroup reads the same block: each starts at its own (even)
    // rotation of it, so the CUs of an XCD do not all ask the same L2 lines
    // at the same moment.  Vector i of the thread is block vector rot(i).
    const int rot = (blockIdx.x * 258) % kVec;
    auto rot_of = [&](int i) { return i + rot < kVec ? i + rot : i + rot - kVec; };
    uint4 xr[kPer];
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
        const int i = threadIdx.x + u * kSwThreads;
        const int v = rot_of(i);
        const int row = v / (K / 16), c = v % (K / 16);
        xr[u] = (i < kVec && row < M) ? *reinterpret_cast<const uint4 *>(x + row * x_s0 + c * 16)
                                      : make_uint4(0, 0, 0, 0);
    }
    float sr[kSxPer];
#pragma unroll
    for (int u = 0; u < kSxPer; ++u) {
        const int i = threadIdx.x + u * kSwThreads;
        // element i of the [K block][row] table
        sr[u] = (i < kSx && i % kSwRows < M) ? sx[(i % kSwRows) * sx_s0 + i / kSwRows] : 0.f;
    }
    // 2. the wave's weights (16 packed rows over its K quarter) and scales:
    // gate rows 8t.. lie in 128-row block t / 16, up rows in (I + 8t) / 128
    int8v_t wr[QS];
    {
        const uint8_t *row = w + static_cast<int64_t>(tile * 16 + r16) * w_s0 + kb0 * 128 + kq * 32;
#pragma unroll
        for (int j = 0; j < QS; ++j) wr[j] = *reinterpret_cast<const int8v_t *>(row + j * 128);
    }
    float swg[QS], swu[QS];
    {
        const float *g = sw + static_cast<int64_t>(tile * 8 / 128) * sw_s0 + kb0;
        const float *u = sw + static_cast<int64_t>((I + tile * 8) / 128) * sw_s0 + kb0;
#pragma unroll
        for (int j = 0; j < QS; ++j) {
            swg[j] = g[j];
            swu[j] = u[j];
        }
    }
    // keep every weight load ahead of the wait for the X block
    __builtin_amdgcn_sched_barrier(0);
    {
        // adjacent vectors belong to the two LDS planes (whose starts share banks): each store
        // writes one plane, so its active lanes fill consecutive 16-byte chunks
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int u = 0; u < kPer; ++u) {
                const int i = threadIdx.x + u * kSwThreads;
                const int v = rot_of(i);  // same parity as i: rot is even
                if (i < kVec && (i & 1) == h)
                    *reinterpret_cast<uint4 *>(xs + Lds::stage_offset(v / (K / 16), v % (K / 16))) = xr[u];
            }
        }
#pragma unroll
        for (int u = 0; u < kSxPer; ++u) {
            const int i = threadIdx.x + u * kSwThreads;
            if (i < kSx) sxs[i] = sr[u];
        }
    }
    __syncthreads();

    // 3. the quarter's MFMAs, scaled per K block: lane columns 0, 1 are gate, 2, 3 up
    floatx4_t acc[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) acc[m] = floatx4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < QS; ++j) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            const int row = m * 16 + r16;
            const int8v_t b = Lds::read(xs, row, kb0 + j, kq);
            const floatx4_t t = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                wr[j], b, floatx4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
            const float sxv = sxs[(kb0 + j) * kSwRows + row];
            const float sg = sxv * swg[j], su = sxv * swu[j];
            acc[m][0] = fmaf(t[0], sg, acc[m][0]);
            acc[m][1] = fmaf(t[1], sg, acc[m][1]);
            acc[m][2] = fmaf(t[2], su, acc[m][2]);
            acc[m][3] = fmaf(t[3], su, acc[m][3]);
        }
        // pin the block's sums here: the MFMAs (which start from zero and touch no
        // memory) may otherwise sink below every later LDS read
#pragma unroll
        for (int m = 0; m < 4; ++m) asm volatile("" : "+v"(acc[m]));
        __builtin_amdgcn_sched_barrier(0);
    }

    // 4. every quarter wave hands its sums over through the (now free) X area;
    // the wave of quarter q then finishes 16-row tile m = q of its column tile,
    // adding the quarters in order 0, 1, 2, 3
    __syncthreads();
    float *red = reinterpret_cast<float *>(xs);
    // layout [quarter][tile][m][lane][4]: a float4 access touches 64 consecutive float4s
    {
        float *dst = red + ((quarter * kSwTiles + tl) * 4 * kWave + lane) * 4;
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
    for (int q = 1; q < kSwQuarters; ++q) {
        const float4 v = *reinterpret_cast<const float4 *>(red + (((q * kSwTiles + tl) * 4 + m) * kWave + lane) * 4);
        sum[0] += v.x;
        sum[1] += v.y;
        sum[2] += v.z;
        sum[3] += v.w;
    }
    // 5. SwiGLU of the bf16 projection values: act columns 8t + 2kq + {0, 1}
    const int col = tile * 8 + kq * 2;
    {
        const int row = m * 16 + r16;
        if (row >= M) return;
        float a[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
            const float g = bf16_to_f32(f32_to_bf16(sum[e]));
            const float u = bf16_to_f32(f32_to_bf16(sum[2 + e]));
            a[e] = g / (1.0f + expf(-g)) * u;
        }
        *reinterpret_cast<uint32_t *>(out + row * o_s0 + col) = pack2_bf16(a[0], a[1]);
    }
}

// Packed row p = 16 t + 4 q + e of the interleaved gate/up matrix is gate row
// 8t + 2q + e (e < 2) or up row 8t + 2q + e - 2 (e >= 2) of the [gate; up] one.
__global__ void __launch_bounds__(256)
pack_swiglu_kernel(const uint8_t *__restrict__ q, int64_t q_s0, int I, int K, uint8_t *__restrict__ packed,
                   int64_t p_s0) {
    const int p = blockIdx.x;
    const int t = p / 16, qq = (p % 16) / 4, e = p % 4;
    const int src = e < 2 ? 8 * t + 2 * qq + e : I + 8 * t + 2 * qq + e - 2;
    for (int c = threadIdx.x * 16; c < K; c += 256 * 16)
        *reinterpret_cast<uint4 *>(packed + static_cast<int64_t>(p) * p_s0 + c) =
            *reinterpret_cast<const uint4 *>(q + static_cast<int64_t>(src) * q_s0 + c);
}

// ---------------------------------------------------------------------------
// Pieces of the tiled FP8 gate/up + SwiGLU below.

typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));  // staging registers (a plain vector type
                                                                    // keeps them out of scratch)

// Global loads of K block kb of the X codes, the weight codes and (thread t < rows) the row scale.
template <int XV, int WV>
__device__ __forceinline__ void tf8_load(u32x4_t (&xr)[XV], u32x4_t (&wr)[WV], float &sr,
                                         const uint8_t *const (&xp)[XV], const uint8_t *const (&wp)[WV],
                                         const float *sxp, int kb, int rows) {
#pragma unroll
    for (int q = 0; q < WV; ++q) wr[q] = *reinterpret_cast<const u32x4_t *>(wp[q] + kb * 128);
#pragma unroll
    for (int q = 0; q < XV; ++q) xr[q] = *reinterpret_cast<const u32x4_t *>(xp[q] + kb * 128);
    if (static_cast<int>(threadIdx.x) < rows) sr = sxp[kb];
}

// A register set into LDS (one plane per pass: the two planes' starts share banks).
template <int BM, int BN, int XV, int WV, int T>
__device__ __forceinline__ void tf8_store(const u32x4_t (&xr)[XV], const u32x4_t (&wr)[WV], float sr, uint8_t *xs,
                                          uint8_t *ws, float *sxs, int chunk) {
    using XL = Fp8Lds<BM, 128>;
    using WL = Fp8Lds<BN, 128>;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        if ((chunk & 1) != h) continue;
#pragma unroll
        for (int q = 0; q < XV; ++q)
            *reinterpret_cast<u32x4_t *>(xs + XL::stage_offset((threadIdx.x + q * T) / 8, chunk)) = xr[q];
#pragma unroll
        for (int q = 0; q < WV; ++q)
            *reinterpret_cast<u32x4_t *>(ws + WL::stage_offset((threadIdx.x + q * T) / 8, chunk)) = wr[q];
    }
    if (static_cast<int>(threadIdx.x) < BM) sxs[threadIdx.x] = sr;
}

// The scaled MFMAs of one staged K block: per 16 x 16 tile one MFMA from zero, then
// acc += t * sx[row] * (gate scale on lane columns 0, 1 | up scale on 2, 3).
template <int MT, int NT, int WM, int WN>
__device__ __forceinline__ void tf8_compute(floatx4_t (&acc)[MT][NT], const uint8_t *xs, const uint8_t *ws,
                                            const float *sxs, const float *ssw, int kb, int wm, int wn, int r16,
                                            int kq) {
    using XL = Fp8Lds<16 * MT * WM, 128>;
    using WL = Fp8Lds<16 * NT * WN, 128>;
    float gs[NT], us[NT];
    const float *sk = ssw + (kb * WN * NT + wn * NT) * 2;
#pragma unroll
    for (int n = 0; n < NT; ++n) {
        gs[n] = sk[2 * n];
        us[n] = sk[2 * n + 1];
    }
    int8v_t a[NT];
#pragma unroll
    for (int n = 0; n < NT; ++n) a[n] = WL::read(ws, wn * 16 * NT + n * 16 + r16, 0, kq);
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int row = wm * 16 * MT + m * 16 + r16;
        const int8v_t b = XL::read(xs, row, 0, kq);
        const float sxv = sxs[row];
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const floatx4_t tt = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(
                a[n], b, floatx4_t{0.f, 0.f, 0.f, 0.f}, 0, 0, 0, 127, 0, 127);
            const float sg = sxv * gs[n], su = sxv * us[n];
            acc[m][n][0] = fmaf(tt[0], sg, acc[m][n][0]);
            acc[m][n][1] = fmaf(tt[1], sg, acc[m][n][1]);
            acc[m][n][2] = fmaf(tt[2], su, acc[m][n][2]);
            acc[m][n][3] = fmaf(tt[3], su, acc[m][n][3]);
        }
    }
}

// ---------------------------------------------------------------------------
constexpr int kTf8MaxBlocks = 32;  // 128-wide K blocks of the tiled FP8 gate/up (K <= 4096)

// Tiled FP8 gate/up + SwiGLU for prefill-sized row counts (a prefill bucket's
// packed prompt tokens, up to 640 rows).  A workgroup owns (16 MT WM) activation
// rows x (16 NT WN) rows of the interleaved gate/up matrix (8 NT WN act columns);
// each of its WM x WN waves a (16 MT) x (16 NT) part.  The K loop stages one 128-byte
// K block -- one scale block -- of the X codes, their scales and the packed
// weight rows per stage through LDS, double buffered, with two register stages
// keeping the global loads of the next two blocks in flight while the MFMAs
// run.  Per block and 16 x 16 tile: one scaled MFMA from zero, then acc += t * sx[row, kb] * sw[block, kb] with the gate scale on
// lane columns 0, 1 and the up scale on 2, 3 -- the per-block arithmetic of the
// decode kernels -- and the epilogue is the fused kernel's SwiGLU.
template <int MT, int NT, int WM, int WN>
__global__ void __launch_bounds__(WM * WN * kWave)
tgemm_fp8_swiglu_kernel(const uint8_t *__restrict__ x, int64_t x_s0, const float *__restrict__ sx, int64_t sx_s0,
                        int M, const uint8_t *__restrict__ w, int64_t w_s0, const float *__restrict__ sw,
                        int64_t sw_s0, int I, int K, uint16_t *__restrict__ out, int64_t o_s0, int tiles_m,
                        int tiles) {
    constexpr int T = WM * WN * kWave;
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    using XL = Fp8Lds<BM, 128>;
    using WL = Fp8Lds<BN, 128>;
    constexpr int XV = BM * 8 / T;  // 16-byte vectors per thread and stage (8 per 128-byte row)
    constexpr int WV = BN * 8 / T;
    static_assert(XV >= 1 && WV >= 1 && XV * T == BM * 8 && WV * T == BN * 8 && BM <= T,
                  "stage splits evenly over the threads");
    __shared__ __attribute__((aligned(16))) uint8_t xs[2][XL::kBytes];
    __shared__ __attribute__((aligned(16))) uint8_t ws[2][WL::kBytes];
    __shared__ float sxs[2][BM];
    __shared__ float ssw[kTf8MaxBlocks * 2 * WN * NT];

    // tile of this workgroup: XCD b % 8 takes tiles (b % 8) * per .. + per - 1, m fastest
    const int per = (tiles + 7) / 8;
    const int t = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (t >= tiles) return;
    const int tm = t % tiles_m, tn = t / tiles_m;
    const int m0 = tm * BM, p0 = tn * BN;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15, kq = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;
    const int chunk = threadIdx.x & 7;  // the thread's 16-byte vector of every staged row

    const uint8_t *xp[XV];
    const uint8_t *wp[WV];
#pragma unroll
    for (int q = 0; q < XV; ++q) {
        const int row = m0 + (threadIdx.x + q * T) / 8;
        xp[q] = x + static_cast<int64_t>(row < M ? row : M - 1) * x_s0 + chunk * 16;
    }
#pragma unroll
    for (int q = 0; q < WV; ++q)
        wp[q] = w + static_cast<int64_t>(p0 + (threadIdx.x + q * T) / 8) * w_s0 + chunk * 16;
    const int srow = m0 + static_cast<int>(threadIdx.x);
    const float *sxp = sx + static_cast<int64_t>(srow < M ? srow : M - 1) * sx_s0;
    // the weight-block scales of every K block, gate then up per 16-row packed tile t of the
    // workgroup: gate rows 8 pt .. of packed tile pt lie in 128-row block 8 pt / 128, up rows in
    // (I + 8 pt) / 128.  Loaded first and kept in LDS, so that no K block's MFMAs wait on a global
    // load queued behind the register stages' loads.
    const int blocks = K / 128;
    constexpr int kSwPer = (kTf8MaxBlocks * 2 * WN * NT + T - 1) / T;
    float swr[kSwPer];
#pragma unroll
    for (int q = 0; q < kSwPer; ++q) {
        const int i = static_cast<int>(threadIdx.x) + q * T;  // (kb, t, gate | up)
        const int kb = i / (2 * WN * NT), t = (i >> 1) - kb * (WN * NT);
        const int r = 8 * (p0 / 16 + t) + ((i & 1) ? I : 0);
        swr[q] = kb < blocks ? sw[static_cast<int64_t>(r / 128) * sw_s0 + kb] : 0.f;
    }

    // two register stages: the global loads of two K blocks are in flight while the MFMAs run
    u32x4_t xa[XV], wa[WV], xb[XV], wb[WV];
    float sa = 0.f, sb = 0.f;

    floatx4_t acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[m][n] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // block k sits in register set k % 2 (a, b) and LDS buffer k % 2.  Step k: MFMAs on buffer
    // k % 2, block k + 1 to LDS, then the loads of block k + 3 into the set block k + 1 left free.
    tf8_load<XV, WV>(xa, wa, sa, xp, wp, sxp, 0, BM);
#pragma unroll
    for (int q = 0; q < kSwPer; ++q) {
        const int i = static_cast<int>(threadIdx.x) + q * T;
        if (i < blocks * 2 * WN * NT) ssw[i] = swr[q];
    }
    tf8_store<BM, BN, XV, WV, T>(xa, wa, sa, xs[0], ws[0], sxs[0], chunk);
    if (blocks > 1) tf8_load<XV, WV>(xb, wb, sb, xp, wp, sxp, 1, BM);
    if (blocks > 2) tf8_load<XV, WV>(xa, wa, sa, xp, wp, sxp, 2, BM);
    __syncthreads();
    for (int kb = 0; kb < blocks; kb += 2) {
        tf8_compute<MT, NT, WM, WN>(acc, xs[0], ws[0], sxs[0], ssw, kb, wm, wn, r16, kq);
        if (kb + 1 < blocks) tf8_store<BM, BN, XV, WV, T>(xb, wb, sb, xs[1], ws[1], sxs[1], chunk);
        if (kb + 3 < blocks) tf8_load<XV, WV>(xb, wb, sb, xp, wp, sxp, kb + 3, BM);
        __syncthreads();
        if (kb + 1 >= blocks) break;
        tf8_compute<MT, NT, WM, WN>(acc, xs[1], ws[1], sxs[1], ssw, kb + 1, wm, wn, r16, kq);
        if (kb + 2 < blocks) tf8_store<BM, BN, XV, WV, T>(xa, wa, sa, xs[0], ws[0], sxs[0], chunk);
        if (kb + 4 < blocks) tf8_load<XV, WV>(xa, wa, sa, xp, wp, sxp, kb + 4, BM);
        __syncthreads();
    }

    // act columns 8 pt + 2 kq + {0, 1} of row m0 + wm 16 MT + 16 m + r16
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int row = m0 + wm * 16 * MT + m * 16 + r16;
        if (row >= M) continue;
#pragma unroll
        for (int n = 0; n < NT; ++n) {
            const int col = (p0 + wn * 16 * NT + n * 16) / 2 + kq * 2;
            float a2[2];
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const float g = bf16_to_f32(f32_to_bf16(acc[m][n][e]));
                const float u = bf16_to_f32(f32_to_bf16(acc[m][n][2 + e]));
                a2[e] = g / (1.0f + expf(-g)) * u;
            }
            *reinterpret_cast<uint32_t *>(out + static_cast<int64_t>(row) * o_s0 + col) = pack2_bf16(a2[0], a2[1]);
        }
    }
}

template <int MT, int NT, int WM, int WN>
int launch_tgemm_fp8_swiglu(const uint8_t *x, int64_t x_s0, const float *sx, int64_t sx_s0, int M, const uint8_t *w,
                            int64_t w_s0, const float *sw, int64_t sw_s0, int I, int K, uint16_t *out, int64_t o_s0,
                            hipStream_t st) {
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    const int tiles_m = (M + BM - 1) / BM, tiles = tiles_m * (2 * I / BN);
    hipLaunchKernelGGL((tgemm_fp8_swiglu_kernel<MT, NT, WM, WN>), dim3((tiles + 7) / 8 * 8), dim3(WM * WN * kWave),
                       0, st, x, x_s0, sx, sx_s0, M, w, w_s0, sw, sw_s0, I, K, out, o_s0, tiles_m, tiles);
    return NQ_LAUNCH_STATUS();
}

// Tile shapes of the tiled FP8 gate/up.  Square: 128 x 128 tiles over 4 x 4 waves of 32 x 32 (101
// registers, sixteen waves in the one workgroup a CU holds; on the 640-token prefill captures 20.1 ms per
// decision against 20.8 for 64 x 128 tiles of 2 x 2 waves, 20.3 for 64 x 128 of 2 x 4 waves and 20.4
// for 128 x 128 of 4 x 2 waves).  Wide: 128 x 256 tiles over 2 x 4 waves of 64 x 64 (256 registers,
// 149 KB of LDS): a 64 x 64 wave tile reads half the LDS bytes per MFMA of a 32 x 32 one, and the
// 32 x 32 tiles' LDS reads (128 KB per CU per K block) outlast their MFMAs.  A round of either shape
// (every CU one workgroup) costs about the same whatever the row count: 19.5 us square, 31 us wide
// (I = 6144, K = 2048: e.g. 640 rows, 2 square rounds 39.1-39.5 us against 1 wide round 33.9-34.5 us;
// 768 rows, 3 square rounds 53.8-54.4 us against 2 wide 60.1-60.4 us), so the launch takes the shape
// with the smaller rounds x round cost.  Fewer than 256 square tiles run the 64 x 64 tiles of 2 x 2
// waves, which fill more CUs.
constexpr int kTf8Square[4] = {2, 2, 4, 4};
constexpr int kTf8Wide[4] = {4, 4, 2, 4};
constexpr int kTf8SquareRound = 39;  // round costs in half microseconds
constexpr int kTf8WideRound = 62;

constexpr int kFp8Slice = 1024;  // K bytes per workgroup slice (M <= 64)

int fp8_slice_of(int M) { return M > 64 ? 512 : kFp8Slice; }

template <int MT, int KS>
void launch_fp8(const uint8_t *x, int64_t x_s0, const float *sx, int64_t sx_s0, int M, const uint8_t *w,
                int64_t w_s0, const float *sw, int64_t sw_s0, int N, int K, uint16_t *out, int64_t o_s0,
                float *part, hipStream_t st) {
    dim3 grid(N / 64, K / KS);
    hipLaunchKernelGGL((gemm_fp8_kernel<MT, KS>), grid, dim3(kFp8Threads), 0, st, x, x_s0, sx, sx_s0, M, w, w_s0,
                       sw, sw_s0, N, out, o_s0, part);
}

bool al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_quantize_fp8_blocks(const uint16_t *w, int64_t w_s0, int N, int K, uint8_t *q, int64_t q_s0,
                                      float *scales, int64_t s_s0, void *stream) {
    NQ_CHECK_ARG(w && q && scales && N >= 0 && K >= 0);
    NQ_CHECK_ARG(N % 128 == 0 && K % 128 == 0);
    NQ_CHECK_ARG(w_s0 >= K && q_s0 >= K && s_s0 >= K / 128 && w_s0 % 8 == 0 && q_s0 % 8 == 0);
    NQ_CHECK_ARG(al16(w) && reinterpret_cast<uintptr_t>(q) % 8 == 0);
    if (N == 0 || K == 0) return NQ_OK;
    hipLaunchKernelGGL(quantize_blocks_kernel, dim3(K / 128, N / 128), dim3(kFp8Threads), 0,
                       static_cast<hipStream_t>(stream), w, w_s0, q, q_s0, scales, s_s0);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_quantize_fp8_rows(const uint16_t *x, int64_t x_s0, int M, int K, uint8_t *q, int64_t q_s0,
                                    float *scales, int64_t s_s0, void *stream) {
    NQ_CHECK_ARG(x && q && scales && M >= 0 && K >= 0 && K % 128 == 0);
    NQ_CHECK_ARG(x_s0 >= K && q_s0 >= K && s_s0 >= K / 128 && x_s0 % 8 == 0 && q_s0 % 8 == 0);
    NQ_CHECK_ARG(al16(x) && reinterpret_cast<uintptr_t>(q) % 8 == 0);
    if (M == 0 || K == 0) return NQ_OK;
    const int64_t total = static_cast<int64_t>(M) * (K / 8);
    const int64_t blocks = (total + kFp8Threads - 1) / kFp8Threads;
    hipLaunchKernelGGL(quantize_rows_kernel, dim3(static_cast<unsigned>(blocks > 4096 ? 4096 : blocks)),
                       dim3(kFp8Threads), 0, static_cast<hipStream_t>(stream), x, x_s0, M, K, q, q_s0, scales, s_s0);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_linear_fp8_splits(int M, int N, int K) {
    if (M <= 0 || M > 128 || N <= 0 || N % 128 != 0 || K <= 0 || K % fp8_slice_of(M) != 0) return -1;
    return K / fp8_slice_of(M);
}

extern "C" int64_t nq_linear_fp8_workspace_bytes(int M, int N, int K, int epilogue) {
    const int S = nq_linear_fp8_splits(M, N, K);
    if (S < 0 || (epilogue != NQ_EPI_NONE && epilogue != NQ_EPI_SILU_MUL && epilogue != NQ_EPI_PARTIALS)) return -1;
    if (S == 1 && epilogue == NQ_EPI_NONE) return 0;
    return static_cast<int64_t>(S) * M * N * 4;
}

extern "C" int nq_linear_fp8(const uint8_t *xq, int64_t x_s0, const float *sx, int64_t sx_s0, const uint8_t *wq,
                             int64_t w_s0, const float *sw, int64_t sw_s0, int M, int N, int K, int epilogue,
                             uint16_t *out, int64_t o_s0, void *workspace, int64_t workspace_bytes, void *stream) {
    NQ_CHECK_ARG(xq && sx && wq && sw && M > 0 && N > 0 && K > 0);
    NQ_CHECK_ARG(epilogue == NQ_EPI_NONE || epilogue == NQ_EPI_SILU_MUL || epilogue == NQ_EPI_PARTIALS);
    const int S = nq_linear_fp8_splits(M, N, K);
    if (S < 0) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K && x_s0 % 16 == 0 && w_s0 % 16 == 0 && al16(xq) && al16(wq));
    NQ_CHECK_ARG(sx_s0 >= K / 128 && sw_s0 >= K / 128);
    const int out_width = epilogue == NQ_EPI_SILU_MUL ? N / 2 : N;
    if (epilogue != NQ_EPI_PARTIALS) NQ_CHECK_ARG(out && o_s0 >= out_width && o_s0 % 8 == 0 && al16(out));
    const int64_t need = nq_linear_fp8_workspace_bytes(M, N, K, epilogue);
    NQ_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need && al16(workspace)));
    float *part = need ? static_cast<float *>(workspace) : nullptr;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int mt = M <= 16 ? 1 : M <= 32 ? 2 : M <= 64 ? 4 : 8;
    switch (mt) {
        case 1: launch_fp8<1, kFp8Slice>(xq, x_s0, sx, sx_s0, M, wq, w_s0, sw, sw_s0, N, K, out, o_s0, part, st); break;
        case 2: launch_fp8<2, kFp8Slice>(xq, x_s0, sx, sx_s0, M, wq, w_s0, sw, sw_s0, N, K, out, o_s0, part, st); break;
        case 4: launch_fp8<4, kFp8Slice>(xq, x_s0, sx, sx_s0, M, wq, w_s0, sw, sw_s0, N, K, out, o_s0, part, st); break;
        default: launch_fp8<8, 512>(xq, x_s0, sx, sx_s0, M, wq, w_s0, sw, sw_s0, N, K, out, o_s0, part, st); break;
    }
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    switch (epilogue) {
        case NQ_EPI_NONE:
            return S > 1 ? launch_reduce_partials(part, S, M, N, out, o_s0, nullptr, st) : NQ_OK;
        case NQ_EPI_SILU_MUL:
            return launch_silu_mul_partials(part, S, M, N / 2, out, o_s0, st);
        default:
            return NQ_OK;
    }
}

extern "C" int nq_fp8_pack_swiglu(const uint8_t *q, int64_t q_s0, int I, int K, uint8_t *packed, int64_t p_s0,
                                  void *stream) {
    NQ_CHECK_ARG(q && packed && I > 0 && K > 0 && I % 8 == 0 && K % 16 == 0);
    NQ_CHECK_ARG(q_s0 >= K && p_s0 >= K && q_s0 % 16 == 0 && p_s0 % 16 == 0 && al16(q) && al16(packed));
    NQ_CHECK_ARG(q != packed);
    hipLaunchKernelGGL(pack_swiglu_kernel, dim3(2 * I), dim3(256), 0, static_cast<hipStream_t>(stream), q, q_s0, I,
                       K, packed, p_s0);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_linear_fp8_swiglu(const uint8_t *xq, int64_t x_s0, const float *sx, int64_t sx_s0, int M,
                                    const uint8_t *packed, int64_t w_s0, const float *sw, int64_t sw_s0, int I, int K,
                                    uint16_t *out, int64_t o_s0, void *stream) {
    NQ_CHECK_ARG(xq && sx && packed && sw && out && M > 0 && I > 0 && K > 0);
    if (M > kSwRows || K != kSwK || I % (8 * kSwTiles) != 0 || I % 128 != 0) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K && x_s0 % 16 == 0 && w_s0 % 16 == 0 && al16(xq) && al16(packed));
    NQ_CHECK_ARG(sx_s0 >= K / 128 && sw_s0 >= K / 128 && o_s0 >= I && o_s0 % 2 == 0);
    NQ_CHECK_ARG(reinterpret_cast<uintptr_t>(out) % 4 == 0);
    hipLaunchKernelGGL((fp8_swiglu_kernel<kSwK>), dim3(I / (8 * kSwTiles)), dim3(kSwThreads), 0,
                       static_cast<hipStream_t>(stream), xq, x_s0, sx, sx_s0, M, packed, w_s0, sw, sw_s0, I, out, o_s0);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_tgemm_fp8_swiglu(const uint8_t *xq, int64_t x_s0, const float *sx, int64_t sx_s0, int M,
                                   const uint8_t *packed, int64_t w_s0, const float *sw, int64_t sw_s0, int I, int K,
                                   uint16_t *out, int64_t o_s0, void *stream) {
    NQ_CHECK_ARG(xq && sx && packed && sw && out && M > 0 && I > 0 && K > 0);
    if (K % 128 || I % 128 || K / 128 > kTf8MaxBlocks) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K && x_s0 % 16 == 0 && w_s0 % 16 == 0 && al16(xq) && al16(packed));
    NQ_CHECK_ARG(sx_s0 >= K / 128 && sw_s0 >= K / 128 && o_s0 >= I && o_s0 % 2 == 0);
    NQ_CHECK_ARG(reinterpret_cast<uintptr_t>(out) % 4 == 0);
    hipStream_t st = static_cast<hipStream_t>(stream);
    constexpr int bm = 16 * kTf8Square[0] * kTf8Square[2], bn = 16 * kTf8Square[1] * kTf8Square[3];
    constexpr int wbm = 16 * kTf8Wide[0] * kTf8Wide[2], wbn = 16 * kTf8Wide[1] * kTf8Wide[3];
    const int square = (M + bm - 1) / bm * (2 * I / bn);
    if (square < 256)
        return launch_tgemm_fp8_swiglu<2, 2, 2, 2>(xq, x_s0, sx, sx_s0, M, packed, w_s0, sw, sw_s0, I, K, out, o_s0,
                                                   st);
    const int wide = (2 * I) % wbn == 0 ? (M + wbm - 1) / wbm * (2 * I / wbn) : 0;
    if (wide > 0 && kTf8WideRound * ((wide + 255) / 256) < kTf8SquareRound * ((square + 255) / 256))
        return launch_tgemm_fp8_swiglu<kTf8Wide[0], kTf8Wide[1], kTf8Wide[2], kTf8Wide[3]>(
            xq, x_s0, sx, sx_s0, M, packed, w_s0, sw, sw_s0, I, K, out, o_s0, st);
    return launch_tgemm_fp8_swiglu<kTf8Square[0], kTf8Square[1], kTf8Square[2], kTf8Square[3]>(
        xq, x_s0, sx, sx_s0, M, packed, w_s0, sw, sw_s0, I, K, out, o_s0, st);
}
