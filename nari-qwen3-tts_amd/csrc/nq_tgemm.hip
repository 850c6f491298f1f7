// Tiled bf16 GEMM for prefill-sized row counts: Y[M, N] = X[M, K] . W[N, K]^T
// with M in the hundreds (a prefill bucket's packed prompt tokens, up to 640)
// -- the talker layer's projections (model/layers.py:195-317 QKV / o / gate_up
// / down) at the shapes of the prefill captures (planner/catalog.py:262-314).
//
// Unlike the decode GEMM (nq_gemm.hip: weights streamed once into registers,
// a few activation rows, split-K planes) the prefill product has enough rows to
// be MFMA work: each workgroup owns a (16 MT WM) x (16 NT WN) output tile, its
// WM x WN waves a (16 MT) x (16 NT) part of it, and the K loop stages 64-wide slices
// of the X and W tiles through LDS, double buffered (the next slice's global
// loads are in flight while the MFMAs run on the current one).  Both operands
// are K-contiguous, so a lane's 16-byte LDS read is one MFMA operand: W rows as
// the A operand (16 output columns x 32 k), X rows as the B operand, and a lane
// ends with four consecutive output columns of one row.  Tiles are handed to
// workgroups XCD by XCD (workgroups go to the 8 XCDs round-robin), m fastest,
// so the workgroups that share a weight tile share one L2.
//
// Epilogues: the bf16 product, or SwiGLU on [gate; up] weights (rows
// 0 .. I - 1 gate, I .. 2I - 1 up): a wave's first NT/2 column tiles take gate
// rows and its last NT/2 the up rows of the same act columns, so a lane holds
// both and stores bf16(silu(bf16(g)) * bf16(u)) -- the rounding of the
// reference's bf16 gate_up followed by silu_and_mul.
#include "nq_common.h"
#include "nq_internal.h"

namespace nq {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float floatx4_t __attribute__((ext_vector_type(4)));
typedef unsigned int u32x4_t __attribute__((ext_vector_type(4)));  // staging registers (a plain vector type
                                                                    // keeps them out of scratch)

constexpr int kTgK = 64;             // K elements per stage
constexpr int kTgC = kTgK / 8;       // 16-byte chunks of a staged row
constexpr int kTgPitch = kTgK + 16;  // LDS row pitch in bf16 (32 bytes of padding)

bool tg_al16(const void *p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

__device__ __forceinline__ bf16x8_t tg_bf16x8(const uint4 &v) {
    bf16x8_t r;
    __builtin_memcpy(&r, &v, sizeof(r));
    return r;
}

// Output modes: bf16 product, SwiGLU of [gate; up], or fp32 split-K planes [S, M, N].
constexpr int kTgBf16 = 0, kTgSwiglu = 1, kTgPlanes = 2;

// Work unit u of a launch: tile (tm, tn) and K slice, m fastest, then n, then the slice; the units
// are handed out XCD by XCD (workgroup b runs on XCD b % 8 and takes units (b % 8) * per ..).
struct TgUnit {
    int tm, tn, slice;
};
__device__ __forceinline__ bool tg_unit(int tiles_m, int tiles_n, int units, TgUnit &u) {
    const int per = (units + 7) / 8;
    const int t = static_cast<int>(blockIdx.x % 8) * per + static_cast<int>(blockIdx.x / 8);
    if (t >= units) return false;
    u.tm = t % tiles_m;
    const int rest = t / tiles_m;
    u.tn = rest % tiles_n;
    u.slice = rest / tiles_n;
    return true;
}

// Global loads of one K slice (stage) of the X and W tiles into a register set.
template <int XV, int WV>
__device__ __forceinline__ void tg_load(u32x4_t (&xr)[XV], u32x4_t (&wr)[WV], const uint16_t *const (&xp)[XV],
                                        const uint16_t *const (&wp)[WV], int stage) {
    const int k0 = stage * kTgK;
#pragma unroll
    for (int q = 0; q < WV; ++q) wr[q] = *reinterpret_cast<const u32x4_t *>(wp[q] + k0);
#pragma unroll
    for (int q = 0; q < XV; ++q) xr[q] = *reinterpret_cast<const u32x4_t *>(xp[q] + k0);
}

// A register set into LDS: vector i = threadIdx.x + T q is tile row i / kTgC, 8-element chunk i % kTgC.
template <int XV, int WV, int T>
__device__ __forceinline__ void tg_store(const u32x4_t (&xr)[XV], const u32x4_t (&wr)[WV], uint16_t *xbuf,
                                         uint16_t *wbuf) {
#pragma unroll
    for (int q = 0; q < XV; ++q) {
        const int i = threadIdx.x + q * T;
        *reinterpret_cast<u32x4_t *>(xbuf + (i / kTgC) * kTgPitch + (i % kTgC) * 8) = xr[q];
    }
#pragma unroll
    for (int q = 0; q < WV; ++q) {
        const int i = threadIdx.x + q * T;
        *reinterpret_cast<u32x4_t *>(wbuf + (i / kTgC) * kTgPitch + (i % kTgC) * 8) = wr[q];
    }
}

// The MFMAs of one staged kTgK-wide K slice: the wave's (16 MT) x (16 NT) part of the tile.
template <int MT, int NT>
__device__ __forceinline__ void tg_compute(floatx4_t (&acc)[MT][NT], const uint16_t *xbuf, const uint16_t *wbuf,
                                           int wm, int wn, int r16, int kq) {
    const uint16_t *wt = wbuf + (wn * 16 * NT + r16) * kTgPitch + kq * 8;
    const uint16_t *xt = xbuf + (wm * 16 * MT + r16) * kTgPitch + kq * 8;
#pragma unroll
    for (int j = 0; j < kTgK / 32; ++j) {
        bf16x8_t a[NT], b[MT];
#pragma unroll
        for (int n = 0; n < NT; ++n) a[n] = tg_bf16x8(*reinterpret_cast<const uint4 *>(wt + n * 16 * kTgPitch + j * 32));
#pragma unroll
        for (int m = 0; m < MT; ++m) b[m] = tg_bf16x8(*reinterpret_cast<const uint4 *>(xt + m * 16 * kTgPitch + j * 32));
#pragma unroll
        for (int m = 0; m < MT; ++m)
#pragma unroll
            for (int n = 0; n < NT; ++n)
                acc[m][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a[n], b[m], acc[m][n], 0, 0, 0);
    }
}

template <int MT, int NT, int WM, int WN, int kMode>
__global__ void __launch_bounds__(WM * WN * kWave)
tgemm_kernel(const uint16_t *__restrict__ x, int64_t x_s0, int M, const uint16_t *__restrict__ w, int64_t w_s0,
             int N, int k_slice, uint16_t *__restrict__ out, int64_t o_s0, float *__restrict__ part, int tiles_m,
             int tiles_n, int units) {
    constexpr int T = WM * WN * kWave;
    constexpr int BM = 16 * MT * WM, BN = 16 * NT * WN;
    constexpr int XV = BM * (kTgK / 8) / T;  // 16-byte vectors per thread and stage
    constexpr int WV = BN * (kTgK / 8) / T;
    static_assert(XV >= 1 && WV >= 1 && XV * T == BM * kTgK / 8 && WV * T == BN * kTgK / 8,
                  "stage splits evenly over the threads");
    static_assert(kMode != kTgSwiglu || NT % 2 == 0, "SwiGLU pairs gate and up column tiles");
    __shared__ __attribute__((aligned(16))) uint16_t xs[2][BM * kTgPitch];
    __shared__ __attribute__((aligned(16))) uint16_t ws[2][BN * kTgPitch];

    TgUnit unit;
    if (!tg_unit(tiles_m, tiles_n, units, unit)) return;
    const int tn = unit.tn;
    const int m0 = unit.tm * BM;
    const int k_begin = unit.slice * k_slice;
    const int I = N / 2;

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int r16 = lane & 15, kq = lane >> 4;
    const int wm = wave / WN, wn = wave % WN;

    // weight row of local tile row r: plain, or (SwiGLU) gate / up rows of the wave's act columns
    auto w_row = [&](int r) __attribute__((always_inline)) -> int64_t {
        if constexpr (kMode == kTgSwiglu) {
            const int half = 8 * NT;  // act columns per wave
            const int wv = r / (16 * NT), rr = r % (16 * NT);
            const int col = tn * (BN / 2) + wv * half + (rr % half);
            return rr < half ? col : I + col;
        } else {
            return static_cast<int64_t>(tn) * BN + r;
        }
    };
    // staging vector i = threadIdx.x + q * T: tile row i / kTgC, 8-element chunk i % kTgC
    const uint16_t *xp[XV];
    const uint16_t *wp[WV];
#pragma unroll
    for (int q = 0; q < XV; ++q) {
        const int i = threadIdx.x + q * T;
        const int row = m0 + i / kTgC;
        xp[q] = x + static_cast<int64_t>(row < M ? row : M - 1) * x_s0 + k_begin + (i % kTgC) * 8;
    }
#pragma unroll
    for (int q = 0; q < WV; ++q) {
        const int i = threadIdx.x + q * T;
        wp[q] = w + w_row(i / kTgC) * w_s0 + k_begin + (i % kTgC) * 8;
    }
    floatx4_t acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int n = 0; n < NT; ++n) acc[m][n] = floatx4_t{0.f, 0.f, 0.f, 0.f};

    // three register stages: the global loads of three K slices are in flight while the MFMAs run.
    // Stage j sits in register set j % 3 (a, b, c) and LDS buffer j % 2.  Step k: MFMAs on buffer
    // k % 2, stage k + 1 to LDS, then the loads of stage k + 4 into the set stage k + 1 left free.
    u32x4_t xa[XV], wa[WV], xb[XV], wb[WV], xc[XV], wc[WV];
    const int stages = k_slice / kTgK;
    tg_load<XV, WV>(xa, wa, xp, wp, 0);
    tg_store<XV, WV, T>(xa, wa, xs[0], ws[0]);
    if (stages > 1) tg_load<XV, WV>(xb, wb, xp, wp, 1);
    if (stages > 2) tg_load<XV, WV>(xc, wc, xp, wp, 2);
    if (stages > 3) tg_load<XV, WV>(xa, wa, xp, wp, 3);
    __syncthreads();
#define NQ_TG_STEP(BUF, XS, WS, K)                                                              \
    tg_compute<MT, NT>(acc, xs[BUF], ws[BUF], wm, wn, r16, kq);                                 \
    if ((K) + 1 < stages) tg_store<XV, WV, T>(XS, WS, xs[(BUF) ^ 1], ws[(BUF) ^ 1]);                \
    if ((K) + 4 < stages) tg_load<XV, WV>(XS, WS, xp, wp, (K) + 4);                              \
    __syncthreads();                                                                            \
    if ((K) + 1 >= stages) break;
    for (int k = 0;; k += 6) {
        NQ_TG_STEP(0, xb, wb, k)
        NQ_TG_STEP(1, xc, wc, k + 1)
        NQ_TG_STEP(0, xa, wa, k + 2)
        NQ_TG_STEP(1, xb, wb, k + 3)
        NQ_TG_STEP(0, xc, wc, k + 4)
        NQ_TG_STEP(1, xa, wa, k + 5)
    }
#undef NQ_TG_STEP

    // the lane holds Y[m0 + wm 16 MT + 16 m + r16][tile column + 16 n + 4 kq + e]
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int row = m0 + wm * 16 * MT + m * 16 + r16;
        if (row >= M) continue;
        if constexpr (kMode == kTgSwiglu) {
            uint16_t *orow = out + static_cast<int64_t>(row) * o_s0;
            const int col0 = tn * (BN / 2) + wn * 8 * NT + kq * 4;
#pragma unroll
            for (int n = 0; n < NT / 2; ++n) {
                float a4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const float g = bf16_to_f32(f32_to_bf16(acc[m][n][e]));
                    const float u = bf16_to_f32(f32_to_bf16(acc[m][n + NT / 2][e]));
                    a4[e] = g / (1.0f + expf(-g)) * u;
                }
                *reinterpret_cast<uint2 *>(orow + col0 + n * 16) =
                    make_uint2(pack2_bf16(a4[0], a4[1]), pack2_bf16(a4[2], a4[3]));
            }
        } else if constexpr (kMode == kTgPlanes) {
            float *prow = part + (static_cast<int64_t>(unit.slice) * M + row) * N;
            const int col0 = tn * BN + wn * 16 * NT + kq * 4;
#pragma unroll
            for (int n = 0; n < NT; ++n)
                *reinterpret_cast<float4 *>(prow + col0 + n * 16) =
                    make_float4(acc[m][n][0], acc[m][n][1], acc[m][n][2], acc[m][n][3]);
        } else {
            uint16_t *orow = out + static_cast<int64_t>(row) * o_s0;
            const int col0 = tn * BN + wn * 16 * NT + kq * 4;
#pragma unroll
            for (int n = 0; n < NT; ++n)
                *reinterpret_cast<uint2 *>(orow + col0 + n * 16) =
                    make_uint2(pack2_bf16(acc[m][n][0], acc[m][n][1]), pack2_bf16(acc[m][n][2], acc[m][n][3]));
        }
    }
}

// 128 x 128 tiles over 4 x 4 waves of 32 x 32 (2 x 2 MFMA tiles each): 68 registers, so the
// sixteen waves of the one workgroup a CU holds (80 KB of LDS) are resident together.  Measured on
// the 640-token prefill captures against 64 x 128 tiles of 2 x 2 waves at two workgroups per CU:
// 20.75 against 21.57 ms per decision (2 x 4 waves of 32 x 64 at 128 x 128: 21.06 ms).
constexpr int kTgShape[4] = {2, 2, 4, 4};
constexpr int kTgMT = kTgShape[0], kTgNT = kTgShape[1], kTgWM = kTgShape[2], kTgWN = kTgShape[3];
constexpr int kTgBM = 16 * kTgMT * kTgWM, kTgBN = 16 * kTgNT * kTgWN;
constexpr int64_t kTgRound = 256;  // workgroups resident at once (one per CU)

// K slices of a launch.  One workgroup fits a CU, so the units run in rounds of 256 and a launch
// costs about rounds x (slice length + a unit's fixed cost, in K columns): the slice
// count minimising that (each slice a multiple of 64 columns and at least 256 of them), the fewest
// slices on a tie.
int tgemm_splits(int M, int N, int K) {
    constexpr int64_t kUnitCost = 512;
    const int64_t tiles = static_cast<int64_t>((M + kTgBM - 1) / kTgBM) * (N / kTgBN);
    int best = 1;
    int64_t best_cost = (tiles + kTgRound - 1) / kTgRound * (K + kUnitCost);
    for (int s = 2; s <= 8; ++s) {
        if (K % (s * kTgK) || K / s < 256) continue;
        const int64_t cost = (tiles * s + kTgRound - 1) / kTgRound * (K / s + kUnitCost);
        if (cost < best_cost) {
            best_cost = cost;
            best = s;
        }
    }
    return best;
}

template <int kMode>
int launch_tgemm(const uint16_t *x, int64_t x_s0, int M, const uint16_t *w, int64_t w_s0, int N, int K, int S,
                 uint16_t *out, int64_t o_s0, float *part, hipStream_t st) {
    const int tiles_m = (M + kTgBM - 1) / kTgBM, tiles_n = N / kTgBN;
    const int units = tiles_m * tiles_n * S;
    hipLaunchKernelGGL((tgemm_kernel<kTgMT, kTgNT, kTgWM, kTgWN, kMode>), dim3((units + 7) / 8 * 8),
                       dim3(kTgWM * kTgWN * kWave), 0, st, x,
                       x_s0, M, w, w_s0, N, K / S, out, o_s0, part, tiles_m, tiles_n, units);
    return NQ_LAUNCH_STATUS();
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_tgemm_splits(int M, int N, int K) {
    if (M <= 0 || N <= 0 || K <= 0 || N % kTgBN || K % kTgK) return -1;
    return tgemm_splits(M, N, K);
}

extern "C" int64_t nq_tgemm_workspace_bytes(int M, int N, int K, int epilogue) {
    const int S = nq_tgemm_splits(M, N, K);
    if (S < 0 || epilogue < NQ_EPI_NONE || epilogue > NQ_EPI_PARTIALS) return -1;
    if (epilogue == NQ_EPI_SILU_MUL || (epilogue == NQ_EPI_NONE && S == 1)) return 0;
    return static_cast<int64_t>(S) * M * N * 4;
}

extern "C" int nq_tgemm(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M, int N, int K,
                        int epilogue, uint16_t *out, int64_t o_s0, uint16_t *residual, const uint16_t *norm_weight,
                        float eps, void *workspace, int64_t workspace_bytes, void *stream) {
    NQ_CHECK_ARG(x && w && M > 0 && N > 0 && K > 0);
    NQ_CHECK_ARG(epilogue >= NQ_EPI_NONE && epilogue <= NQ_EPI_PARTIALS);
    const int S0 = nq_tgemm_splits(M, N, K);
    if (S0 < 0 || x_s0 % 8 || w_s0 % 8 || !tg_al16(x) || !tg_al16(w)) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K);
    const bool swiglu = epilogue == NQ_EPI_SILU_MUL;
    if (swiglu && (N / 2) % (kTgBN / 2)) return NQ_ERR_UNSUPPORTED;
    const int out_width = swiglu ? N / 2 : N;
    if (epilogue != NQ_EPI_PARTIALS) {
        NQ_CHECK_ARG(out && o_s0 >= out_width && o_s0 % 4 == 0 && reinterpret_cast<uintptr_t>(out) % 8 == 0);
    }
    if (epilogue == NQ_EPI_ADD_RMSNORM) {
        NQ_CHECK_ARG(residual && norm_weight && tg_al16(residual) && tg_al16(norm_weight) && o_s0 % 8 == 0 &&
                     tg_al16(out));
        if (N > 8192) return NQ_ERR_UNSUPPORTED;
    }
    const int64_t need = nq_tgemm_workspace_bytes(M, N, K, epilogue);
    NQ_CHECK_ARG(need == 0 || (workspace && workspace_bytes >= need && tg_al16(workspace)));
    float *part = static_cast<float *>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
    if (swiglu) return launch_tgemm<kTgSwiglu>(x, x_s0, M, w, w_s0, N, K, 1, out, o_s0, nullptr, st);
    if (epilogue == NQ_EPI_NONE && S0 == 1)
        return launch_tgemm<kTgBf16>(x, x_s0, M, w, w_s0, N, K, 1, out, o_s0, nullptr, st);
    const int rc = launch_tgemm<kTgPlanes>(x, x_s0, M, w, w_s0, N, K, S0, nullptr, 0, part, st);
    if (rc != NQ_OK) return rc;
    switch (epilogue) {
        case NQ_EPI_NONE:
            return launch_reduce_partials(part, S0, M, N, out, o_s0, nullptr, st);
        case NQ_EPI_ADD_RMSNORM:
            return launch_add_rmsnorm_partials(part, S0, M, N, out, o_s0, residual, norm_weight, eps, st);
        default:
            return NQ_OK;  // the planes stay in the workspace for the caller's consumer
    }
}

extern "C" int nq_tgemm_add_rmsnorm_fp8(const uint16_t *x, int64_t x_s0, const uint16_t *w, int64_t w_s0, int M,
                                        int N, int K, uint16_t *residual, const uint16_t *norm_weight, float eps,
                                        uint8_t *xq, int64_t xq_s0, float *sx, int64_t sx_s0, void *workspace,
                                        int64_t workspace_bytes, void *stream) {
    NQ_CHECK_ARG(x && w && residual && norm_weight && xq && sx && M > 0 && N > 0 && K > 0);
    const int S = nq_tgemm_splits(M, N, K);
    if (S < 0 || N % 128 || N > 8192 || x_s0 % 8 || w_s0 % 8 || !tg_al16(x) || !tg_al16(w))
        return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG(x_s0 >= K && w_s0 >= K && tg_al16(residual) && tg_al16(norm_weight));
    NQ_CHECK_ARG(xq_s0 >= N && xq_s0 % 8 == 0 && reinterpret_cast<uintptr_t>(xq) % 8 == 0 && sx_s0 >= N / 128);
    const int64_t need = static_cast<int64_t>(S) * M * N * 4;
    NQ_CHECK_ARG(workspace && workspace_bytes >= need && tg_al16(workspace));
    float *part = static_cast<float *>(workspace);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int rc = launch_tgemm<kTgPlanes>(x, x_s0, M, w, w_s0, N, K, S, nullptr, 0, part, st);
    if (rc != NQ_OK) return rc;
    return launch_add_rmsnorm_partials_fp8(part, S, M, N, residual, norm_weight, eps, xq, xq_s0, sx, sx_s0, st);
}
