// Incremental codec-decoder step: the stateful kernels of a batch of streams
// decoded together (model/incremental_codec.py:58-466), fp32 like the
// reference codec (no autocast, executor/build.py:91-95).
//
// Layout.  Activations are channels-last [T, C] with the fresh rows of all
// streams concatenated: stream b owns rows [off[b] * u, off[b + 1] * u) of a
// stage whose time axis is u samples per codec frame (u = 1 at the frame rate,
// then x2, x4, x20 ... x2000 after the upsampling layers).  `off` is the
// frame-level exclusive prefix of the streams' fresh frame counts, so ragged
// chunks (12-48 frames) share every launch.  Each stream's state lives in slot
// slots[b] of per-layer device arrays:
//   - causal Conv1d history  [slots, pad, Cin]  (post-activation inputs)
//   - ConvTranspose1d overlap [slots, s, Cout]  (bias-free expansion tail)
//   - transformer K/V          [slots, R, H, D]  (rotated keys, R = window - 1)
//   - frame position / valid context count [slots]
// A conv or transconv reads the old state, then a second small kernel writes
// the new state (in place: each thread owns one (stream, channel) column and
// walks it forward, so no element is overwritten before it is read).
#include <type_traits>

#include "nq_common.h"

namespace nq {
namespace {

constexpr int kCodecThreads = 256;
constexpr int kHistoryPerThread = 16;  // history_update_kernel covers pad * C <= 256 * 16

// stream of stage row t: the largest b with off[b] * u <= t
__device__ __forceinline__ int stream_of(const int32_t *__restrict__ off, int B, int64_t t, int u) {
    int lo = 0, hi = B - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (static_cast<int64_t>(off[mid]) * u <= t) lo = mid;
        else hi = mid - 1;
    }
    return lo;
}

// SnakeBeta x + sin(a x)^2 / b with a = exp(alpha), b = exp(beta) (per channel)
__device__ __forceinline__ float snake(float x, float a, float inv_b) {
    const float s = __sinf(a * x);
    return x + inv_b * s * s;
}

struct Act {
    const float *alpha;  // log-scale, [C] or null (identity)
    const float *beta;
    __device__ __forceinline__ float a_of(int c) const { return expf(alpha[c]); }
    __device__ __forceinline__ float inv_b_of(int c) const { return 1.0f / (expf(beta[c]) + 1e-9f); }
    __device__ __forceinline__ float apply(float x, int c) const {
        if (!alpha) return x;
        return snake(x, a_of(c), inv_b_of(c));
    }
};

// ---------------------------------------------------------------------------
// codebook sum: out[t, c] = sum_q book[q, codes[t, q], c]

__global__ void __launch_bounds__(kCodecThreads)
embed_sum_kernel(const int32_t *__restrict__ codes, int T, int Q, const float *__restrict__ books, int V, int C,
                 float *__restrict__ out, int32_t *status) {
    const int64_t n = static_cast<int64_t>(T) * C;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kCodecThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kCodecThreads) {
        const int64_t t = i / C;
        const int c = static_cast<int>(i - t * C);
        float s = 0.f;
        for (int q = 0; q < Q; ++q) {
            const int id = codes[t * Q + q];
            if (static_cast<unsigned>(id) >= static_cast<unsigned>(V)) {
                if (status) atomicExch(status, NQ_ERR_INVALID_ARGUMENT);
                continue;
            }
            s += books[(static_cast<int64_t>(q) * V + id) * C + c];
        }
        out[i] = s;
    }
}

// ---------------------------------------------------------------------------
// causal Conv1d (groups 1), direct form.  A workgroup covers 256 / CG rows and
// CG groups of 16 output channels; weights of 16 input channels x K taps are
// staged in LDS per round.  Row r, tap k reads input time local - (K-1-k)*dil
// of its own stream: from x when >= 0, else from the stream's history.

constexpr int kConvCi = 16;
constexpr int kConvKMax = 7;

template <int CG>
__global__ void __launch_bounds__(kCodecThreads)
conv_kernel(const float *__restrict__ x, int64_t ldx, int64_t T, const int32_t *__restrict__ off, int B, int u,
            const int32_t *__restrict__ slots, const float *__restrict__ hist, const float *__restrict__ w,
            const float *__restrict__ bias, int Cin, int Cout, int K, int dil, Act act,
            const float *__restrict__ res, int64_t ldres, float *__restrict__ out, int64_t ldo) {
    constexpr int kRows = kCodecThreads / CG;
    __shared__ float ws[CG * 16][kConvCi][kConvKMax];
    __shared__ float sa[kConvCi], sb[kConvCi];
    const int r = threadIdx.x % kRows;
    const int cg = threadIdx.x / kRows;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRows + r;
    const int co0 = blockIdx.y * CG * 16;
    const int pad = (K - 1) * dil;
    const bool live = row < T;
    int b = 0;
    int64_t local = 0, base = 0;
    if (live) {
        b = stream_of(off, B, row, u);
        base = static_cast<int64_t>(off[b]) * u;
        local = row - base;
    }
    const float *hrow = hist + static_cast<int64_t>(live ? slots[b] : 0) * pad * Cin;
    float acc[16];
#pragma unroll
    for (int j = 0; j < 16; ++j) acc[j] = 0.f;

    for (int ci0 = 0; ci0 < Cin; ci0 += kConvCi) {
        const int nci = min(kConvCi, Cin - ci0);
        __syncthreads();
        for (int e = threadIdx.x; e < CG * 16 * kConvCi * K; e += kCodecThreads) {
            const int co = e / (kConvCi * K);
            const int rem = e - co * kConvCi * K;
            const int ci = rem / K, k = rem - ci * K;
            float v = 0.f;
            if (co0 + co < Cout && ci < nci) v = w[(static_cast<int64_t>(co0 + co) * Cin + ci0 + ci) * K + k];
            ws[co][ci][k] = v;
        }
        if (act.alpha && threadIdx.x < nci) {
            sa[threadIdx.x] = act.a_of(ci0 + threadIdx.x);
            sb[threadIdx.x] = act.inv_b_of(ci0 + threadIdx.x);
        }
        __syncthreads();
        if (!live) continue;
        for (int k = 0; k < K; ++k) {
            const int64_t src = local - static_cast<int64_t>(K - 1 - k) * dil;
            const float *p = src >= 0 ? x + (base + src) * ldx + ci0 : hrow + (pad + src) * Cin + ci0;
            const bool activate = src >= 0 && act.alpha;
            for (int ci = 0; ci < nci; ++ci) {
                float xv = p[ci];
                if (activate) xv = snake(xv, sa[ci], sb[ci]);
#pragma unroll
                for (int j = 0; j < 16; ++j) acc[j] += xv * ws[cg * 16 + j][ci][k];
            }
        }
    }
    if (!live) return;
#pragma unroll
    for (int j = 0; j < 16; ++j) {
        const int co = co0 + cg * 16 + j;
        if (co >= Cout) break;
        float y = acc[j] + (bias ? bias[co] : 0.f);
        if (res) y += res[row * ldres + co];
        out[row * ldo + co] = y;
    }
}

// Narrow causal Conv1d (Cin, Cout <= 64): each thread computes every output
// channel of R rows (rows t, t + 256, ..., of the workgroup's 256 R), so each
// weight read from LDS feeds R rows.  The workgroup stages its 256 R rows plus
// the `pad` rows before them, activated once, in LDS (row pitch Cin + 1, so the
// 64 rows a wave reads at one channel hit distinct banks) with the weights as
// [ci][k][co].  A tap whose input time is >= 0 reads the staged row (it lies in
// the same stream); a tap before the stream's first fresh row reads the
// stream's history from global memory.  The thread finds its first row's
// stream by binary search and steps forward for its later rows.  Outputs (and
// the residual) move as float4 when the row strides allow it.
//
// kUnit: the decoder's whole residual unit in one launch (Cin == Cout == C):
// out = res + conv1x1(snake2(conv(snake1(x)) + bias)) + bias2, with res the
// input x itself.  The 1x1 convolution runs in registers on the thread's
// conv outputs (its weights [ci][co] in LDS), in the order of the separate
// 1x1 launch, so the bits are those of the two launches; the intermediate
// tensor never reaches memory.
template <int CO, int R, bool kUnit = false>
__global__ void __launch_bounds__(kCodecThreads)
conv_small_kernel(const float *__restrict__ x, int64_t ldx, int64_t T, const int32_t *__restrict__ off, int B, int u,
                  const int32_t *__restrict__ slots, const float *__restrict__ hist, const float *__restrict__ w,
                  const float *__restrict__ bias, int Cin, int Cout, int K, int dil, Act act,
                  const float *__restrict__ res, int64_t ldres, float *__restrict__ out, int64_t ldo,
                  const float *__restrict__ w2 = nullptr, const float *__restrict__ bias2 = nullptr,
                  Act act2 = Act{nullptr, nullptr}) {
    constexpr int ROWS = kCodecThreads * R;
    extern __shared__ float lds[];
    const int pad = (K - 1) * dil;
    const int pitch = Cin + 1;
    float *xs = lds;                                            // [(ROWS + pad) * pitch]
    float *wsm = xs + ((ROWS + pad) * pitch + 3) / 4 * 4;       // [Cin * K * CO], 16-byte aligned
    float *sa = wsm + Cin * K * CO;                             // [Cin]
    float *sb = sa + Cin;                                       // [Cin]
    float *w2s = sb + Cin + (kUnit ? (4 - (Cin * K * CO + 2 * Cin) % 4) % 4 : 0);  // [Cin][CO], 16-byte aligned
    float *sa2 = w2s + Cin * CO;                                // [Cin]
    float *sb2 = sa2 + Cin;                                     // [Cin]
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * ROWS;
    for (int e = threadIdx.x; e < Cin * K * CO; e += kCodecThreads) {
        const int co = e % CO;
        const int ck = e / CO;
        const int ci = ck / K, k = ck - ci * K;
        wsm[e] = co < Cout ? w[(static_cast<int64_t>(co) * Cin + ci) * K + k] : 0.f;
    }
    if (act.alpha && threadIdx.x < Cin) {
        sa[threadIdx.x] = act.a_of(threadIdx.x);
        sb[threadIdx.x] = act.inv_b_of(threadIdx.x);
    }
    if constexpr (kUnit) {
        for (int e = threadIdx.x; e < Cin * CO; e += kCodecThreads) {
            const int co = e % CO, ci = e / CO;
            w2s[e] = co < Cout ? w2[static_cast<int64_t>(co) * Cin + ci] : 0.f;
        }
        if (act2.alpha && threadIdx.x < Cin) {
            sa2[threadIdx.x] = act2.a_of(threadIdx.x);
            sb2[threadIdx.x] = act2.inv_b_of(threadIdx.x);
        }
    }
    __syncthreads();
    if ((Cin & 3) == 0 && (ldx & 3) == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0) {
        // 128-bit loads, eight per thread in flight before any is activated and stored
        const int vpr = Cin / 4;
        const int nvec = (ROWS + pad) * vpr;
        for (int e0 = threadIdx.x; e0 < nvec; e0 += 8 * kCodecThreads) {
            float4 v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = e0 + i * kCodecThreads;
                const int rr = e / vpr;
                const int64_t g = row0 - pad + rr;
                v[i] = (e < nvec && g >= 0 && g < T)
                           ? *reinterpret_cast<const float4 *>(x + g * ldx + (e - rr * vpr) * 4)
                           : make_float4(0.f, 0.f, 0.f, 0.f);
            }
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int e = e0 + i * kCodecThreads;
                if (e >= nvec) break;
                const int rr = e / vpr, c = (e - rr * vpr) * 4;
                const int64_t g = row0 - pad + rr;
                float f[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
                if (act.alpha && g >= 0 && g < T) {
#pragma unroll
                    for (int q = 0; q < 4; ++q) f[q] = snake(f[q], sa[c + q], sb[c + q]);
                }
#pragma unroll
                for (int q = 0; q < 4; ++q) xs[rr * pitch + c + q] = f[q];
            }
        }
    } else {
        for (int e = threadIdx.x; e < (ROWS + pad) * Cin; e += kCodecThreads) {
            const int rr = e / Cin, c = e - rr * Cin;
            const int64_t g = row0 - pad + rr;
            float v = 0.f;
            if (g >= 0 && g < T) {
                v = x[g * ldx + c];
                if (act.alpha) v = snake(v, sa[c], sb[c]);
            }
            xs[rr * pitch + c] = v;
        }
    }
    __syncthreads();
    const int64_t first = row0 + threadIdx.x;
    // the residual unit meets a second barrier below, so its threads past the end stay (they only
    // skip the stores)
    if (!kUnit && first >= T) return;
    // streams of the thread's rows (non-decreasing)
    int sb_[R];
    int64_t local[R];
    {
        int b = stream_of(off, B, first, u);
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int64_t row = first + static_cast<int64_t>(r) * kCodecThreads;
            while (b + 1 < B && static_cast<int64_t>(off[b + 1]) * u <= row) ++b;
            sb_[r] = b;
            local[r] = row - static_cast<int64_t>(off[b]) * u;
        }
    }
    float acc[R][CO];
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
        for (int j = 0; j < CO; ++j) acc[r][j] = 0.f;
    // taps read the staged rows through LDS addressing when every row of the wave has
    // its whole receptive field in the stream's fresh rows (the common case), else through
    // generic pointers that may point into the history
    bool staged = true;
#pragma unroll
    for (int r = 0; r < R; ++r) staged = staged && local[r] >= pad;
    // one tap's multiply-adds over the input channels: the rows' inputs xr[r][ci], the weights at wk
    // ([ci][k][co] with row pitch kw floats)
    auto channel_loop = [&](const float *const (&xr)[R], const float *wk, int kw, int cin) {
        for (int ci = 0; ci < cin; ++ci) {
            float xv[R];
#pragma unroll
            for (int r = 0; r < R; ++r) xv[r] = xr[r][ci];
            const float4 *w4 = reinterpret_cast<const float4 *>(wk + ci * kw);
#pragma unroll
            for (int j = 0; j < CO / 4; ++j) {
                const float4 ww = w4[j];
#pragma unroll
                for (int r = 0; r < R; ++r) {
                    acc[r][4 * j] += xv[r] * ww.x;
                    acc[r][4 * j + 1] += xv[r] * ww.y;
                    acc[r][4 * j + 2] += xv[r] * ww.z;
                    acc[r][4 * j + 3] += xv[r] * ww.w;
                }
            }
        }
    };
    auto taps = [&](auto lds_only) {
        for (int k = 0; k < K; ++k) {
            const int back = (K - 1 - k) * dil;
            const float *xr[R];
#pragma unroll
            for (int r = 0; r < R; ++r) {
                const int64_t src = local[r] - back;
                if constexpr (decltype(lds_only)::value)
                    xr[r] = xs + (threadIdx.x + r * kCodecThreads + pad - back) * pitch;
                else
                    xr[r] = src >= 0 ? xs + (threadIdx.x + r * kCodecThreads + pad - back) * pitch
                                     : hist + (static_cast<int64_t>(slots[sb_[r]]) * pad + pad + src) * Cin;
            }
            channel_loop(xr, wsm + k * CO, K * CO, Cin);
        }
    };
    if (__all(staged)) taps(std::true_type{});
    else taps(std::false_type{});
    if constexpr (kUnit) {
        // the 1x1 convolution of snake2(conv + bias): each thread parks its rows' activated conv
        // outputs in its own rows of the (now free) staging area and reads them back per channel
        __syncthreads();
        const float *yr[R];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            float *yw = xs + (threadIdx.x + r * kCodecThreads) * pitch;
#pragma unroll
            for (int j = 0; j < CO; ++j) {
                const float y = acc[r][j] + (bias ? bias[j] : 0.f);
                yw[j] = act2.alpha ? snake(y, sa2[j], sb2[j]) : y;
                acc[r][j] = 0.f;
            }
            yr[r] = yw;
        }
        channel_loop(yr, w2s, CO, Cin);
        bias = bias2;
    }
    const bool vec = Cout == CO && (ldo & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0 &&
                     (!res || ((ldres & 3) == 0 && (reinterpret_cast<uintptr_t>(res) & 15) == 0));
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int64_t row = first + static_cast<int64_t>(r) * kCodecThreads;
        if (row >= T) break;
        if (vec) {
#pragma unroll
            for (int j = 0; j < CO / 4; ++j) {
                float4 y = make_float4(acc[r][4 * j], acc[r][4 * j + 1], acc[r][4 * j + 2], acc[r][4 * j + 3]);
                if (bias) {
                    y.x += bias[4 * j];
                    y.y += bias[4 * j + 1];
                    y.z += bias[4 * j + 2];
                    y.w += bias[4 * j + 3];
                }
                if (res) {
                    const float4 q = *reinterpret_cast<const float4 *>(res + row * ldres + 4 * j);
                    y.x += q.x;
                    y.y += q.y;
                    y.z += q.z;
                    y.w += q.w;
                }
                *reinterpret_cast<float4 *>(out + row * ldo + 4 * j) = y;
            }
        } else {
#pragma unroll
            for (int j = 0; j < CO; ++j) {
                if (j >= Cout) break;
                float y = acc[r][j] + (bias ? bias[j] : 0.f);
                if (res) y += res[row * ldres + j];
                out[row * ldo + j] = y;
            }
        }
    }
}

constexpr int conv_small_rows(int CO) { return CO <= 16 ? 2 : 1; }

size_t conv_small_lds(int Cin, int K, int dil, int CO, bool unit = false) {
    const size_t rows = static_cast<size_t>(kCodecThreads) * conv_small_rows(CO);
    const size_t unit_floats = unit ? 3 + static_cast<size_t>(Cin) * CO + 2 * Cin : 0;
    return ((rows + (K - 1) * dil) * (Cin + 1) + 3 + static_cast<size_t>(Cin) * K * CO + 2 * Cin + unit_floats) *
           sizeof(float);
}

// depthwise causal Conv1d (groups == C): one thread per (row, channel)
__global__ void __launch_bounds__(kCodecThreads)
dwconv_kernel(const float *__restrict__ x, int64_t ldx, int64_t T, const int32_t *__restrict__ off, int B, int u,
              const int32_t *__restrict__ slots, const float *__restrict__ hist, const float *__restrict__ w,
              const float *__restrict__ bias, int C, int K, int dil, float *__restrict__ out, int64_t ldo) {
    const int64_t n = T * C;
    const int pad = (K - 1) * dil;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kCodecThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kCodecThreads) {
        const int64_t row = i / C;
        const int c = static_cast<int>(i - row * C);
        const int b = stream_of(off, B, row, u);
        const int64_t base = static_cast<int64_t>(off[b]) * u;
        const int64_t local = row - base;
        const float *hrow = hist + static_cast<int64_t>(slots[b]) * pad * C;
        float y = bias ? bias[c] : 0.f;
        for (int k = 0; k < K; ++k) {
            const int64_t src = local - static_cast<int64_t>(K - 1 - k) * dil;
            const float xv = src >= 0 ? x[(base + src) * ldx + c] : hrow[(pad + src) * C + c];
            y += xv * w[c * K + k];
        }
        out[row * ldo + c] = y;
    }
}

// new history = last pad rows of [history ; act(x)] per stream
__global__ void __launch_bounds__(kCodecThreads)
history_update_kernel(const float *__restrict__ x, int64_t ldx, const int32_t *__restrict__ off, int B, int u,
                      const int32_t *__restrict__ slots, float *__restrict__ hist, int C, int pad, Act act) {
    // one workgroup per stream: every (j, c) of its [pad, C] history is read first (the entries that
    // shift down and the fresh tail rows, activated), then all are written after a barrier, so no
    // entry is overwritten before it is read
    constexpr int kPer = kHistoryPerThread;
    const int b = blockIdx.x;
    const int64_t base = static_cast<int64_t>(off[b]) * u;
    const int64_t F = static_cast<int64_t>(off[b + 1]) * u - base;
    float *h = hist + static_cast<int64_t>(slots[b]) * pad * C;
    const int n = pad * C;
    float v[kPer];
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = threadIdx.x + i * kCodecThreads;
        v[i] = 0.f;
        if (e < n) {
            const int j = e / C, c = e - j * C;
            v[i] = j + F < pad ? h[(j + F) * C + c] : act.apply(x[(base + F - pad + j) * ldx + c], c);
        }
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = threadIdx.x + i * kCodecThreads;
        if (e < n) h[e] = v[i];
    }
}

// ---------------------------------------------------------------------------
// causal ConvTranspose1d, kernel 2s, stride s, overlap s.  Output row p of a
// stream (stage u * s): t0 = p / s, j = p % s,
//   y = bias + x[t0] . W[:, :, j] + (t0 > 0 ? x[t0 - 1] . W[:, :, j + s] : overlap[j])

template <int CG>
__global__ void __launch_bounds__(kCodecThreads)
transconv_kernel(const float *__restrict__ x, int64_t ldx, int64_t T_out, const int32_t *__restrict__ off, int B,
                 int u_in, int s, const int32_t *__restrict__ slots, const float *__restrict__ overlap,
                 const float *__restrict__ w, const float *__restrict__ bias, int Cin, int Cout, Act act,
                 float *__restrict__ out, int64_t ldo) {
    constexpr int kRows = kCodecThreads / CG;
    extern __shared__ float tw[];  // [16 ci][CG*16 co][2s]
    __shared__ float sa[kConvCi], sb[kConvCi];
    const int r = threadIdx.x % kRows;
    const int cg = threadIdx.x / kRows;
    const int64_t row = static_cast<int64_t>(blockIdx.x) * kRows + r;
    const int co0 = blockIdx.y * CG * 16;
    const int u_out = u_in * s;
    const bool live = row < T_out;
    int b = 0;
    int64_t local = 0, base_in = 0;
    if (live) {
        b = stream_of(off, B, row, u_out);
        local = row - static_cast<int64_t>(off[b]) * u_out;
        base_in = static_cast<int64_t>(off[b]) * u_in;
    }
    const int64_t t0 = local / s;
    const int j = static_cast<int>(local - t0 * s);
    float acc[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) acc[q] = 0.f;
    const int ks = 2 * s;
    for (int ci0 = 0; ci0 < Cin; ci0 += kConvCi) {
        const int nci = min(kConvCi, Cin - ci0);
        __syncthreads();
        for (int e = threadIdx.x; e < kConvCi * CG * 16 * ks; e += kCodecThreads) {
            const int ci = e / (CG * 16 * ks);
            const int rem = e - ci * CG * 16 * ks;
            const int co = rem / ks, k = rem - co * ks;
            float v = 0.f;
            if (ci < nci && co0 + co < Cout) v = w[(static_cast<int64_t>(ci0 + ci) * Cout + co0 + co) * ks + k];
            tw[e] = v;
        }
        if (act.alpha && threadIdx.x < nci) {
            sa[threadIdx.x] = act.a_of(ci0 + threadIdx.x);
            sb[threadIdx.x] = act.inv_b_of(ci0 + threadIdx.x);
        }
        __syncthreads();
        if (!live) continue;
        const float *x1 = x + (base_in + t0) * ldx + ci0;
        const float *x0 = t0 > 0 ? x + (base_in + t0 - 1) * ldx + ci0 : nullptr;
        for (int ci = 0; ci < nci; ++ci) {
            float a1 = x1[ci], a0 = x0 ? x0[ci] : 0.f;
            if (act.alpha) {
                a1 = snake(a1, sa[ci], sb[ci]);
                if (x0) a0 = snake(a0, sa[ci], sb[ci]);
            }
            const float *wr = tw + (ci * CG * 16 + cg * 16) * ks;
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[q] += a1 * wr[q * ks + j] + a0 * wr[q * ks + j + s];
        }
    }
    if (!live) return;
    const float *ov = overlap + (static_cast<int64_t>(slots[b]) * s + j) * Cout;
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        const int co = co0 + cg * 16 + q;
        if (co >= Cout) break;
        float y = acc[q] + (bias ? bias[co] : 0.f);
        if (t0 == 0) y += ov[co];
        out[row * ldo + co] = y;
    }
}

// Narrow causal transposed Conv1d (Cout <= 16, stride s): output row r reads input
// rows r / s and r / s - 1 (the stream's rows are aligned to s at this stage).
// The workgroup stages the (at most 256 / s + 3) input rows its 256 output rows read,
// activated once, in LDS (row pitch Cin + 1) with the weights as [ci][co][2s];
// the first output rows of a stream add its carried overlap instead of an
// earlier input row.  Outputs move as float4 when the row stride allows it.
template <int CO>
__global__ void __launch_bounds__(kCodecThreads)
transconv_small_kernel(const float *__restrict__ x, int64_t ldx, int64_t T_out, const int32_t *__restrict__ off,
                       int B, int u_in, int s, const int32_t *__restrict__ slots, const float *__restrict__ overlap,
                       const float *__restrict__ w, const float *__restrict__ bias, int Cin, int Cout, Act act,
                       float *__restrict__ out, int64_t ldo) {
    extern __shared__ float lds[];
    const int ks = 2 * s;
    const int pitch = Cin + 1;
    const int n_max = kCodecThreads / s + 3;  // >= the staged rows for every stride
    float *xs = lds;                                    // [n_max * pitch]
    float *tw = xs + (n_max * pitch + 3) / 4 * 4;       // [Cin][CO][2s]
    float *sa = tw + Cin * CO * ks;                     // [Cin]
    float *sb = sa + Cin;                               // [Cin]
    const int64_t T_in = T_out / s;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * kCodecThreads;
    const int64_t last = row0 + kCodecThreads - 1 < T_out ? row0 + kCodecThreads - 1 : T_out - 1;
    const int64_t in0 = row0 / s - 1;  // staged input row 0 (may be -1)
    const int n_in = static_cast<int>(last / s - in0 + 1);
    for (int e = threadIdx.x; e < Cin * CO * ks; e += kCodecThreads) {
        const int ci = e / (CO * ks);
        const int rem = e - ci * CO * ks;
        const int co = rem / ks, k = rem - co * ks;
        tw[e] = co < Cout ? w[(static_cast<int64_t>(ci) * Cout + co) * ks + k] : 0.f;
    }
    if (act.alpha && threadIdx.x < Cin) {
        sa[threadIdx.x] = act.a_of(threadIdx.x);
        sb[threadIdx.x] = act.inv_b_of(threadIdx.x);
    }
    __syncthreads();
    for (int e = threadIdx.x; e < n_in * Cin; e += kCodecThreads) {
        const int rr = e / Cin, c = e - rr * Cin;
        const int64_t g = in0 + rr;
        float v = 0.f;
        if (g >= 0 && g < T_in) {
            v = x[g * ldx + c];
            if (act.alpha) v = snake(v, sa[c], sb[c]);
        }
        xs[rr * pitch + c] = v;
    }
    __syncthreads();
    const int64_t row = row0 + threadIdx.x;
    if (row >= T_out) return;
    const int u_out = u_in * s;
    const int b = stream_of(off, B, row, u_out);
    const int64_t gi = row / s;
    const int j = static_cast<int>(row - gi * s);
    const bool first = gi == static_cast<int64_t>(off[b]) * u_in;  // the stream's first input row
    const float *x1 = xs + (gi - in0) * pitch;
    const float *x0 = x1 - pitch;
    float acc[CO];
#pragma unroll
    for (int q = 0; q < CO; ++q) acc[q] = 0.f;
    for (int ci = 0; ci < Cin; ++ci) {
        const float a1 = x1[ci], a0 = first ? 0.f : x0[ci];
        const float *wr = tw + ci * CO * ks;
#pragma unroll
        for (int q = 0; q < CO; ++q) acc[q] += a1 * wr[q * ks + j] + a0 * wr[q * ks + j + s];
    }
    const float *ov = overlap + (static_cast<int64_t>(slots[b]) * s + j) * Cout;
    float y[CO];
#pragma unroll
    for (int q = 0; q < CO; ++q) {
        y[q] = acc[q] + (bias && q < Cout ? bias[q] : 0.f);
        if (first && q < Cout) y[q] += ov[q];
    }
    if (Cout == CO && (ldo & 3) == 0 && (reinterpret_cast<uintptr_t>(out) & 15) == 0) {
#pragma unroll
        for (int q = 0; q < CO; q += 4)
            *reinterpret_cast<float4 *>(out + row * ldo + q) = make_float4(y[q], y[q + 1], y[q + 2], y[q + 3]);
    } else {
#pragma unroll
        for (int q = 0; q < CO; ++q)
            if (q < Cout) out[row * ldo + q] = y[q];
    }
}

size_t transconv_small_lds(int Cin, int s, int CO) {
    const size_t n_max = kCodecThreads / s + 3;
    return ((n_max * (Cin + 1) + 3) / 4 * 4 + static_cast<size_t>(Cin) * CO * 2 * s + 2 * Cin) * sizeof(float);
}

// new overlap[j, co] = act(x[F - 1]) . W[:, co, s + j]; thread per (stream, j, co)
__global__ void __launch_bounds__(kCodecThreads)
overlap_update_kernel(const float *__restrict__ x, int64_t ldx, const int32_t *__restrict__ off, int B, int u_in,
                      int s, const int32_t *__restrict__ slots, float *__restrict__ overlap,
                      const float *__restrict__ w, int Cin, int Cout, Act act) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(kCodecThreads) + threadIdx.x;
    if (i >= static_cast<int64_t>(B) * s * Cout) return;
    const int b = static_cast<int>(i / (static_cast<int64_t>(s) * Cout));
    const int rem = static_cast<int>(i - static_cast<int64_t>(b) * s * Cout);
    const int j = rem / Cout, co = rem - j * Cout;
    const int64_t base = static_cast<int64_t>(off[b]) * u_in;
    const int64_t F = static_cast<int64_t>(off[b + 1]) * u_in - base;
    if (F <= 0) return;  // no fresh input: the stored overlap stays
    const float *xl = x + (base + F - 1) * ldx;
    float sum = 0.f;
    for (int ci = 0; ci < Cin; ++ci) sum += act.apply(xl[ci], ci) * w[(static_cast<int64_t>(ci) * Cout + co) * 2 * s + s + j];
    overlap[(static_cast<int64_t>(slots[b]) * s + j) * Cout + co] = sum;
}

// ---------------------------------------------------------------------------
// Gathered operand for running a wide conv or transconv as one GEMM.
//   conv:      A[t, k*Cin + ci] = input of row t at tap k (activated x, or raw history)
//   transconv: A[t, ci] = act(x[t]), A[t, Cin + ci] = act(x[t - 1]) (0 for a stream's
//              first fresh frame; its overlap is added after the GEMM)
// One thread per (row, 4 channels); Cin % 4 == 0.

__global__ void __launch_bounds__(kCodecThreads)
im2col_kernel(const float *__restrict__ x, int64_t ldx, int64_t T, const int32_t *__restrict__ off, int B, int u,
              const int32_t *__restrict__ slots, const float *__restrict__ hist, int Cin, int K, int dil, int transconv,
              Act act, float *__restrict__ a, int64_t lda) {
    const int c4 = Cin / 4;
    const int64_t n = T * K * c4;
    const int pad = transconv ? 0 : (K - 1) * dil;
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kCodecThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kCodecThreads) {
        const int64_t row = i / (K * c4);
        const int rem = static_cast<int>(i - row * K * c4);
        const int k = rem / c4, c = (rem - k * c4) * 4;
        const int b = stream_of(off, B, row, u);
        const int64_t base = static_cast<int64_t>(off[b]) * u;
        const int64_t local = row - base;
        const int64_t src = transconv ? local - k : local - static_cast<int64_t>(K - 1 - k) * dil;
        float4 v = make_float4(0.f, 0.f, 0.f, 0.f);
        if (src >= 0) {
            v = *reinterpret_cast<const float4 *>(x + (base + src) * ldx + c);
            if (act.alpha) {
                v.x = act.apply(v.x, c);
                v.y = act.apply(v.y, c + 1);
                v.z = act.apply(v.z, c + 2);
                v.w = act.apply(v.w, c + 3);
            }
        } else if (!transconv) {
            v = *reinterpret_cast<const float4 *>(hist + (static_cast<int64_t>(slots[b]) * pad + pad + src) * Cin + c);
        }
        *reinterpret_cast<float4 *>(a + row * lda + static_cast<int64_t>(k) * Cin + c) = v;
    }
}

// GEMM-path transconv: add the stored overlap to each stream's first `s`
// output rows, then store the new overlap, which the caller computed as
// (last fresh frame) x (kernel tail): new_ov [B, s * Cout].  Thread per
// (stream, j, co) touches one overlap element only.
__global__ void __launch_bounds__(kCodecThreads)
overlap_fixup_kernel(const int32_t *__restrict__ off, int B, int u_in, int s, const int32_t *__restrict__ slots,
                     float *__restrict__ overlap, const float *__restrict__ new_ov, int Cout, float *__restrict__ out,
                     int64_t ldo) {
    const int64_t i = blockIdx.x * static_cast<int64_t>(kCodecThreads) + threadIdx.x;
    if (i >= static_cast<int64_t>(B) * s * Cout) return;
    const int b = static_cast<int>(i / (static_cast<int64_t>(s) * Cout));
    const int rem = static_cast<int>(i - static_cast<int64_t>(b) * s * Cout);
    const int j = rem / Cout, co = rem - j * Cout;
    const int64_t base = static_cast<int64_t>(off[b]) * u_in;
    const int64_t F = static_cast<int64_t>(off[b + 1]) * u_in - base;
    if (F <= 0) return;
    float *ov = overlap + (static_cast<int64_t>(slots[b]) * s + j) * Cout + co;
    out[(base * s + j) * ldo + co] += *ov;
    *ov = new_ov[static_cast<int64_t>(b) * s * Cout + rem];
}

// ---------------------------------------------------------------------------
// transformer attention of one (stream, head): per-head RMSNorm + RoPE of q
// and of the fresh k (positions = frame_position[slot] + fresh index), the
// sliding-window attention over [retained R frames ; fresh frames], and the
// retained K/V advance, in one workgroup (_pre_transformer, :193-381).
//
// Query i of the stream (position P0 + i) sees the positions P0 + i - R ..
// P0 + i: retained slot j (position P0 - R + j) when j >= R - ctx and j >= i,
// fresh frame f when i - R <= f <= i.  The fresh queries go in blocks of 64;
// for block i0 the key rows are the positions P0 + i0 - R + kappa, kappa in
// [0, R + nq): a retained slot (already rotated in the state) while
// i0 - R + kappa < 0, else fresh frame f = i0 - R + kappa, rotated here (and
// written back in place, so a later block reads it rotated) unless an earlier
// block already did.  K, V and the rotated q of a block are staged in LDS
// (rows of D + 4 floats); query lane j then reads key row j + s for window
// step s, so the 64 lanes read 64 consecutive rows and a 16-byte read covers
// every bank once.  The four waves split the channels: wave w forms partial
// scores over its D/4 channels, the partials meet in LDS, every wave finishes
// the softmax of its lanes and accumulates P V over its own channels.  After
// the last block the new retained rows (the last R positions) are written from
// LDS: the state is read (staged) before this workgroup overwrites it, and no
// other workgroup touches this (stream, head).

constexpr int kWinThreads = 256;
constexpr int kWinWaves = kWinThreads / kWave;
constexpr int kWinQ = 64;     // queries per block (one per lane)
constexpr int kWinMax = 32;   // window (R + 1) the kernel takes

template <int D>
__global__ void __launch_bounds__(kWinThreads)
window_block_kernel(const float *__restrict__ q, float *__restrict__ k, const float *__restrict__ v, int64_t ld,
                    int H, const float *__restrict__ qn, const float *__restrict__ kn, float eps, float log_theta,
                    const int32_t *__restrict__ off, const int32_t *__restrict__ slots,
                    const int64_t *__restrict__ frame_pos, const int32_t *__restrict__ ctx_len, float *state_k,
                    float *state_v, int64_t state_slot_stride, int R, float scale, float *__restrict__ out,
                    int64_t ldo) {
    static_assert(D % 16 == 0 && D <= 64, "four waves of D / 4 channels, 4-channel chunks");
    constexpr int P = D + 4;                // LDS row pitch (floats)
    constexpr int LPR = D / 4;              // lanes (4-channel chunks) per row
    constexpr int RPP = kWinThreads / LPR;  // rows staged per pass
    constexpr int DW = D / kWinWaves;       // channels per wave
    constexpr int CW = DW / 4;              // chunks per wave
    __shared__ __attribute__((aligned(16))) float ks[(kWinMax - 1 + kWinQ) * P];
    __shared__ __attribute__((aligned(16))) float vs[(kWinMax - 1 + kWinQ) * P];
    __shared__ __attribute__((aligned(16))) float qs[kWinQ * P];
    __shared__ float ps[kWinWaves * kWinMax * kWinQ];

    const int b = blockIdx.x / H, h = blockIdx.x - (blockIdx.x / H) * H;
    const int64_t t0 = off[b];
    const int F = off[b + 1] - off[b];
    if (F <= 0) return;  // no fresh frames: nothing attends and the state stays as it is
    const int slot = slots[b];
    const int ctx = ctx_len[slot];
    const int64_t P0 = frame_pos[slot];
    const int W = R + 1;
    const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
    const int c = threadIdx.x % LPR;  // the thread's 4-channel chunk when staging
    float *sk = state_k + static_cast<int64_t>(slot) * state_slot_stride + h * D;
    float *sv = state_v + static_cast<int64_t>(slot) * state_slot_stride + h * D;
    const int64_t srow = static_cast<int64_t>(H) * D;  // state row stride

    // RMSNorm (weight wn) + rotate-half RoPE of a row held as one 4-channel chunk per lane of its
    // LPR-lane group: the group sums the squares, and chunk c pairs with chunk c ^ (LPR / 2)
    // (channels d and d + D / 2, inv_freq of pair d = theta^(-2d/D)), as the reference rotates them
    const bool first = c < LPR / 2;
    float inv_freq[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        const int d = 4 * (first ? c : c - LPR / 2) + e;  // the pair's first channel
        inv_freq[e] = expf(-log_theta * (2.0f * static_cast<float>(d) / static_cast<float>(D)));
    }
    auto norm_rope = [&](float4 x, const float *wn, float pos) {
        float ssq = x.x * x.x + x.y * x.y + x.z * x.z + x.w * x.w;
#pragma unroll
        for (int m = 1; m < LPR; m <<= 1) ssq += __shfl_xor(ssq, m, kWave);
        const float inv = 1.0f / sqrtf(ssq / static_cast<float>(D) + eps);
        const float4 w4 = *reinterpret_cast<const float4 *>(wn + 4 * c);
        const float y[4] = {x.x * inv * w4.x, x.y * inv * w4.y, x.z * inv * w4.z, x.w * inv * w4.w};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            const float partner = __shfl_xor(y[e], LPR / 2, kWave);
            float sn, cs;
            sincosf(pos * inv_freq[e], &sn, &cs);
            o[e] = first ? y[e] * cs - partner * sn : y[e] * cs + partner * sn;
        }
        return make_float4(o[0], o[1], o[2], o[3]);
    };

    int last_i0 = 0;
    for (int i0 = 0; i0 < F; i0 += kWinQ) {
        last_i0 = i0;
        const int nq = F - i0 < kWinQ ? F - i0 : kWinQ;
        const int rows = R + nq;
        // stage K and V rows kappa (position P0 + i0 - R + kappa) and the block's rotated q; a group
        // of LPR lanes owns one row per pass (every lane of a group takes the same branch).  Every
        // load of the block is issued before the first is used, so the passes share one round trip.
        constexpr int KVP = (kWinMax - 1 + kWinQ + RPP - 1) / RPP;  // K/V passes at most
        constexpr int QP = (kWinQ + RPP - 1) / RPP;                 // q passes at most
        float4 kreg[KVP], vreg[KVP], qreg[QP];
#pragma unroll
        for (int pp = 0; pp < KVP; ++pp) {
            const int kappa = pp * RPP + threadIdx.x / LPR;
            const int fi = i0 - R + kappa;
            kreg[pp] = vreg[pp] = make_float4(0.f, 0.f, 0.f, 0.f);
            if (kappa < rows) {
                if (fi < 0) {  // retained slot i0 + kappa, rotated when it was stored
                    kreg[pp] = *reinterpret_cast<const float4 *>(sk + (i0 + kappa) * srow + 4 * c);
                    vreg[pp] = *reinterpret_cast<const float4 *>(sv + (i0 + kappa) * srow + 4 * c);
                } else {
                    kreg[pp] = *reinterpret_cast<const float4 *>(k + (t0 + fi) * ld + h * D + 4 * c);
                    vreg[pp] = *reinterpret_cast<const float4 *>(v + (t0 + fi) * ld + h * D + 4 * c);
                }
            }
        }
#pragma unroll
        for (int pp = 0; pp < QP; ++pp) {
            const int jq = pp * RPP + threadIdx.x / LPR;
            qreg[pp] = jq < nq ? *reinterpret_cast<const float4 *>(q + (t0 + i0 + jq) * ld + h * D + 4 * c)
                               : make_float4(0.f, 0.f, 0.f, 0.f);
        }
#pragma unroll
        for (int pp = 0; pp < KVP; ++pp) {
            const int kappa = pp * RPP + threadIdx.x / LPR;
            const int fi = i0 - R + kappa;
            if (kappa < rows) {
                float4 kv = kreg[pp];
                if (fi >= i0) {  // this block's own frame: rotate it, and keep it rotated in place
                    kv = norm_rope(kv, kn, static_cast<float>(P0 + fi));
                    *reinterpret_cast<float4 *>(k + (t0 + fi) * ld + h * D + 4 * c) = kv;
                }
                *reinterpret_cast<float4 *>(ks + kappa * P + 4 * c) = kv;
                *reinterpret_cast<float4 *>(vs + kappa * P + 4 * c) = vreg[pp];
            }
        }
#pragma unroll
        for (int pp = 0; pp < QP; ++pp) {
            const int jq = pp * RPP + threadIdx.x / LPR;
            if (jq < nq)
                *reinterpret_cast<float4 *>(qs + jq * P + 4 * c) =
                    norm_rope(qreg[pp], qn, static_cast<float>(P0 + i0 + jq));
        }
        __syncthreads();

        // partial scores over wave w's channels: lane j = query i0 + j, window step s = key row j + s
        const int j = lane;
        const bool live = j < nq;
        float4 qv[CW];
#pragma unroll
        for (int u = 0; u < CW; ++u)
            qv[u] = live ? *reinterpret_cast<const float4 *>(qs + j * P + wave * DW + 4 * u) : make_float4(0, 0, 0, 0);
#pragma unroll
        for (int s = 0; s < kWinMax; ++s) {
            if (s >= W) break;
            float dot = 0.f;
            if (live) {
                const float *kr = ks + (j + s) * P + wave * DW;
#pragma unroll
                for (int u = 0; u < CW; ++u) {
                    const float4 kk = *reinterpret_cast<const float4 *>(kr + 4 * u);
                    dot += qv[u].x * kk.x + qv[u].y * kk.y + qv[u].z * kk.z + qv[u].w * kk.w;
                }
            }
            ps[(wave * kWinMax + s) * kWinQ + j] = dot;
        }
        __syncthreads();

        // softmax of the lane's window (in every wave, for its own channels of P V)
        float sc[kWinMax];
        float mx = -INFINITY;
#pragma unroll
        for (int s = 0; s < kWinMax; ++s) {
            sc[s] = -INFINITY;
            const int fi = i0 + j - R + s;  // the key's fresh index (< 0: retained slot R + fi)
            if (s < W && live && (fi >= 0 || R + fi >= R - ctx)) {
                float full = 0.f;
#pragma unroll
                for (int w = 0; w < kWinWaves; ++w) full += ps[(w * kWinMax + s) * kWinQ + j];
                sc[s] = full * scale;
                mx = fmaxf(mx, sc[s]);
            }
        }
        float l = 0.f;
        float acc[DW];
#pragma unroll
        for (int d = 0; d < DW; ++d) acc[d] = 0.f;
#pragma unroll
        for (int s = 0; s < kWinMax; ++s) {
            if (sc[s] != -INFINITY) {
                const float pr = expf(sc[s] - mx);
                l += pr;
                const float *vr = vs + (j + s) * P + wave * DW;
#pragma unroll
                for (int u = 0; u < CW; ++u) {
                    const float4 vv = *reinterpret_cast<const float4 *>(vr + 4 * u);
                    acc[4 * u] += pr * vv.x;
                    acc[4 * u + 1] += pr * vv.y;
                    acc[4 * u + 2] += pr * vv.z;
                    acc[4 * u + 3] += pr * vv.w;
                }
            }
        }
        if (live) {
            float *op = out + (t0 + i0 + j) * ldo + h * D + wave * DW;
            const float il = 1.0f / l;
#pragma unroll
            for (int u = 0; u < CW; ++u)
                *reinterpret_cast<float4 *>(op + 4 * u) =
                    make_float4(acc[4 * u] * il, acc[4 * u + 1] * il, acc[4 * u + 2] * il, acc[4 * u + 3] * il);
        }
        if (i0 + kWinQ < F) __syncthreads();  // the block's LDS rows are read before the next block restages them
    }
    // retained rows jr = 0 .. R-1 <- positions P0 + F - R + jr: row kappa = jr + F - last_i0 of the last
    // block's staged K/V (a retained slot or a rotated fresh frame); staged before the first block's
    // barrier, so every read of the old state precedes these stores
    for (int e = threadIdx.x; e < R * LPR; e += kWinThreads) {
        const int jr = e / LPR, cc = e % LPR;
        const int kappa = jr + F - last_i0;
        *reinterpret_cast<float4 *>(sk + jr * srow + 4 * cc) = *reinterpret_cast<const float4 *>(ks + kappa * P + 4 * cc);
        *reinterpret_cast<float4 *>(sv + jr * srow + 4 * cc) = *reinterpret_cast<const float4 *>(vs + kappa * P + 4 * cc);
    }
}

__global__ void advance_kernel(const int32_t *__restrict__ off, int B, const int32_t *__restrict__ slots,
                               int64_t *__restrict__ frame_pos, int32_t *__restrict__ ctx_len, int R) {
    const int b = blockIdx.x * blockDim.x + threadIdx.x;
    if (b >= B) return;
    const int F = off[b + 1] - off[b];
    const int slot = slots[b];
    frame_pos[slot] += F;
    ctx_len[slot] = min(R, ctx_len[slot] + F);
}

__global__ void __launch_bounds__(kCodecThreads)
pcm16_kernel(const float *__restrict__ x, int64_t n, float *__restrict__ wav, int16_t *__restrict__ pcm) {
    for (int64_t i = blockIdx.x * static_cast<int64_t>(kCodecThreads) + threadIdx.x; i < n;
         i += static_cast<int64_t>(gridDim.x) * kCodecThreads) {
        const float c = fminf(fmaxf(x[i], -1.0f), 1.0f);
        if (wav) wav[i] = c;
        if (pcm) pcm[i] = static_cast<int16_t>(rintf(c * 32767.0f));
    }
}

// ---------------------------------------------------------------------------
// A decoder residual unit of C = 8, 16 or 32 channels on MFMA, for the decoder's
// "high" float32 matmul precision (the reference's convolutions run on cuDNN with
// its TF32 default): out = x + conv1x1(snake2(conv7(snake1(x)) + b1)) + b2 as two
// implicit GEMMs with bf16x3 split products and fp32 sums, each operand v = hi +
// lo + e with hi = bf16(v), lo = bf16(v - hi), |e| <= 2^-16 |v|, a product
// hi*hi + hi*lo + lo*hi.  The 7-tap convolution is D[co][t] = sum_k W[co][k]
// X[k][t] with k = tap * C + ci (zero weights past the seventh tap), X[k][t] =
// snake1(x)[t - (6 - tap) dil][ci]: the weights are the A operand of
// v_mfma_f32_16x16x32_bf16 (split once per workgroup into an LDS fragment table,
// one 16-byte read per lane), the activated input rows the B operand (a lane's 8
// consecutive k are 8 consecutive channels of one input row, staged split in LDS
// as [row][C hi | C lo] with a 16-byte row pad, 8 rows of a lane group then
// cover distinct banks), so a lane ends with 4 consecutive output channels of
// one row.  Rows within (K-1) dil of their stream's start take those taps from
// the stream's history (the wave takes that path only when one of its rows
// needs it).  The activated 7-tap outputs go split, one 16-row tile at a time,
// through the wave's own LDS rows into the B operand of the 1x1 convolution.  A
// workgroup of 4 waves owns 4 x 16 x unit_tiles<C>() output rows.

typedef __bf16 cu_bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 cu_bf16x2 __attribute__((ext_vector_type(2)));
typedef float cu_floatx2 __attribute__((ext_vector_type(2)));
typedef float cu_floatx4 __attribute__((ext_vector_type(4)));

constexpr int kUnitThreads = 256;
constexpr int kUnitTaps = 7;

// 16-row tiles per wave (256 output rows per workgroup): 8 and 16 tiles for 8 and 16 channels measured
// 130 / 48 us against 85 / 39 us per launch, the workgroup's chain being latency-bound
constexpr int kUnitStreamsLds = 1024;  // stream offsets searched in LDS (more streams: in global memory)
template <int C>
constexpr int unit_tiles() {
    return 4;
}
template <int C>
constexpr int unit_rows() {
    return kUnitThreads / kWave * unit_tiles<C>() * 16;  // output rows per workgroup
}

__device__ __forceinline__ uint32_t cu_pack(float a, float b) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((cu_floatx2){a, b}, cu_bf16x2));
}

// hi / lo bf16 words of the pair (a, b); a - bf16(a) is exact in fp32
__device__ __forceinline__ void cu_split2(float a, float b, uint32_t &hi, uint32_t &lo) {
    hi = cu_pack(a, b);
    lo = cu_pack(a - __uint_as_float(hi << 16), b - __uint_as_float(hi & 0xffff0000u));
}

__device__ __forceinline__ cu_bf16x8 cu_frag(const uint4 &v) { return __builtin_bit_cast(cu_bf16x8, v); }

template <int C>
constexpr int unit_ksteps() {
    return (kUnitTaps * C + 31) / 32;
}

template <int C>
size_t unit_mfma_lds(int pad) {
    constexpr int NT = C <= 16 ? 1 : 2;
    constexpr int RB = 4 * C + 16;
    return static_cast<size_t>(unit_ksteps<C>() * NT * 2 * kWave + NT * 2 * kWave) * 16 +
           static_cast<size_t>(unit_rows<C>() + pad) * RB + static_cast<size_t>(kUnitThreads / kWave) * 16 * RB;
}

template <int C>
__global__ void __launch_bounds__(kUnitThreads)
unit_mfma_kernel(const float *__restrict__ x, int64_t ldx, int64_t T, const int32_t *__restrict__ off, int B, int u,
                 const int32_t *__restrict__ slots, const float *__restrict__ hist, int dil,
                 const float *__restrict__ w1, const float *__restrict__ b1, Act act1,
                 const float *__restrict__ w2, const float *__restrict__ b2, Act act2,
                 float *__restrict__ out, int64_t ldo) {
    static_assert(C == 8 || C == 16 || C == 32, "8, 16 or 32 channels");
    constexpr int NT = C <= 16 ? 1 : 2;     // 16-wide output-channel tiles
    constexpr int KS = unit_ksteps<C>();     // 32-k steps of the 7-tap convolution
    constexpr int RB = 4 * C + 16;           // LDS row bytes
    constexpr int VPR = C / 4;               // float4 per input row
    constexpr int MT = unit_tiles<C>();      // 16-row tiles per wave
    constexpr int ROWS = unit_rows<C>();     // output rows per workgroup
    extern __shared__ __attribute__((aligned(16))) char ulds[];
    __shared__ float sp[4][32];              // snake1 a, 1/b; snake2 a, 1/b
    __shared__ int32_t soff[kUnitStreamsLds + 1];
    uint4 *wf1 = reinterpret_cast<uint4 *>(ulds);      // [KS][NT][hi, lo][64 lanes]
    uint4 *wf2 = wf1 + KS * NT * 2 * kWave;            // [NT][hi, lo][64 lanes]
    char *xs = reinterpret_cast<char *>(wf2 + NT * 2 * kWave);
    const int pad = (kUnitTaps - 1) * dil;
    char *ys = xs + (ROWS + pad) * RB;                 // [wave][16 rows][RB]
    const int tid = threadIdx.x;
    const int64_t row0 = static_cast<int64_t>(blockIdx.x) * ROWS;

    // 1. the input rows row0 - pad .. row0 + ROWS - 1, activated and split (rows outside [0, T) zero), in
    // batches of eight 128-bit loads per thread; the first batch is issued before the weight table is
    // built, so that its round trip overlaps the table's
    const int nvec = (ROWS + pad) * VPR;
    auto load_batch = [&](int e0, float4 (&v)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + i * kUnitThreads;
            const int rr = e / VPR;
            const int64_t g = row0 - pad + rr;
            v[i] = (e < nvec && g >= 0 && g < T)
                       ? *reinterpret_cast<const float4 *>(x + g * ldx + (e - rr * VPR) * 4)
                       : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    };
    auto store_batch = [&](int e0, const float4 (&v)[8]) {
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int e = e0 + i * kUnitThreads;
            if (e >= nvec) break;
            const int rr = e / VPR, c4 = (e - rr * VPR) * 4;
            const int64_t g = row0 - pad + rr;
            float f[4] = {v[i].x, v[i].y, v[i].z, v[i].w};
            if (act1.alpha && g >= 0 && g < T) {
#pragma unroll
                for (int q = 0; q < 4; ++q) f[q] = snake(f[q], sp[0][c4 + q], sp[1][c4 + q]);
            }
            uint32_t h0, l0, h1, l1;
            cu_split2(f[0], f[1], h0, l0);
            cu_split2(f[2], f[3], h1, l1);
            *reinterpret_cast<uint2 *>(xs + rr * RB + 2 * c4) = make_uint2(h0, h1);
            *reinterpret_cast<uint2 *>(xs + rr * RB + 2 * C + 2 * c4) = make_uint2(l0, l1);
        }
    };
    float4 vb[8];
    load_batch(tid, vb);

    // 2. the weights as split MFMA A fragments: lane (r16, kq) of step j holds W[co = 16 nt + r16][k = 32 j + 8 kq .. + 7]
    for (int e = tid; e < KS * NT * kWave; e += kUnitThreads) {
        const int ln = e % kWave, nt = (e / kWave) % NT, j = e / (kWave * NT);
        const int co = nt * 16 + (ln & 15), k0 = 32 * j + 8 * (ln >> 4);
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            float v2[2];
#pragma unroll
            for (int q = 0; q < 2; ++q) {
                const int kk = k0 + 2 * p + q, tap = kk / C, ci = kk - (kk / C) * C;
                v2[q] = (co < C && tap < kUnitTaps) ? w1[(static_cast<int64_t>(co) * C + ci) * kUnitTaps + tap] : 0.f;
            }
            cu_split2(v2[0], v2[1], hi[p], lo[p]);
        }
        wf1[((j * NT + nt) * 2) * kWave + ln] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        wf1[((j * NT + nt) * 2 + 1) * kWave + ln] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    for (int e = tid; e < NT * kWave; e += kUnitThreads) {
        const int ln = e % kWave, nt = e / kWave;
        const int co = nt * 16 + (ln & 15), ci0 = 8 * (ln >> 4);
        uint32_t hi[4], lo[4];
#pragma unroll
        for (int p = 0; p < 4; ++p) {
            const int ci = ci0 + 2 * p;
            const float a = (co < C && ci < C) ? w2[co * C + ci] : 0.f;
            const float b = (co < C && ci + 1 < C) ? w2[co * C + ci + 1] : 0.f;
            cu_split2(a, b, hi[p], lo[p]);
        }
        wf2[(nt * 2) * kWave + ln] = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        wf2[(nt * 2 + 1) * kWave + ln] = make_uint4(lo[0], lo[1], lo[2], lo[3]);
    }
    const bool off_lds = B <= kUnitStreamsLds;
    if (off_lds)
        for (int i = tid; i <= B; i += kUnitThreads) soff[i] = off[i];
    if (tid < C) {
        sp[0][tid] = act1.alpha ? act1.a_of(tid) : 0.f;
        sp[1][tid] = act1.alpha ? act1.inv_b_of(tid) : 0.f;
        sp[2][tid] = act2.alpha ? act2.a_of(tid) : 0.f;
        sp[3][tid] = act2.alpha ? act2.inv_b_of(tid) : 0.f;
    }

    __syncthreads();  // the snake parameters and stream offsets
    store_batch(tid, vb);
    for (int e0 = tid + 8 * kUnitThreads; e0 < nvec; e0 += 8 * kUnitThreads) {
        load_batch(e0, vb);
        store_batch(e0, vb);
    }
    __syncthreads();

    // 3. the 7-tap convolution: wave w owns rows row0 + (MT w + m) 16 + r16, m < MT
    const int lane = tid & (kWave - 1), wave = tid / kWave;
    const int r16 = lane & 15, kq = lane >> 4;
    // the lane's row of tile m is row0 + (MT w + m) 16 + r16; its offset from its stream's first row
    // (pad when far enough: the rows of a workgroup lie in few streams, so the search runs once per tile)
    const int32_t *offs = off_lds ? soff : off;
    int local[MT];
    bool near_start = false;
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int64_t t = row0 + (wave * MT + m) * 16 + r16;
        local[m] = pad;
        if (t < T) {
            const int b = stream_of(offs, B, t, u);
            const int64_t l = t - static_cast<int64_t>(offs[b]) * u;
            local[m] = l < pad ? static_cast<int>(l) : pad;
            near_start = near_start || l < pad;
        }
    }
    // the residual rows of the epilogue, loaded now so that their round trip overlaps the MFMAs
    float4 xres[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m) {
        const int64_t t = row0 + (wave * MT + m) * 16 + r16;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int co = nt * 16 + 4 * kq;
            xres[m][nt] = (co < C && t < T) ? *reinterpret_cast<const float4 *>(x + t * ldx + co)
                                            : make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
    const bool slow = __any(near_start);
    cu_floatx4 acc[MT][NT];
#pragma unroll
    for (int m = 0; m < MT; ++m)
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) acc[m][nt] = cu_floatx4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < KS; ++j) {
        cu_bf16x8 ah[NT], al[NT];
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            ah[nt] = cu_frag(wf1[((j * NT + nt) * 2) * kWave + lane]);
            al[nt] = cu_frag(wf1[((j * NT + nt) * 2 + 1) * kWave + lane]);
        }
        const int k0 = 32 * j + 8 * kq, tap = k0 / C, cb = k0 - (k0 / C) * C;
        const int back = tap < kUnitTaps ? (kUnitTaps - 1 - tap) * dil : 0;  // past the 7th tap: zero weights
#pragma unroll
        for (int m = 0; m < MT; ++m) {
            const char *rp = xs + ((wave * MT + m) * 16 + r16 + pad - back) * RB + 2 * cb;
            uint4 bh = *reinterpret_cast<const uint4 *>(rp);
            uint4 bl = *reinterpret_cast<const uint4 *>(rp + 2 * C);
            if (slow && tap < kUnitTaps && local[m] - back < 0) {
                // a row within pad of its stream's start: this tap reads the stream's history
                const int b = stream_of(offs, B, row0 + (wave * MT + m) * 16 + r16, u);
                const float *hp =
                    hist + (static_cast<int64_t>(slots[b]) * pad + pad + local[m] - back) * C + cb;
                const float4 h0 = *reinterpret_cast<const float4 *>(hp);
                const float4 h1 = *reinterpret_cast<const float4 *>(hp + 4);
                cu_split2(h0.x, h0.y, bh.x, bl.x);
                cu_split2(h0.z, h0.w, bh.y, bl.y);
                cu_split2(h1.x, h1.y, bh.z, bl.z);
                cu_split2(h1.z, h1.w, bh.w, bl.w);
            }
#pragma unroll
            for (int nt = 0; nt < NT; ++nt) {
                acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(al[nt], cu_frag(bh), acc[m][nt], 0, 0, 0);
                acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[nt], cu_frag(bl), acc[m][nt], 0, 0, 0);
                acc[m][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(ah[nt], cu_frag(bh), acc[m][nt], 0, 0, 0);
            }
        }
    }

    // 4. per tile: y = snake2(conv + b1), split into the wave's own 16 LDS rows (lane (r16, kq) holds
    // y[row r16][co = 16 nt + 4 kq .. + 3]), read back as the B operand of the 1x1 convolution (lane
    // (r16, kq) = y[row r16][ci = 8 kq .. + 7]), then the residual
    char *yw = ys + wave * 16 * RB;
    cu_bf16x8 a2h[NT], a2l[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
        a2h[nt] = cu_frag(wf2[(nt * 2) * kWave + lane]);
        a2l[nt] = cu_frag(wf2[(nt * 2 + 1) * kWave + lane]);
    }
#pragma unroll
    for (int m = 0; m < MT; ++m) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            const int co = nt * 16 + 4 * kq;
            if (co >= C) continue;
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                y[e] = acc[m][nt][e] + (b1 ? b1[co + e] : 0.f);
                if (act2.alpha) y[e] = snake(y[e], sp[2][co + e], sp[3][co + e]);
            }
            uint32_t h0, l0, h1, l1;
            cu_split2(y[0], y[1], h0, l0);
            cu_split2(y[2], y[3], h1, l1);
            char *rp = yw + r16 * RB + 2 * co;
            *reinterpret_cast<uint2 *>(rp) = make_uint2(h0, h1);
            *reinterpret_cast<uint2 *>(rp + 2 * C) = make_uint2(l0, l1);
        }
        __builtin_amdgcn_wave_barrier();  // the wave reads back what its own lanes wrote (LDS keeps its order)
        uint4 bh = make_uint4(0, 0, 0, 0), bl = make_uint4(0, 0, 0, 0);
        if (8 * kq < C) {
            const char *rp = yw + r16 * RB + 16 * kq;
            bh = *reinterpret_cast<const uint4 *>(rp);
            bl = *reinterpret_cast<const uint4 *>(rp + 2 * C);
        }
        __builtin_amdgcn_wave_barrier();  // every lane has read the tile before the next one is written
        const int64_t t = row0 + (wave * MT + m) * 16 + r16;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
            cu_floatx4 d = cu_floatx4{0.f, 0.f, 0.f, 0.f};
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2l[nt], cu_frag(bh), d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2h[nt], cu_frag(bl), d, 0, 0, 0);
            d = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a2h[nt], cu_frag(bh), d, 0, 0, 0);
            const int co = nt * 16 + 4 * kq;
            if (co >= C || t >= T) continue;
            const float4 xr = xres[m][nt];
            float4 o;
            o.x = xr.x + d[0] + (b2 ? b2[co] : 0.f);
            o.y = xr.y + d[1] + (b2 ? b2[co + 1] : 0.f);
            o.z = xr.z + d[2] + (b2 ? b2[co + 2] : 0.f);
            o.w = xr.w + d[3] + (b2 ? b2[co + 3] : 0.f);
            *reinterpret_cast<float4 *>(out + t * ldo + co) = o;
        }
    }
}

int grid_for(int64_t n) {
    const int64_t g = (n + kCodecThreads - 1) / kCodecThreads;
    return static_cast<int>(g < 1 ? 1 : g > 8192 ? 8192 : g);
}

}  // namespace
}  // namespace nq

using namespace nq;

extern "C" int nq_codec_embed_sum(const int32_t *codes, int T, int Q, const float *books, int V, int C, float *out,
                                  int32_t *status, void *stream) {
    NQ_CHECK_ARG(codes && books && out && T >= 0 && Q > 0 && V > 0 && C > 0);
    if (T == 0) return NQ_OK;
    hipLaunchKernelGGL(embed_sum_kernel, dim3(grid_for(static_cast<int64_t>(T) * C)), dim3(kCodecThreads), 0,
                       static_cast<hipStream_t>(stream), codes, T, Q, books, V, C, out, status);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_causal_conv(const float *x, int64_t ldx, int64_t T, const int32_t *offsets, int B, int u,
                                    const int32_t *slots, float *history, const float *w, const float *bias, int Cin,
                                    int Cout, int K, int dilation, int groups, const float *act_alpha,
                                    const float *act_beta, const float *residual, int64_t ldres, float *out,
                                    int64_t ldo, void *stream) {
    NQ_CHECK_ARG(x && offsets && slots && w && out && B > 0 && u > 0 && T >= 0);
    NQ_CHECK_ARG(Cin > 0 && Cout > 0 && K >= 1 && K <= kConvKMax && dilation >= 1);
    NQ_CHECK_ARG(groups == 1 || (groups == Cin && Cin == Cout && !residual && !act_alpha));
    NQ_CHECK_ARG((act_alpha == nullptr) == (act_beta == nullptr));
    NQ_CHECK_ARG(ldx >= Cin && ldo >= Cout && (!residual || ldres >= Cout));
    const int pad = (K - 1) * dilation;
    NQ_CHECK_ARG(pad == 0 || history);
    if (pad * Cin > kCodecThreads * kHistoryPerThread) return NQ_ERR_UNSUPPORTED;
    if (T == 0) return NQ_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const Act act{act_alpha, act_beta};
    const int co_pad = Cout <= 8 ? 8 : Cout <= 16 ? 16 : Cout <= 32 ? 32 : 64;
    if (groups == 1 && Cin <= 64 && Cout <= 64 && conv_small_lds(Cin, K, dilation, co_pad) <= 150 * 1024) {
        const size_t lds = conv_small_lds(Cin, K, dilation, co_pad);
        const int64_t rows = static_cast<int64_t>(kCodecThreads) * conv_small_rows(co_pad);
        const dim3 grid(static_cast<unsigned>((T + rows - 1) / rows));
#define NQ_SMALL(CO)                                                                                              \
        hipLaunchKernelGGL((conv_small_kernel<CO, conv_small_rows(CO)>), grid, dim3(kCodecThreads), lds, st, x, ldx, \
                           T, offsets, B, u, slots, history, w, bias, Cin, Cout, K, dilation, act, residual, ldres,   \
                           out, ldo)
        if (co_pad == 8) NQ_SMALL(8);
        else if (co_pad == 16) NQ_SMALL(16);
        else if (co_pad == 32) NQ_SMALL(32);
        else NQ_SMALL(64);
#undef NQ_SMALL
    } else if (groups == 1) {
        const int cg = Cout <= 16 ? 1 : Cout <= 32 ? 2 : 4;
        const int rows = kCodecThreads / cg;
        dim3 grid(static_cast<unsigned>((T + rows - 1) / rows), static_cast<unsigned>((Cout + cg * 16 - 1) / (cg * 16)));
        if (cg == 1)
            hipLaunchKernelGGL(conv_kernel<1>, grid, dim3(kCodecThreads), 0, st, x, ldx, T, offsets, B, u, slots,
                               history, w, bias, Cin, Cout, K, dilation, act, residual, ldres, out, ldo);
        else if (cg == 2)
            hipLaunchKernelGGL(conv_kernel<2>, grid, dim3(kCodecThreads), 0, st, x, ldx, T, offsets, B, u, slots,
                               history, w, bias, Cin, Cout, K, dilation, act, residual, ldres, out, ldo);
        else
            hipLaunchKernelGGL(conv_kernel<4>, grid, dim3(kCodecThreads), 0, st, x, ldx, T, offsets, B, u, slots,
                               history, w, bias, Cin, Cout, K, dilation, act, residual, ldres, out, ldo);
    } else {
        hipLaunchKernelGGL(dwconv_kernel, dim3(grid_for(T * Cin)), dim3(kCodecThreads), 0, st, x, ldx, T, offsets, B,
                           u, slots, history, w, bias, Cin, K, dilation, out, ldo);
    }
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    if (pad > 0) {
        hipLaunchKernelGGL(history_update_kernel, dim3(B), dim3(kCodecThreads),
                           0, st, x, ldx, offsets, B, u, slots, history, Cin, pad, groups == 1 ? act : Act{nullptr, nullptr});
    }
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_residual_unit(const float *x, int64_t ldx, int64_t T, const int32_t *offsets, int B, int u,
                                      const int32_t *slots, float *history, int C, int K, int dilation, const float *w1,
                                      const float *b1, const float *a1_alpha, const float *a1_beta, const float *w2,
                                      const float *b2, const float *a2_alpha, const float *a2_beta, float *out,
                                      int64_t ldo, int precision, void *stream) {
    NQ_CHECK_ARG(x && offsets && slots && history && w1 && w2 && out && B > 0 && u > 0 && T >= 0);
    NQ_CHECK_ARG(C > 0 && K >= 2 && K <= kConvKMax && dilation >= 1 && ldx >= C && ldo >= C && out != x);
    NQ_CHECK_ARG(precision == NQ_MATMUL_HIGHEST || precision == NQ_MATMUL_HIGH);
    if (K != kConvKMax) return NQ_ERR_UNSUPPORTED;  // the fused kernels are built for 7 taps
    if ((K - 1) * dilation * C > kCodecThreads * kHistoryPerThread) return NQ_ERR_UNSUPPORTED;
    NQ_CHECK_ARG((a1_alpha == nullptr) == (a1_beta == nullptr) && (a2_alpha == nullptr) == (a2_beta == nullptr));
    const int co_pad = C <= 8 ? 8 : C <= 16 ? 16 : 32;
    if (C > 32 || C != co_pad) return NQ_ERR_UNSUPPORTED;
    // the split-product MFMA kernel for 16 and 32 channels; 8 channels keep the fp32 direct kernel at
    // either precision (at 1.98 M rows: 58 us against 84 us for the MFMA kernel, whose workgroups are
    // latency-bound at that width)
    const bool split = precision == NQ_MATMUL_HIGH && C >= 16;
    const int pad = (K - 1) * dilation;
    if (split && (ldx % 4 || ldo % 4 || ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(out) |
                                          reinterpret_cast<uintptr_t>(history)) & 15)))
        return NQ_ERR_UNSUPPORTED;
    const size_t lds = split ? (C == 8 ? unit_mfma_lds<8>(pad) : C == 16 ? unit_mfma_lds<16>(pad)
                                                                          : unit_mfma_lds<32>(pad))
                             : conv_small_lds(C, K, dilation, co_pad, true);
    if (lds > 150 * 1024) return NQ_ERR_UNSUPPORTED;
    if (T == 0) return NQ_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const Act act1{a1_alpha, a1_beta}, act2{a2_alpha, a2_beta};
    if (split) {
#define NQ_UNIT(CC)                                                                                                  \
        hipLaunchKernelGGL(unit_mfma_kernel<CC>, dim3(static_cast<unsigned>((T + unit_rows<CC>() - 1) / unit_rows<CC>())), \
                           dim3(kUnitThreads), lds, st, x, ldx, T, offsets, B, u, slots, history, dilation, w1, b1,     \
                           act1, w2, b2, act2, out, ldo)
        if (C == 8) NQ_UNIT(8);
        else if (C == 16) NQ_UNIT(16);
        else NQ_UNIT(32);
#undef NQ_UNIT
    } else {
        const int64_t rows = static_cast<int64_t>(kCodecThreads) * conv_small_rows(co_pad);
        const dim3 grid(static_cast<unsigned>((T + rows - 1) / rows));
#define NQ_UNIT(CO)                                                                                                 \
        hipLaunchKernelGGL((conv_small_kernel<CO, conv_small_rows(CO), true>), grid, dim3(kCodecThreads), lds, st, x, \
                           ldx, T, offsets, B, u, slots, history, w1, b1, C, C, K, dilation, act1, x, ldx, out, ldo, \
                           w2, b2, act2)
        if (co_pad == 8) NQ_UNIT(8);
        else if (co_pad == 16) NQ_UNIT(16);
        else NQ_UNIT(32);
#undef NQ_UNIT
    }
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL(history_update_kernel, dim3(B), dim3(kCodecThreads), 0, st,
                       x, ldx, offsets, B, u, slots, history, C, (K - 1) * dilation, act1);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_causal_transconv(const float *x, int64_t ldx, int64_t T_in, const int32_t *offsets, int B,
                                         int u_in, int stride_s, const int32_t *slots, float *overlap, const float *w,
                                         const float *bias, int Cin, int Cout, const float *act_alpha,
                                         const float *act_beta, float *out, int64_t ldo, void *stream) {
    NQ_CHECK_ARG(x && offsets && slots && overlap && w && out && B > 0 && u_in > 0 && stride_s >= 1 && T_in >= 0);
    NQ_CHECK_ARG(Cin > 0 && Cout > 0 && ldx >= Cin && ldo >= Cout);
    NQ_CHECK_ARG((act_alpha == nullptr) == (act_beta == nullptr));
    if (T_in == 0) return NQ_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const Act act{act_alpha, act_beta};
    const int cg = Cout <= 16 ? 1 : Cout <= 32 ? 2 : 4;
    const int rows = kCodecThreads / cg;
    const int64_t T_out = T_in * stride_s;
    const int co_pad = Cout <= 8 ? 8 : 16;
    if (Cout <= 16 && transconv_small_lds(Cin, stride_s, co_pad) <= 64 * 1024) {
        const size_t lds = transconv_small_lds(Cin, stride_s, co_pad);
        const dim3 grid(static_cast<unsigned>((T_out + kCodecThreads - 1) / kCodecThreads));
        if (co_pad == 8)
            hipLaunchKernelGGL(transconv_small_kernel<8>, grid, dim3(kCodecThreads), lds, st, x, ldx, T_out, offsets, B,
                               u_in, stride_s, slots, overlap, w, bias, Cin, Cout, act, out, ldo);
        else
            hipLaunchKernelGGL(transconv_small_kernel<16>, grid, dim3(kCodecThreads), lds, st, x, ldx, T_out, offsets,
                               B, u_in, stride_s, slots, overlap, w, bias, Cin, Cout, act, out, ldo);
        if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
        hipLaunchKernelGGL(overlap_update_kernel, dim3(grid_for(static_cast<int64_t>(B) * stride_s * Cout)),
                           dim3(kCodecThreads), 0, st, x, ldx, offsets, B, u_in, stride_s, slots, overlap, w, Cin, Cout,
                           act);
        return NQ_LAUNCH_STATUS();
    }
    const size_t lds = static_cast<size_t>(kConvCi) * cg * 16 * 2 * stride_s * sizeof(float);
    if (lds > 64 * 1024) return NQ_ERR_UNSUPPORTED;
    dim3 grid(static_cast<unsigned>((T_out + rows - 1) / rows), static_cast<unsigned>((Cout + cg * 16 - 1) / (cg * 16)));
    if (cg == 1)
        hipLaunchKernelGGL(transconv_kernel<1>, grid, dim3(kCodecThreads), lds, st, x, ldx, T_out, offsets, B, u_in,
                           stride_s, slots, overlap, w, bias, Cin, Cout, act, out, ldo);
    else if (cg == 2)
        hipLaunchKernelGGL(transconv_kernel<2>, grid, dim3(kCodecThreads), lds, st, x, ldx, T_out, offsets, B, u_in,
                           stride_s, slots, overlap, w, bias, Cin, Cout, act, out, ldo);
    else
        hipLaunchKernelGGL(transconv_kernel<4>, grid, dim3(kCodecThreads), lds, st, x, ldx, T_out, offsets, B, u_in,
                           stride_s, slots, overlap, w, bias, Cin, Cout, act, out, ldo);
    if (hipGetLastError() != hipSuccess) return NQ_ERR_LAUNCH;
    hipLaunchKernelGGL(overlap_update_kernel, dim3(grid_for(static_cast<int64_t>(B) * stride_s * Cout)),
                       dim3(kCodecThreads), 0, st, x, ldx, offsets, B, u_in, stride_s, slots, overlap, w, Cin, Cout, act);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_window_attention(float *q, float *k, const float *v, int64_t ld, int T, int H, int D,
                                         const float *q_norm, const float *k_norm, float eps, float rope_theta,
                                         const int32_t *offsets, int B, const int32_t *slots, const int64_t *frame_pos,
                                         const int32_t *ctx_len, float *state_k, float *state_v,
                                         int64_t state_slot_stride, int R, int window, float *out, int64_t ldo,
                                         void *stream) {
    NQ_CHECK_ARG(q && k && v && q_norm && k_norm && offsets && slots && frame_pos && ctx_len && out);
    NQ_CHECK_ARG(state_k && state_v && T >= 0 && B > 0 && H > 0 && R >= 0 && window == R + 1);
    NQ_CHECK_ARG(state_slot_stride >= static_cast<int64_t>(R) * H * D);
    NQ_CHECK_ARG(ld >= static_cast<int64_t>(H) * D && ldo >= static_cast<int64_t>(H) * D && rope_theta > 0.f);
    if (D != 16 && D != 32 && D != 64) return NQ_ERR_UNSUPPORTED;
    if (window > nq::kWinMax) return NQ_ERR_UNSUPPORTED;
    if (ld % 4 || ldo % 4 || state_slot_stride % 4 ||
        ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) |
          reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(state_k) |
          reinterpret_cast<uintptr_t>(state_v) | reinterpret_cast<uintptr_t>(q_norm) |
          reinterpret_cast<uintptr_t>(k_norm)) & 15))
        return NQ_ERR_UNSUPPORTED;
    if (T == 0) return NQ_OK;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const float lt = logf(rope_theta), scale = 1.0f / sqrtf(static_cast<float>(D));
#define NQ_WIN(DD)                                                                                                \
    hipLaunchKernelGGL(nq::window_block_kernel<DD>, dim3(static_cast<unsigned>(B) * H), dim3(nq::kWinThreads), 0, \
                       st, q, k, v, ld, H, q_norm, k_norm, eps, lt, offsets, slots, frame_pos, ctx_len, state_k,    \
                       state_v, state_slot_stride, R, scale, out, ldo)
    if (D == 64) NQ_WIN(64);
    else if (D == 32) NQ_WIN(32);
    else NQ_WIN(16);
#undef NQ_WIN
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_advance(const int32_t *offsets, int B, const int32_t *slots, int64_t *frame_pos,
                                int32_t *ctx_len, int R, void *stream) {
    NQ_CHECK_ARG(offsets && slots && frame_pos && ctx_len && B > 0 && R >= 0);
    hipLaunchKernelGGL(advance_kernel, dim3((B + 63) / 64), dim3(64), 0, static_cast<hipStream_t>(stream), offsets, B,
                       slots, frame_pos, ctx_len, R);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_pcm16(const float *x, int64_t n, float *wav, int16_t *pcm, void *stream) {
    NQ_CHECK_ARG(x && n >= 0 && (wav || pcm));
    if (n == 0) return NQ_OK;
    hipLaunchKernelGGL(pcm16_kernel, dim3(grid_for(n)), dim3(kCodecThreads), 0, static_cast<hipStream_t>(stream), x, n,
                       wav, pcm);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_im2col(const float *x, int64_t ldx, int64_t T, const int32_t *offsets, int B, int u,
                               const int32_t *slots, const float *history, int Cin, int K, int dilation, int transconv,
                               const float *act_alpha, const float *act_beta, float *a, int64_t lda, void *stream) {
    NQ_CHECK_ARG(x && offsets && slots && a && B > 0 && u > 0 && T >= 0 && Cin > 0 && Cin % 4 == 0);
    NQ_CHECK_ARG(ldx % 4 == 0 && lda % 4 == 0 && ldx >= Cin);
    NQ_CHECK_ARG((act_alpha == nullptr) == (act_beta == nullptr));
    if (transconv) {
        NQ_CHECK_ARG(K == 2);
    } else {
        NQ_CHECK_ARG(K >= 1 && dilation >= 1 && (K == 1 || history));
    }
    NQ_CHECK_ARG(lda >= static_cast<int64_t>(K) * Cin);
    if (T == 0) return NQ_OK;
    hipLaunchKernelGGL(im2col_kernel, dim3(grid_for(T * K * (Cin / 4))), dim3(kCodecThreads), 0,
                       static_cast<hipStream_t>(stream), x, ldx, T, offsets, B, u, slots, history, Cin, K, dilation,
                       transconv, Act{act_alpha, act_beta}, a, lda);
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_history_update(const float *x, int64_t ldx, const int32_t *offsets, int B, int u,
                                       const int32_t *slots, float *history, int C, int pad, const float *act_alpha,
                                       const float *act_beta, void *stream) {
    NQ_CHECK_ARG(x && offsets && slots && history && B > 0 && u > 0 && C > 0 && pad > 0 && ldx >= C);
    NQ_CHECK_ARG((act_alpha == nullptr) == (act_beta == nullptr));
    if (pad * C > nq::kCodecThreads * nq::kHistoryPerThread) return NQ_ERR_UNSUPPORTED;
    hipLaunchKernelGGL(history_update_kernel, dim3(B), dim3(kCodecThreads), 0,
                       static_cast<hipStream_t>(stream), x, ldx, offsets, B, u, slots, history, C, pad,
                       Act{act_alpha, act_beta});
    return NQ_LAUNCH_STATUS();
}

extern "C" int nq_codec_transconv_overlap(const int32_t *offsets, int B, int u_in, int stride_s,
                                          const int32_t *slots, float *overlap, const float *new_overlap, int Cout,
                                          float *out, int64_t ldo, void *stream) {
    NQ_CHECK_ARG(offsets && slots && overlap && new_overlap && out && B > 0 && u_in > 0 && stride_s >= 1);
    NQ_CHECK_ARG(Cout > 0 && ldo >= Cout);
    hipLaunchKernelGGL(overlap_fixup_kernel, dim3(grid_for(static_cast<int64_t>(B) * stride_s * Cout)),
                       dim3(kCodecThreads), 0, static_cast<hipStream_t>(stream), offsets, B, u_in, stride_s, slots,
                       overlap, new_overlap, Cout, out, ldo);
    return NQ_LAUNCH_STATUS();
}
