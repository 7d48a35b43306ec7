// kernels.hip — gfx950 kernels of the mynah-asr linear-layer backend.
//
// EXACT numerics (the default). For output (m, n):
//   x row m is scaled by 2^sh_m (sh_m puts max|x_m| in [2^14, 2^15)) and split
//   into two f16 terms xh + xl (22 significant bits). Weight quants are small
//   integers, exact in f16. Per kstep (32 of K) one MFMA pair gives
//   t = sum(xh*q) + sum(xl*q) in f32; the sub-block factor is applied in f32:
//   a = fma(sc, t, a) [; a = fma(-mn, sum_x, a) for affine formats]. a restarts
//   at zero every chunk (128 of K) and total = total + a, chunk by chunk in
//   order. y = total * 2^-sh_m.
// That sequence depends on K only — never on M, on the tile a row lands in, or
// on the kernel (GEMM or GEMV) that runs it — which makes every row of the
// output bit-identical whatever the batch size.
#include "fmt.h"

#define KSTEPS 4  // ksteps per chunk

__device__ __forceinline__ f4 mfma16(half8 a, half8 b, f4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float silu_f(float v) {
    // the reference's stable sigmoid (src/qmat.h:31-35)
    if (v >= 0.0f) return v * (1.0f / (1.0f + expf(-v)));
    const float e = expf(v);
    return v * (e / (1.0f + e));
}

// A-fragment address of the prepared activations: [G][chunk][kstep][term][64][16 B]
__device__ __forceinline__ half8 load_a(const uint8_t *xp, int Kc, int G, int c, int s, int term,
                                        int lane) {
    const size_t off = (((((size_t)G * Kc + c) * KSTEPS + s) * 2 + term) * 64 + lane) * 16;
    return *(const half8 *)(xp + off);
}

// One chunk of the exact product for a WM x WN block of 16x16 tiles.
// gm[i] / gn[j]: row groups of activations / weights. acc must be zero on entry.
template <int QT, int WM, int WN>
__device__ __forceinline__ void chunk_exact(const DevW &W, int Kc, const uint8_t *xp,
                                            const float *xs16, int Kp16, const int (&gm)[WM],
                                            const int (&gn)[WN], int c, int lane,
                                            f4 (&acc)[WM][WN]) {
    using F = Fmt<QT>;
    typename F::Raw raw[WN];
#pragma unroll
    for (int j = 0; j < WN; j++) F::load(W, Kc, gn[j], c, lane, raw[j]);
    const int g = lane >> 4;
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) {
        half8 ah[WM], al[WM];
#pragma unroll
        for (int i = 0; i < WM; i++) {
            ah[i] = load_a(xp, Kc, gm[i], c, s, 0, lane);
            al[i] = load_a(xp, Kc, gm[i], c, s, 1, lane);
        }
        f4 xsum[WM][2];
        if constexpr (F::MINS) {
#pragma unroll
            for (int i = 0; i < WM; i++) {
                // sums over the kstep's 16-element halves for rows 4g..4g+3
                const int sb = 8 * c + 2 * s;
                xsum[i][0] = *(const f4 *)(xs16 + (((size_t)gm[i] * Kp16 + sb) * 16 + 4 * g));
                xsum[i][1] = *(const f4 *)(xs16 + (((size_t)gm[i] * Kp16 + sb + 1) * 16 + 4 * g));
            }
        }
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const half8 b = F::decode(raw[j], s);
            if constexpr (!F::SUB16) {
                float sc, mn;
                F::scale(raw[j], s, 0, sc, mn);
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    f4 t = mfma16(ah[i], b, f4{0.f, 0.f, 0.f, 0.f});
                    t = mfma16(al[i], b, t);
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = __builtin_fmaf(sc, t[r], acc[i][j][r]);
                    if constexpr (F::MINS) {
                        const f4 xs = xsum[i][0] + xsum[i][1];
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[i][j][r] = __builtin_fmaf(-mn, xs[r], acc[i][j][r]);
                    }
                }
            } else {
                const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
                const half8 b0 = g < 2 ? b : z, b1 = g < 2 ? z : b;
                float sc0, mn0, sc1, mn1;
                F::scale(raw[j], s, 0, sc0, mn0);
                F::scale(raw[j], s, 1, sc1, mn1);
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    f4 t0 = mfma16(ah[i], b0, f4{0.f, 0.f, 0.f, 0.f});
                    t0 = mfma16(al[i], b0, t0);
                    f4 t1 = mfma16(ah[i], b1, f4{0.f, 0.f, 0.f, 0.f});
                    t1 = mfma16(al[i], b1, t1);
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        acc[i][j][r] = __builtin_fmaf(sc0, t0[r], acc[i][j][r]);
                        acc[i][j][r] = __builtin_fmaf(sc1, t1[r], acc[i][j][r]);
                    }
                    if constexpr (F::MINS) {
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            acc[i][j][r] = __builtin_fmaf(-mn0, xsum[i][0][r], acc[i][j][r]);
                            acc[i][j][r] = __builtin_fmaf(-mn1, xsum[i][1][r], acc[i][j][r]);
                        }
                    }
                }
            }
        }
    }
}

// f32 weights: resident as (wh, wl) f16 pairs scaled per row by 2^shw_n;
// per kstep t += xh*wh + xh*wl + xl*wh, all of the chunk in one accumulator.
template <int WM, int WN>
__device__ __forceinline__ void chunk_f32(const DevW &W, int Kc, const uint8_t *xp,
                                          const int (&gm)[WM], const int (&gn)[WN], int c,
                                          int lane, f4 (&acc)[WM][WN]) {
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) {
        half8 ah[WM], al[WM], bh[WN], bl[WN];
#pragma unroll
        for (int i = 0; i < WM; i++) {
            ah[i] = load_a(xp, Kc, gm[i], c, s, 0, lane);
            al[i] = load_a(xp, Kc, gm[i], c, s, 1, lane);
        }
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const size_t base = ((size_t)gn[j] * Kc + c) * 8;
            bh[j] = *(const half8 *)(W.p0 + ((base + 2 * s) * 64 + lane) * 16);
            bl[j] = *(const half8 *)(W.p0 + ((base + 2 * s + 1) * 64 + lane) * 16);
        }
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++) {
                acc[i][j] = mfma16(ah[i], bh[j], acc[i][j]);
                acc[i][j] = mfma16(ah[i], bl[j], acc[i][j]);
                acc[i][j] = mfma16(al[i], bh[j], acc[i][j]);
            }
    }
}

template <int QT, int WM, int WN>
__device__ __forceinline__ void chunk_any(const DevW &W, int Kc, const uint8_t *xp, const float *xs16,
                                          int Kp16, const int (&gm)[WM], const int (&gn)[WN], int c,
                                          int lane, f4 (&acc)[WM][WN]) {
    if constexpr (QT == QT_F32)
        chunk_f32<WM, WN>(W, Kc, xp, gm, gn, c, lane, acc);
    else
        chunk_exact<QT, WM, WN>(W, Kc, xp, xs16, Kp16, gm, gn, c, lane, acc);
}

template <int QT>
__device__ __forceinline__ float finish(const DevW &W, float total, int sh_m, int n, int act) {
    int sh = sh_m;
    if constexpr (QT == QT_F32) sh += (int)W.h2[n];
    float v = ldexpf(total, -sh);
    if (act) v = silu_f(v);
    return v;
}

// ---------------------------------------------------------------------------
// Large-M GEMM: 4 waves in 2x2, each a WM x WN block of 16x16 tiles.
// grid.x = Np / (32*WN), grid.y = Mpad / (32*WM).
template <int QT, int WM, int WN>
__global__ __launch_bounds__(256) void k_gemm(DevW W, const uint8_t *__restrict__ xp,
                                              const float *__restrict__ xs16,
                                              const int *__restrict__ xsh, float *__restrict__ y,
                                              int M, int act) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int Kc = W.Kp / 128, Kp16 = W.Kp / 16;
    int gm[WM], gn[WN];
#pragma unroll
    for (int i = 0; i < WM; i++) gm[i] = (blockIdx.y * 2 + (wave >> 1)) * WM + i;
#pragma unroll
    for (int j = 0; j < WN; j++) gn[j] = (blockIdx.x * 2 + (wave & 1)) * WN + j;
    f4 total[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) total[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < Kc; c++) {
        f4 acc[WM][WN];
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        chunk_any<QT, WM, WN>(W, Kc, xp, xs16, Kp16, gm, gn, c, lane, acc);
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++) total[i][j] = total[i][j] + acc[i][j];
    }
    const int g = lane >> 4, col = lane & 15;
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * gm[i] + 4 * g + r;
            if (m >= M) continue;
            const int sh = xsh[m];
#pragma unroll
            for (int j = 0; j < WN; j++) {
                const int n = 16 * gn[j] + col;
                if (n < W.n) y[(size_t)m * W.n + n] = finish<QT>(W, total[i][j][r], sh, n, act);
            }
        }
}

// ---------------------------------------------------------------------------
// Small-M GEMV (M <= 16): one 16-column group per workgroup; the NW waves
// take chunks c = w, w+NW, ...; chunk partials meet in LDS and are summed in
// chunk order — the same sequence k_gemm runs in registers.
template <int QT, int NW>
__global__ __launch_bounds__(NW * 64) void k_gemv(DevW W, const uint8_t *__restrict__ xp,
                                                  const float *__restrict__ xs16,
                                                  const int *__restrict__ xsh, float *__restrict__ y,
                                                  int M, int act) {
    extern __shared__ f4 part[];  // [Kc][64]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int Kc = W.Kp / 128, Kp16 = W.Kp / 16;
    const int gm[1] = {0};
    const int gn[1] = {(int)blockIdx.x};
    for (int c = wave; c < Kc; c += NW) {
        f4 acc[1][1] = {{f4{0.f, 0.f, 0.f, 0.f}}};
        chunk_any<QT, 1, 1>(W, Kc, xp, xs16, Kp16, gm, gn, c, lane, acc);
        part[c * 64 + lane] = acc[0][0];
    }
    __syncthreads();
    if (wave != 0) return;
    f4 total = f4{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < Kc; c++) total = total + part[c * 64 + lane];
    const int g = lane >> 4, n = 16 * gn[0] + (lane & 15);
    if (n >= W.n) return;
#pragma unroll
    for (int r = 0; r < 4; r++) {
        const int m = 4 * g + r;
        if (m < M) y[(size_t)m * W.n + n] = finish<QT>(W, total[r], xsh[m], n, act);
    }
}

// ---------------------------------------------------------------------------
// Activation preparation: one workgroup per 16-row group.
//   xsh[m]  = 15 - e where max|x_m| = f * 2^e, f in [0.5, 1)  (0 for a zero row)
//   xp      = A fragments of (xh, xl), zero beyond M and K
//   xs16    = per row and 16-element sub-block: sum of the scaled x (for the
//             affine formats), (first 8 in order) + (next 8 in order)
__global__ __launch_bounds__(256) void k_prep(const float *__restrict__ x, int M, int K, int Kp,
                                              uint8_t *__restrict__ xp, float *__restrict__ xs16,
                                              int *__restrict__ xsh, int want_xsum, int vec) {
    __shared__ int shs[16];
    const int G = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // phase 1: row maxima (wave w: rows 4w .. 4w+3)
    for (int rr = 0; rr < 4; rr++) {
        const int m = 16 * G + 4 * wave + rr;
        float amax = 0.0f;
        if (m < M) {
            const float *row = x + (size_t)m * K;
            for (int j = lane; j < K; j += 64) amax = fmaxf(amax, fabsf(row[j]));
        }
        for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        if (lane == 0) {
            int e = 0;
            if (amax > 0.0f) (void)frexpf(amax, &e);
            const int sh = amax > 0.0f ? 15 - e : 0;
            shs[4 * wave + rr] = sh;
            if (m < M) xsh[m] = sh;
        }
    }
    __syncthreads();
    // phase 2: wave w writes kstep w of every chunk
    const int r = lane & 15, g = lane >> 4, m = 16 * G + r;
    const int sh = shs[r];
    const int Kc = Kp / 128;
    const float *row = x + (size_t)m * K;
    for (int c = 0; c < Kc; c++) {
        const int k0 = 128 * c + 32 * wave + 8 * g;
        float v[8];
        if (vec && m < M && k0 + 8 <= K) {
            const float4 a = *(const float4 *)(row + k0), b = *(const float4 *)(row + k0 + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = (m < M && k0 + j < K) ? row[k0 + j] : 0.0f;
        }
        half8 hi, lo;
        float s8 = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float xs = ldexpf(v[j], sh);
            const _Float16 h = (_Float16)xs;
            hi[j] = h;
            lo[j] = (_Float16)(xs - (float)h);
            s8 += xs;
        }
        const size_t off = ((((size_t)G * Kc + c) * KSTEPS + wave) * 2) * 64 * 16;
        *(half8 *)(xp + off + lane * 16) = hi;
        *(half8 *)(xp + off + (64 + lane) * 16) = lo;
        if (want_xsum) {
            const float other = __shfl_xor(s8, 16);  // lanes g and g^1 hold the two halves
            if ((g & 1) == 0) {
                const int sb = 8 * c + 2 * wave + (g >> 1);
                xs16[((size_t)G * (Kp / 16) + sb) * 16 + r] = s8 + other;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Dequantization from the resident layout: one wave per (row group, chunk).
// Values are formed exactly as the reference decoders form them.
template <int QT>
__global__ __launch_bounds__(64) void k_dequant(DevW W, float *__restrict__ out) {
    using F = Fmt<QT>;
    const int lane = threadIdx.x, c = blockIdx.x, G = blockIdx.y;
    const int Kc = W.Kp / 128;
    typename F::Raw raw;
    F::load(W, Kc, G, c, lane, raw);
    const int n = 16 * G + (lane & 15), g = lane >> 4;
    if (n >= W.n) return;
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) {
        const half8 q = F::decode(raw, s);
        float sc, mn;
        F::scale(raw, s, F::SUB16 ? (g >> 1) : 0, sc, mn);
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int k = 128 * c + 32 * s + 8 * g + j;
            if (k >= W.k) continue;
            const float qv = (float)q[j];
            float v;
            if constexpr (F::MINS) v = __fsub_rn(__fmul_rn(sc, qv), mn);
            else v = __fmul_rn(sc, qv);
            out[(size_t)n * W.k + k] = v;
        }
    }
}

__global__ void k_silu(float *__restrict__ x, size_t n) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) x[i] = silu_f(x[i]);
}

// ---------------------------------------------------------------------------
// Host-side launchers (C++ linkage inside the library).
#include "launch.h"

template <int QT>
static hipError_t launch_gemm_t(const DevW &W, const uint8_t *xp, const float *xs16, const int *xsh,
                                float *y, int M, int act, hipStream_t st) {
    const int Kc = W.Kp / 128;
    if (M <= 16 && Kc <= 64) {
        // GEMV: NW waves per column group
        if (Kc >= 16) {
            hipLaunchKernelGGL((k_gemv<QT, 16>), dim3(W.Np / 16), dim3(1024), Kc * 64 * 16, st,
                               W, xp, xs16, xsh, y, M, act);
        } else if (Kc >= 8) {
            hipLaunchKernelGGL((k_gemv<QT, 8>), dim3(W.Np / 16), dim3(512), Kc * 64 * 16, st,
                               W, xp, xs16, xsh, y, M, act);
        } else {
            hipLaunchKernelGGL((k_gemv<QT, 4>), dim3(W.Np / 16), dim3(256), Kc * 64 * 16, st,
                               W, xp, xs16, xsh, y, M, act);
        }
    } else if (M <= 512) {
        const int Mpad = (M + 31) / 32 * 32;
        hipLaunchKernelGGL((k_gemm<QT, 1, 4>), dim3(W.Np / 128, Mpad / 32), dim3(256), 0, st,
                           W, xp, xs16, xsh, y, M, act);
    } else if (M <= 2048) {
        const int Mpad = (M + 63) / 64 * 64;
        hipLaunchKernelGGL((k_gemm<QT, 2, 4>), dim3(W.Np / 128, Mpad / 64), dim3(256), 0, st,
                           W, xp, xs16, xsh, y, M, act);
    } else {
        const int Mpad = (M + 127) / 128 * 128;
        hipLaunchKernelGGL((k_gemm<QT, 4, 4>), dim3(W.Np / 128, Mpad / 128), dim3(256), 0, st,
                           W, xp, xs16, xsh, y, M, act);
    }
    return hipGetLastError();
}

hipError_t mh_launch_gemm(int qtype, const DevW &W, const uint8_t *xp, const float *xs16,
                          const int *xsh, float *y, int M, int act, hipStream_t st) {
    switch (qtype) {
    case QT_F32: return launch_gemm_t<QT_F32>(W, xp, xs16, xsh, y, M, act, st);
    case QT_INT8: return launch_gemm_t<QT_INT8>(W, xp, xs16, xsh, y, M, act, st);
    case QT_INT4: return launch_gemm_t<QT_INT4>(W, xp, xs16, xsh, y, M, act, st);
    case QT_Q4_0: return launch_gemm_t<QT_Q4_0>(W, xp, xs16, xsh, y, M, act, st);
    case QT_Q8_0: return launch_gemm_t<QT_Q8_0>(W, xp, xs16, xsh, y, M, act, st);
    case QT_Q2_K: return launch_gemm_t<QT_Q2_K>(W, xp, xs16, xsh, y, M, act, st);
    case QT_Q3_K: return launch_gemm_t<QT_Q3_K>(W, xp, xs16, xsh, y, M, act, st);
    case QT_Q4_K: return launch_gemm_t<QT_Q4_K>(W, xp, xs16, xsh, y, M, act, st);
    case QT_Q5_K: return launch_gemm_t<QT_Q5_K>(W, xp, xs16, xsh, y, M, act, st);
    case QT_Q6_K: return launch_gemm_t<QT_Q6_K>(W, xp, xs16, xsh, y, M, act, st);
    }
    return hipErrorInvalidValue;
}

hipError_t mh_launch_prep(const float *x, int M, int K, int Kp, int Mpad, uint8_t *xp, float *xs16,
                          int *xsh, int want_xsum, int vec, hipStream_t st) {
    hipLaunchKernelGGL(k_prep, dim3(Mpad / 16), dim3(256), 0, st, x, M, K, Kp, xp, xs16, xsh,
                       want_xsum, vec);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_dq(const DevW &W, float *out, hipStream_t st) {
    hipLaunchKernelGGL((k_dequant<QT>), dim3(W.Kp / 128, W.Np / 16), dim3(64), 0, st, W, out);
    return hipGetLastError();
}

hipError_t mh_launch_dequant(int qtype, const DevW &W, float *out, hipStream_t st) {
    switch (qtype) {
    case QT_INT8: return launch_dq<QT_INT8>(W, out, st);
    case QT_INT4: return launch_dq<QT_INT4>(W, out, st);
    case QT_Q4_0: return launch_dq<QT_Q4_0>(W, out, st);
    case QT_Q8_0: return launch_dq<QT_Q8_0>(W, out, st);
    case QT_Q2_K: return launch_dq<QT_Q2_K>(W, out, st);
    case QT_Q3_K: return launch_dq<QT_Q3_K>(W, out, st);
    case QT_Q4_K: return launch_dq<QT_Q4_K>(W, out, st);
    case QT_Q5_K: return launch_dq<QT_Q5_K>(W, out, st);
    case QT_Q6_K: return launch_dq<QT_Q6_K>(W, out, st);
    }
    return hipErrorInvalidValue;
}

hipError_t mh_launch_silu(float *x, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_silu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n);
    return hipGetLastError();
}
