// kernels.hip — gfx950 kernels of the mynah-asr linear-layer backend.
//
// EXACT numerics (the default). K is cut into chunks of 128. For output (m, n)
// and chunk c:
//   * x_m's chunk is scaled by 2^sh (sh puts its largest magnitude in
//     [2^14, 2^15)) and split into two f16 terms xh + xl (22 significant bits);
//   * weight quants are small integers, exact in f16; per kstep (32 of K) one
//     MFMA pair gives t = sum(xh*q) + sum(xl*q) in f32 and the sub-block
//     factor is applied in f32: a = fma(sc, t, a) [; a = fma(-mn, sum_x, a)
//     for the affine formats], a starting at zero in every chunk;
//   * total = total + a * 2^-sh, chunks in order from zero. y = total.
// Every step depends only on row m's own data and on K — never on M, on the
// tile the row lands in, or on the kernel (GEMM or GEMV) that runs it — so
// each row's bits are the same whatever the batch size.
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

// ---------------------------------------------------------------------------
// Activation split of one chunk, in the A-operand layout: lane (r = l&15,
// g = l>>4) holds elements 8g..8g+7 of each kstep for row m. The chunk's
// largest magnitude is shared by the four lanes of a row through two xor
// shuffles (every lane of the wave must call this).
struct XChunk {
    half8 h[KSTEPS], l[KSTEPS];
    float s8[KSTEPS];  // sum of the 8 scaled values, in order
    int sh;
};

__device__ __forceinline__ void split_chunk(const float *__restrict__ x, int M, int K, int m, int c,
                                            int g, int vec, XChunk &o) {
    float v[KSTEPS][8];
    const bool live = m < M;
    const float *row = x + (size_t)(live ? m : 0) * K;
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) {
        const int k0 = 128 * c + 32 * s + 8 * g;
        if (live && vec && k0 + 8 <= K) {
            const float4 a = *(const float4 *)(row + k0), b = *(const float4 *)(row + k0 + 4);
            v[s][0] = a.x; v[s][1] = a.y; v[s][2] = a.z; v[s][3] = a.w;
            v[s][4] = b.x; v[s][5] = b.y; v[s][6] = b.z; v[s][7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[s][j] = (live && k0 + j < K) ? row[k0 + j] : 0.0f;
        }
    }
    float amax = 0.0f;
#pragma unroll
    for (int s = 0; s < KSTEPS; s++)
#pragma unroll
        for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[s][j]));
    amax = fmaxf(amax, __shfl_xor(amax, 16));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    int e = 0;
    if (amax > 0.0f) (void)frexpf(amax, &e);
    o.sh = amax > 0.0f ? 15 - e : 0;
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const float xs = ldexpf(v[s][j], o.sh);
            const _Float16 h = (_Float16)xs;
            o.h[s][j] = h;
            o.l[s][j] = (_Float16)(xs - (float)h);
            acc += xs;
        }
        o.s8[s] = acc;
    }
}

// ---------------------------------------------------------------------------
// Sources of the A operand: an object with h(i, c, s, lane), l(...) (the two
// f16 terms of kstep s for row group i) and xsum(i, c, s, half, lane) (the
// sub-block sums of rows 4g..4g+3, for the affine formats).
// Prepared buffers read straight from global memory (no LDS staging):
// xp [G][chunk][kstep][term][64][16 B], xs16 [G][K/16][16 rows].
template <int WM>
struct AFromPrep {
    const uint8_t *xp;
    const float *xs16;
    int Kc, Kp16;
    const int *gm;
    __device__ __forceinline__ half8 h(int i, int c, int s, int lane) const {
        return *(const half8 *)(xp + (((((size_t)gm[i] * Kc + c) * KSTEPS + s) * 2 + 0) * 64 + lane) * 16);
    }
    __device__ __forceinline__ half8 l(int i, int c, int s, int lane) const {
        return *(const half8 *)(xp + (((((size_t)gm[i] * Kc + c) * KSTEPS + s) * 2 + 1) * 64 + lane) * 16);
    }
    __device__ __forceinline__ f4 xsum(int i, int c, int s, int hh, int lane) const {
        return *(const f4 *)(xs16 + (((size_t)gm[i] * Kp16 + 8 * c + 2 * s + hh) * 16 + 4 * (lane >> 4)));
    }
};

// Registers (small M): one row group, split in the calling wave.
struct AFromRegs {
    const XChunk *xc;
    const f4 *xs;  // [KSTEPS][2], C-layout rows
    __device__ __forceinline__ half8 h(int, int, int s, int) const { return xc->h[s]; }
    __device__ __forceinline__ half8 l(int, int, int s, int) const { return xc->l[s]; }
    __device__ __forceinline__ f4 xsum(int, int, int s, int hh, int) const { return xs[2 * s + hh]; }
};

// Raw weight registers of one chunk for WN column groups (none for F32,
// whose fragments are read per kstep).
template <int QT, int WN> struct BRaw { typename Fmt<QT>::Raw r[WN]; };
template <int WN> struct BRaw<QT_F32, WN> {};

template <int QT, int WN>
__device__ __forceinline__ void load_b(const DevW &W, int Kc, const int (&gn)[WN], int c, int lane,
                                       BRaw<QT, WN> &b) {
    if constexpr (QT != QT_F32) {
#pragma unroll
        for (int j = 0; j < WN; j++) Fmt<QT>::load(W, Kc, gn[j], c, lane, b.r[j]);
    }
}

// The exact product kstep by kstep. kstep_issue loads the A fragments,
// decodes the weights and issues the MFMAs of one kstep into a pending
// record; kstep_apply folds a pending record into the chunk accumulator
// (acc = fma(sc, t, acc) [- mn * sum_x]). Callers issue kstep s+1 before
// applying kstep s, so the VALU epilogue of one kstep runs while the matrix
// core works on the next; the float operations each output sees, and their
// order, are the same in every caller.
template <int QT, int WM, int WN> struct KPend {
    static constexpr bool SUB = QT != QT_F32 && Fmt<QT == QT_F32 ? QT_Q8_0 : QT>::SUB16;
    static constexpr bool MIN = QT != QT_F32 && Fmt<QT == QT_F32 ? QT_Q8_0 : QT>::MINS;
    static constexpr int NH = SUB ? 2 : 1;
    f4 t[WM][WN][NH];
    float sc[WN][NH], mn[WN][NH];
    f4 xs[WM][2];
};

template <int QT, int WM, int WN, class A>
__device__ __forceinline__ void kstep_issue(const DevW &W, int Kc, const A &src, const BRaw<QT, WN> &braw,
                                            const int (&gn)[WN], int c, int s, int lane,
                                            KPend<QT, WM, WN> &p, f4 (&acc)[WM][WN]) {
    half8 ah[WM], al[WM];
#pragma unroll
    for (int i = 0; i < WM; i++) {
        ah[i] = src.h(i, c, s, lane);
        al[i] = src.l(i, c, s, lane);
    }
    if constexpr (QT == QT_F32) {
        // f32 weights: resident as (wh, wl) f16 pairs scaled per row by
        // 2^shw_n; t += xh*wh + xh*wl + xl*wh straight into the chunk
        // accumulator (no per-kstep factor)
        half8 bh[WN], bl[WN];
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
    } else {
        using F = Fmt<QT>;
        const int g = lane >> 4;
        if constexpr (F::MINS) {
#pragma unroll
            for (int i = 0; i < WM; i++) {
                p.xs[i][0] = src.xsum(i, c, s, 0, lane);
                p.xs[i][1] = src.xsum(i, c, s, 1, lane);
            }
        }
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const half8 b = F::decode(braw.r[j], s);
            if constexpr (!F::SUB16) {
                F::scale(braw.r[j], s, 0, p.sc[j][0], p.mn[j][0]);
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    f4 t = mfma16(ah[i], b, f4{0.f, 0.f, 0.f, 0.f});
                    p.t[i][j][0] = mfma16(al[i], b, t);
                }
            } else {
                const half8 z = {0, 0, 0, 0, 0, 0, 0, 0};
                const half8 b0 = g < 2 ? b : z, b1 = g < 2 ? z : b;
                F::scale(braw.r[j], s, 0, p.sc[j][0], p.mn[j][0]);
                F::scale(braw.r[j], s, 1, p.sc[j][1], p.mn[j][1]);
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    f4 t0 = mfma16(ah[i], b0, f4{0.f, 0.f, 0.f, 0.f});
                    p.t[i][j][0] = mfma16(al[i], b0, t0);
                    f4 t1 = mfma16(ah[i], b1, f4{0.f, 0.f, 0.f, 0.f});
                    p.t[i][j][1] = mfma16(al[i], b1, t1);
                }
            }
        }
    }
}

template <int QT, int WM, int WN>
__device__ __forceinline__ void kstep_apply(const KPend<QT, WM, WN> &p, f4 (&acc)[WM][WN]) {
    if constexpr (QT != QT_F32) {
        using KP = KPend<QT, WM, WN>;
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++) {
                if constexpr (!KP::SUB) {
#pragma unroll
                    for (int r = 0; r < 4; r++) acc[i][j][r] = __builtin_fmaf(p.sc[j][0], p.t[i][j][0][r], acc[i][j][r]);
                    if constexpr (KP::MIN) {
                        const f4 xs = p.xs[i][0] + p.xs[i][1];
#pragma unroll
                        for (int r = 0; r < 4; r++) acc[i][j][r] = __builtin_fmaf(-p.mn[j][0], xs[r], acc[i][j][r]);
                    }
                } else {
#pragma unroll
                    for (int r = 0; r < 4; r++) {
                        acc[i][j][r] = __builtin_fmaf(p.sc[j][0], p.t[i][j][0][r], acc[i][j][r]);
                        acc[i][j][r] = __builtin_fmaf(p.sc[j][1], p.t[i][j][1][r], acc[i][j][r]);
                    }
                    if constexpr (KP::MIN) {
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            acc[i][j][r] = __builtin_fmaf(-p.mn[j][0], p.xs[i][0][r], acc[i][j][r]);
                            acc[i][j][r] = __builtin_fmaf(-p.mn[j][1], p.xs[i][1][r], acc[i][j][r]);
                        }
                    }
                }
            }
    }
}

template <int QT, int WM, int WN>
constexpr int kstep_mfmas() {
    return QT == QT_F32 ? 3 * WM * WN : (KPend<QT, WM, WN>::SUB ? 4 : 2) * WM * WN;
}

// A whole chunk from one A source. PIPE: issue(s+1) before apply(s) (more
// registers, more overlap); otherwise each kstep is applied right away.
template <int QT, int WM, int WN, class A, bool PIPE = true>
__device__ __forceinline__ void chunk_all(const DevW &W, int Kc, const A &src, const BRaw<QT, WN> &braw,
                                          const int (&gn)[WN], int c, int lane, f4 (&acc)[WM][WN]) {
    if constexpr (!PIPE) {
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            KPend<QT, WM, WN> p;
            kstep_issue<QT, WM, WN>(W, Kc, src, braw, gn, c, s, lane, p, acc);
            kstep_apply<QT, WM, WN>(p, acc);
        }
        return;
    }
    KPend<QT, WM, WN> p0, p1;
    kstep_issue<QT, WM, WN>(W, Kc, src, braw, gn, c, 0, lane, p0, acc);
    kstep_issue<QT, WM, WN>(W, Kc, src, braw, gn, c, 1, lane, p1, acc);
    kstep_apply<QT, WM, WN>(p0, acc);
    kstep_issue<QT, WM, WN>(W, Kc, src, braw, gn, c, 2, lane, p0, acc);
    kstep_apply<QT, WM, WN>(p1, acc);
    kstep_issue<QT, WM, WN>(W, Kc, src, braw, gn, c, 3, lane, p1, acc);
    kstep_apply<QT, WM, WN>(p0, acc);
    kstep_apply<QT, WM, WN>(p1, acc);
}

// the per-row weight shift of the f32 format (0 for the quantized ones)
template <int QT>
__device__ __forceinline__ int wshift(const DevW &W, int n) {
    if constexpr (QT == QT_F32) return (int)W.h2[n];
    return 0;
}

// ---------------------------------------------------------------------------
// Large-M GEMM: 4 waves in 2x2, each a WM x WN block of 16x16 tiles; every
// wave reads its A and B fragments straight from global memory in the
// MFMA-native layouts (one contiguous 1 KiB block per wave-wide 16-byte load),
// and L1/L2 serve the sharing between the waves of a workgroup. Staging A
// through LDS was measured slower on gfx950 for these tiles: the kernel is
// bound by the VALU work of the per-kstep f32 epilogue, and the extra LDS
// traffic, barriers and prefetch registers only add to it.
// grid = tilesM * tilesN workgroups, tiles of (32*WM) x (32*WN).
template <int QT, int WM, int WN, bool PIPE>
__global__ __launch_bounds__(256) void k_gemm_direct(DevW W, const uint8_t *__restrict__ xp,
                                                     const float *__restrict__ xs16,
                                                     const int *__restrict__ xsh, float *__restrict__ y,
                                                     int M, int act, int tilesM, int tilesN) {
    // XCD-aware tile order: workgroups are dealt to the 8 XCDs round-robin
    // (bid % 8), each XCD with its own L2. Give every XCD a contiguous run of
    // tiles in row-band-major order, so that the N tiles of a row band — which
    // all read the same activations, the largest operand — share one L2
    // instead of fetching the band from HBM once per XCD.
    const int ntiles = tilesM * tilesN, bid = blockIdx.x;
    const int q = ntiles / 8, rem = ntiles % 8, xcd = bid % 8, loc = bid / 8;
    const int t = xcd < rem ? xcd * (q + 1) + loc : rem * (q + 1) + (xcd - rem) * q + loc;
    const int tm = t / tilesN, tn = t % tilesN;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int Kc = W.Kp / 128, Kp16 = W.Kp / 16;
    int gm[WM], gn[WN], shw[WN];
#pragma unroll
    for (int i = 0; i < WM; i++) gm[i] = (tm * 2 + (wave >> 1)) * WM + i;
#pragma unroll
    for (int j = 0; j < WN; j++) {
        gn[j] = (tn * 2 + (wave & 1)) * WN + j;
        shw[j] = wshift<QT>(W, 16 * gn[j] + col);
    }
    const AFromPrep<WM> src{xp, xs16, Kc, Kp16, gm};
    f4 total[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) total[i][j] = f4{0.f, 0.f, 0.f, 0.f};
    for (int c = 0; c < Kc; c++) {
        BRaw<QT, WN> braw;
        load_b<QT, WN>(W, Kc, gn, c, lane, braw);
        int4 sh4[WM];  // issued now, used after the chunk
#pragma unroll
        for (int i = 0; i < WM; i++) sh4[i] = *(const int4 *)(xsh + ((size_t)gm[i] * Kc + c) * 16 + 4 * g);
        f4 acc[WM][WN];
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++) acc[i][j] = f4{0.f, 0.f, 0.f, 0.f};
        chunk_all<QT, WM, WN, AFromPrep<WM>, PIPE>(W, Kc, src, braw, gn, c, lane, acc);
#pragma unroll
        for (int i = 0; i < WM; i++) {
            const int sh[4] = {sh4[i].x, sh4[i].y, sh4[i].z, sh4[i].w};
#pragma unroll
            for (int r = 0; r < 4; r++)
#pragma unroll
                for (int j = 0; j < WN; j++)
                    total[i][j][r] = total[i][j][r] + ldexpf(acc[i][j][r], -(sh[r] + shw[j]));
        }
    }
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * gm[i] + 4 * g + r;
            if (m >= M) continue;
#pragma unroll
            for (int j = 0; j < WN; j++) {
                const int n = 16 * gn[j] + col;
                if (n < W.n) y[(size_t)m * W.n + n] = act ? silu_f(total[i][j][r]) : total[i][j][r];
            }
        }
}

// ---------------------------------------------------------------------------
// Small-M GEMV (M <= 16), no preparation pass: each wave splits its chunks of
// x in registers (split_chunk, the same function k_prep runs) and applies
// them to WNG 16-column groups; the NW waves of a workgroup take chunks
// c = w, w+NW, ...; the scaled chunk partials meet in LDS and are summed in
// chunk order from zero — the sequence k_gemm runs in registers.
template <int QT, int NW, int WNG>
__global__ __launch_bounds__(NW * 64) void k_gemv(DevW W, const float *__restrict__ x, int M, int vec,
                                                  float *__restrict__ y, int act) {
    extern __shared__ f4 part[];  // [Kc][WNG][64]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int Kc = W.Kp / 128;
    int gn[WNG], shw[WNG];
#pragma unroll
    for (int j = 0; j < WNG; j++) {
        gn[j] = blockIdx.x * WNG + j;
        shw[j] = wshift<QT>(W, 16 * gn[j] + col);
    }
    for (int c = wave; c < Kc; c += NW) {
        XChunk xc;
        split_chunk(x, M, W.k, col, c, g, vec, xc);  // (weight loads issue below; the
                                                     // compiler hoists them past the split)
        // C layout: lane holds rows 4g+i; fetch their shifts and sub-block sums
        int shc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) shc[i] = __shfl(xc.sh, 4 * g + i);
        f4 xs[2 * KSTEPS];
        if constexpr (Fmt<QT == QT_F32 ? QT_Q8_0 : QT>::MINS) {
#pragma unroll
            for (int s = 0; s < KSTEPS; s++) {
                const float s16 = xc.s8[s] + __shfl_xor(xc.s8[s], 16);
#pragma unroll
                for (int hh = 0; hh < 2; hh++)
#pragma unroll
                    for (int i = 0; i < 4; i++) xs[2 * s + hh][i] = __shfl(s16, 4 * g + i + 32 * hh);
            }
        }
        const AFromRegs src{&xc, xs};
        f4 acc[1][WNG];
#pragma unroll
        for (int j = 0; j < WNG; j++) acc[0][j] = f4{0.f, 0.f, 0.f, 0.f};
        BRaw<QT, WNG> braw;
        load_b<QT, WNG>(W, Kc, gn, c, lane, braw);
        chunk_all<QT, 1, WNG>(W, Kc, src, braw, gn, c, lane, acc);
#pragma unroll
        for (int j = 0; j < WNG; j++) {
            f4 v;
#pragma unroll
            for (int i = 0; i < 4; i++) v[i] = ldexpf(acc[0][j][i], -(shc[i] + shw[j]));
            part[(c * WNG + j) * 64 + lane] = v;
        }
    }
    __syncthreads();
    for (int j = wave; j < WNG; j += NW) {
        f4 total = f4{0.f, 0.f, 0.f, 0.f};
        for (int c = 0; c < Kc; c++) total = total + part[(c * WNG + j) * 64 + lane];
        const int n = 16 * gn[j] + col;
        if (n >= W.n) continue;
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = 4 * g + i;
            if (m < M) y[(size_t)m * W.n + n] = act ? silu_f(total[i]) : total[i];
        }
    }
}

// ---------------------------------------------------------------------------
// Activation preparation for k_gemm: one workgroup (4 waves) per 16-row
// group; wave w splits chunks c = w, w+4, ... with split_chunk and stores
//   xp   A fragments of (xh, xl), zero beyond M and K
//   xs16 per row and 16-element sub-block: (first 8 in order) + (next 8)
//   xsh  per row group, chunk and row: the shift  [G][chunk][16]
__global__ __launch_bounds__(256) void k_prep(const float *__restrict__ x, int M, int K, int Kp,
                                              uint8_t *__restrict__ xp, float *__restrict__ xs16,
                                              int *__restrict__ xsh, int want_xsum, int vec) {
    const int G = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 15, g = lane >> 4, m = 16 * G + r;
    const int Kc = Kp / 128;
    for (int c = wave; c < Kc; c += 4) {
        XChunk xc;
        split_chunk(x, M, K, m, c, g, vec, xc);
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            const size_t off = ((((size_t)G * Kc + c) * KSTEPS + s) * 2) * 64 * 16;
            *(half8 *)(xp + off + lane * 16) = xc.h[s];
            *(half8 *)(xp + off + (64 + lane) * 16) = xc.l[s];
            if (want_xsum) {
                const float s16 = xc.s8[s] + __shfl_xor(xc.s8[s], 16);
                if ((g & 1) == 0) xs16[((size_t)G * (Kp / 16) + 8 * c + 2 * s + (g >> 1)) * 16 + r] = s16;
            }
        }
        if (g == 0) xsh[((size_t)G * Kc + c) * 16 + r] = xc.sh;
    }
}

// ---------------------------------------------------------------------------
// INT8ACT numerics: the reference's small-T int8 path (src/qmat.c:508-552),
// for every M. Activations are quantized per row exactly as
// quantize_act_int8 (qmat.c:186-202); v_mfma_i32_16x16x64_i8 forms the exact
// integer sums; the f32 combine follows the reference's order:
//   INT8   y = ((float)s * ws) * sx           (s over the whole row)
//   INT4   acc = acc + (float)ig * sg per group of 32, in order; y = acc * sx
//   Q8_0/Q4_0  the same with the block factor d (the oracle's block semantics)
// Int8 activation layout: [row group][kstep pair][64][16 B]; each lane's 16
// bytes are kstep 2p then 2p+1, each as dwords {e0,e4,e1,e5} {e2,e6,e3,e7} of
// elements 8g..8g+7 — the byte order of the weight planes, so weight bytes
// (or nibbles expanded with two masks) feed the MFMA unchanged.
typedef int i4v __attribute__((ext_vector_type(4)));

__device__ __forceinline__ i4v mfma_i8(i4v a, i4v b, i4v c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int act_q8(float v, float inv) {
    const float t = __fmul_rn(v, inv);
    int q = (int)(t >= 0.0f ? __fadd_rn(t, 0.5f) : __fsub_rn(t, 0.5f));
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// one workgroup (4 waves) per 16-row group
__global__ __launch_bounds__(256) void k_prep_i8(const float *__restrict__ x, int M, int K, int Kp,
                                                 uint8_t *__restrict__ qx, float *__restrict__ sx,
                                                 int *__restrict__ gsum) {
    __shared__ float invs[16];
    const int G = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int rr = 0; rr < 4; rr++) {
        const int m = 16 * G + 4 * wave + rr;
        float amax = 0.0f;
        if (m < M) {
            const float *row = x + (size_t)m * K;
            for (int j = lane; j < K; j += 64) amax = fmaxf(amax, fabsf(row[j]));
        }
        for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        if (lane == 0) {
            invs[4 * wave + rr] = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
            sx[m] = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 0.0f;
        }
    }
    __syncthreads();
    const int r = lane & 15, g = lane >> 4, m = 16 * G + r;
    const float inv = invs[r];
    const bool live = m < M && inv > 0.0f;
    const float *row = x + (size_t)(m < M ? m : 0) * K;
    const int P = Kp / 64;
    static const int kWord[8] = {0, 0, 1, 1, 0, 0, 1, 1};
    static const int kByte[8] = {0, 2, 0, 2, 1, 3, 1, 3};
    for (int p = wave; p < P; p += 4) {
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int k0 = 64 * p + 32 * h + 8 * g;
            int gs = 0;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int q = (live && k0 + j < K) ? act_q8(row[k0 + j], inv) : 0;
                gs += q;
                w[2 * h + kWord[j]] |= ((uint32_t)q & 0xffu) << (8 * kByte[j]);
            }
            gs += __shfl_xor(gs, 16);
            gs += __shfl_xor(gs, 32);
            if (g == 0) gsum[((size_t)G * (Kp / 32) + 2 * p + h) * 16 + r] = gs;
        }
        *(uint4 *)(qx + (((size_t)G * P + p) * 64 + lane) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// 4 waves per workgroup, one 16-column group each, WM row groups per wave.
template <int QT, int WM>
__global__ __launch_bounds__(256) void k_gemm_i8(DevW W, const uint8_t *__restrict__ qx,
                                                 const float *__restrict__ sx, const int *__restrict__ gsum,
                                                 float *__restrict__ y, int M, int act) {
    constexpr bool NIB = QT == QT_INT4 || QT == QT_Q4_0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int g = lane >> 4, col = lane & 15;
    const int G = blockIdx.x * 4 + wave;       // weight row group
    const int Kc = W.Kp / 128, P = W.Kp / 64;
    int gm[WM];
#pragma unroll
    for (int i = 0; i < WM; i++) gm[i] = blockIdx.y * WM + i;
    i4v si[WM];
    f4 acc[WM];
#pragma unroll
    for (int i = 0; i < WM; i++) {
        si[i] = i4v{0, 0, 0, 0};
        acc[i] = f4{0.f, 0.f, 0.f, 0.f};
    }
    for (int p = 0; p < P; p++) {
        const int c = p >> 1, q = p & 1;
        uint32_t b[4];
        if constexpr (NIB) {
            const uint2 v = *(const uint2 *)(W.p0 + (((size_t)G * Kc + c) * 64 + lane) * 16 + 8 * q);
            b[0] = v.x & 0x0F0F0F0Fu;
            b[1] = (v.x >> 4) & 0x0F0F0F0Fu;
            b[2] = v.y & 0x0F0F0F0Fu;
            b[3] = (v.y >> 4) & 0x0F0F0F0Fu;
        } else {
            const uint4 v = *(const uint4 *)(W.p0 + ((((size_t)G * Kc + c) * 2 + q) * 64 + lane) * 16);
            b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
        }
        float d0 = 0.f, d1 = 0.f;
        if constexpr (QT == QT_Q8_0 || QT == QT_Q4_0) {
            const uint32_t hd = *(const uint32_t *)(W.h + (((size_t)G * Kc + c) * 16 + col) * 8 + 4 * q);
            d0 = h2f(hd & 0xffff);
            d1 = h2f(hd >> 16);
        } else if constexpr (QT == QT_INT4) {
            const float2 v = *(const float2 *)(W.h2 + (((size_t)G * Kc + c) * 16 + col) * 4 + 2 * q);
            d0 = v.x;
            d1 = v.y;
        }
        const i4v bb = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
        const i4v blo = {(int)b[0], (int)b[1], 0, 0}, bhi = {0, 0, (int)b[2], (int)b[3]};
#pragma unroll
        for (int i = 0; i < WM; i++) {
            const i4v a = *(const i4v *)(qx + (((size_t)gm[i] * P + p) * 64 + lane) * 16);
            if constexpr (QT == QT_INT8) {
                si[i] = mfma_i8(a, bb, si[i]);
            } else {
                i4v t0 = mfma_i8(a, blo, i4v{0, 0, 0, 0});
                i4v t1 = mfma_i8(a, bhi, i4v{0, 0, 0, 0});
                if constexpr (NIB) {  // sum (n - 8) * q = sum n * q - 8 * sum q
                    const int4 g0 = *(const int4 *)(gsum + ((size_t)gm[i] * (W.Kp / 32) + 2 * p) * 16 + 4 * g);
                    const int4 g1 = *(const int4 *)(gsum + ((size_t)gm[i] * (W.Kp / 32) + 2 * p + 1) * 16 + 4 * g);
                    t0 -= 8 * i4v{g0.x, g0.y, g0.z, g0.w};
                    t1 -= 8 * i4v{g1.x, g1.y, g1.z, g1.w};
                }
#pragma unroll
                for (int r = 0; r < 4; r++) {
                    acc[i][r] = __fadd_rn(acc[i][r], __fmul_rn((float)t0[r], d0));
                    acc[i][r] = __fadd_rn(acc[i][r], __fmul_rn((float)t1[r], d1));
                }
            }
        }
    }
    const int n = 16 * G + col;
    if (n >= W.n) return;
    const float ws = QT == QT_INT8 ? W.h2[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * gm[i] + 4 * g + r;
            if (m >= M) continue;
            float v;
            if constexpr (QT == QT_INT8) v = __fmul_rn(__fmul_rn((float)si[i][r], ws), sx[m]);
            else v = __fmul_rn(acc[i][r], sx[m]);
            y[(size_t)m * W.n + n] = act ? silu_f(v) : v;
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
#include <stdlib.h>

#include "launch.h"

template <int QT, int NW, int WNG>
static hipError_t launch_gemv(const DevW &W, const float *x, int M, int vec, float *y, int act,
                              hipStream_t st) {
    const int Kc = W.Kp / 128;
    hipLaunchKernelGGL((k_gemv<QT, NW, WNG>), dim3(W.Np / 16 / WNG), dim3(NW * 64),
                       (size_t)Kc * WNG * 64 * 16, st, W, x, M, vec, y, act);
    return hipGetLastError();
}

// column groups per GEMV workgroup: more for wide outputs, so that each chunk
// of x is split once for several groups
static int gemv_wng(const DevW &W) {
    const int Kc = W.Kp / 128, groups = W.Np / 16;
    if (groups >= 1024 && Kc <= 16) return 4;
    if (groups >= 256 && Kc <= 32) return 2;
    return 1;
}

template <int QT>
static hipError_t gemv_t(const DevW &W, const float *x, int M, int vec, float *y, int act,
                         hipStream_t st) {
    const int Kc = W.Kp / 128, wng = gemv_wng(W);
    if (wng == 4) {
        if (Kc >= 8) return launch_gemv<QT, 8, 4>(W, x, M, vec, y, act, st);
        return launch_gemv<QT, 4, 4>(W, x, M, vec, y, act, st);
    }
    if (wng == 2) {
        if (Kc >= 16) return launch_gemv<QT, 16, 2>(W, x, M, vec, y, act, st);
        if (Kc >= 8) return launch_gemv<QT, 8, 2>(W, x, M, vec, y, act, st);
        return launch_gemv<QT, 4, 2>(W, x, M, vec, y, act, st);
    }
    if (Kc >= 16) return launch_gemv<QT, 16, 1>(W, x, M, vec, y, act, st);
    if (Kc >= 8) return launch_gemv<QT, 8, 1>(W, x, M, vec, y, act, st);
    return launch_gemv<QT, 4, 1>(W, x, M, vec, y, act, st);
}

template <int QT, int WM>
static hipError_t launch_direct(const DevW &W, const uint8_t *xp, const float *xs16, const int *xsh, float *y,
                                int M, int act, hipStream_t st) {
    const int tilesM = mh_mpad(M) / (32 * WM), tilesN = W.Np / 128;
    hipLaunchKernelGGL((k_gemm_direct<QT, WM, 4, false>), dim3(tilesM * tilesN), dim3(256), 0, st,
                       W, xp, xs16, xsh, y, M, act, tilesM, tilesN);
    return hipGetLastError();
}

// Rows per wave (WM): 2 for the block-scaled formats at large M, 1 for small
// M and for the K-quants, whose decoders need the registers (measured best on
// the BASELINE shapes). MYNAH_ASR_HIP_GEMM_WM=1|2 overrides, for tuning.
int mh_gemm_wm(int M, bool kquant) {
    static int forced = -2;
    if (forced == -2) {
        const char *e = getenv("MYNAH_ASR_HIP_GEMM_WM");
        forced = e ? atoi(e) : -1;
    }
    if (forced == 1 || forced == 2) return forced;
    return (kquant || M <= 1024) ? 1 : 2;
}

template <int QT>
static hipError_t gemm_t(const DevW &W, const uint8_t *xp, const float *xs16, const int *xsh, float *y,
                         int M, int act, hipStream_t st) {
    constexpr bool kq = QT == QT_Q2_K || QT == QT_Q3_K || QT == QT_Q4_K || QT == QT_Q5_K || QT == QT_Q6_K;
    if (mh_gemm_wm(M, kq) == 2) return launch_direct<QT, 2>(W, xp, xs16, xsh, y, M, act, st);
    return launch_direct<QT, 1>(W, xp, xs16, xsh, y, M, act, st);
}

#define MH_DISPATCH(fn, qtype, ...)                                  \
    switch (qtype) {                                                 \
    case QT_F32: return fn<QT_F32>(__VA_ARGS__);                     \
    case QT_INT8: return fn<QT_INT8>(__VA_ARGS__);                   \
    case QT_INT4: return fn<QT_INT4>(__VA_ARGS__);                   \
    case QT_Q4_0: return fn<QT_Q4_0>(__VA_ARGS__);                   \
    case QT_Q8_0: return fn<QT_Q8_0>(__VA_ARGS__);                   \
    case QT_Q2_K: return fn<QT_Q2_K>(__VA_ARGS__);                   \
    case QT_Q3_K: return fn<QT_Q3_K>(__VA_ARGS__);                   \
    case QT_Q4_K: return fn<QT_Q4_K>(__VA_ARGS__);                   \
    case QT_Q5_K: return fn<QT_Q5_K>(__VA_ARGS__);                   \
    case QT_Q6_K: return fn<QT_Q6_K>(__VA_ARGS__);                   \
    }                                                                \
    return hipErrorInvalidValue;

bool mh_use_gemv(const DevW &W, int M) { return M <= 16 && (W.Kp / 128) * gemv_wng(W) <= 64; }

hipError_t mh_launch_gemv(int qtype, const DevW &W, const float *x, int M, int vec, float *y, int act,
                          hipStream_t st) {
    MH_DISPATCH(gemv_t, qtype, W, x, M, vec, y, act, st)
}

hipError_t mh_launch_gemm(int qtype, const DevW &W, const uint8_t *xp, const float *xs16,
                          const int *xsh, float *y, int M, int act, hipStream_t st) {
    MH_DISPATCH(gemm_t, qtype, W, xp, xs16, xsh, y, M, act, st)
}

hipError_t mh_launch_prep(const float *x, int M, int K, int Kp, int Mpad, uint8_t *xp, float *xs16,
                          int *xsh, int want_xsum, int vec, hipStream_t st) {
    hipLaunchKernelGGL(k_prep, dim3(Mpad / 16), dim3(256), 0, st, x, M, K, Kp, xp, xs16, xsh,
                       want_xsum, vec);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_dq(const DevW &W, float *out, hipStream_t st) {
    if constexpr (QT == QT_F32) {
        return hipErrorInvalidValue;
    } else {
        hipLaunchKernelGGL((k_dequant<QT>), dim3(W.Kp / 128, W.Np / 16), dim3(64), 0, st, W, out);
        return hipGetLastError();
    }
}

hipError_t mh_launch_dequant(int qtype, const DevW &W, float *out, hipStream_t st) {
    MH_DISPATCH(launch_dq, qtype, W, out, st)
}

bool mh_i8_supported(int qtype) {
    return qtype == QT_INT8 || qtype == QT_INT4 || qtype == QT_Q8_0 || qtype == QT_Q4_0;
}

hipError_t mh_launch_prep_i8(const float *x, int M, int K, int Kp, int Mpad, uint8_t *qx, float *sx,
                             int *gsum, hipStream_t st) {
    hipLaunchKernelGGL(k_prep_i8, dim3(Mpad / 16), dim3(256), 0, st, x, M, K, Kp, qx, sx, gsum);
    return hipGetLastError();
}

template <int QT, int WM>
static hipError_t launch_i8(const DevW &W, const uint8_t *qx, const float *sx, const int *gsum, float *y,
                            int M, int act, hipStream_t st) {
    hipLaunchKernelGGL((k_gemm_i8<QT, WM>), dim3(W.Np / 64, mh_mpad(M) / (16 * WM)), dim3(256), 0, st,
                       W, qx, sx, gsum, y, M, act);
    return hipGetLastError();
}

template <int QT>
static hipError_t gemm_i8_t(const DevW &W, const uint8_t *qx, const float *sx, const int *gsum, float *y,
                            int M, int act, hipStream_t st) {
    if (M <= 64) return launch_i8<QT, 1>(W, qx, sx, gsum, y, M, act, st);
    return launch_i8<QT, 2>(W, qx, sx, gsum, y, M, act, st);
}

hipError_t mh_launch_gemm_i8(int qtype, const DevW &W, const uint8_t *qx, const float *sx, const int *gsum,
                             float *y, int M, int act, hipStream_t st) {
    switch (qtype) {
    case QT_INT8: return gemm_i8_t<QT_INT8>(W, qx, sx, gsum, y, M, act, st);
    case QT_INT4: return gemm_i8_t<QT_INT4>(W, qx, sx, gsum, y, M, act, st);
    case QT_Q8_0: return gemm_i8_t<QT_Q8_0>(W, qx, sx, gsum, y, M, act, st);
    case QT_Q4_0: return gemm_i8_t<QT_Q4_0>(W, qx, sx, gsum, y, M, act, st);
    }
    return hipErrorInvalidValue;
}

hipError_t mh_launch_silu(float *x, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_silu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n);
    return hipGetLastError();
}
