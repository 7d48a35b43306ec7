// kernels.hip — gfx950 kernels of the mynah-asr linear-layer backend.
//
// EXACT numerics (the default). K is cut into chunks of 128. For output (m, n)
// and chunk c:
//   * x_m's chunk is scaled by 2^sh (sh puts its largest magnitude in
//     [2^14, 2^15)) and split into two f16 terms xh + xl (22 significant bits);
//   * weight quants are small integers, exact in f16; per kstep (32 of K) four
//     v_mfma_f32_32x32x16_f16 give t = sum(xh*q) + sum(xl*q) in f32 and the
//     sub-block factor is applied in f32: a = fma(sc, t, a) [; a = fma(-mn,
//     sum_x, a) for the affine formats], a starting at zero in every chunk;
//   * total = fma(2^-sh, a, total), chunks in order from zero. y = total.
// Q2_K, Q3_K, Q4_K and Q5_K fold their integer sub-block factors f into the
// decoded quants (q*f, exact in f16): a = the chunk's MFMAs straight through,
// then a = d*a - 32*dmin*(mins MFMA over the rows' split sub-block sums).
// Every step depends only on row m's own data and on K — never on M, on the
// tile the row lands in, or on the kernel (GEMM or GEMV) that runs it — so
// each row's bits are the same whatever the batch size.
//
// The 32x32x16 MFMA is used throughout: on gfx950 it issues twice the work of
// the 16x16x32 shape per cycle (measured 2.04 vs 1.19 PFLOP/s f16).
#include "fmt.h"
#include "launch.h"

#define KSTEPS 4  // ksteps per chunk
#define HSTEPS 8  // half-steps per chunk

__device__ __forceinline__ f16v mfma32(half8 a, half8 b, f16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f16v zero16() {
    f16v z;
#pragma unroll
    for (int e = 0; e < 16; e++) z[e] = 0.0f;
    return z;
}

// D-layout row of accumulator element e for lane half hh
__device__ __forceinline__ int drow(int e, int hh) { return 8 * (e >> 2) + 4 * hh + (e & 3); }

__device__ __forceinline__ float silu_f(float v) {
    // x * sigmoid(x) with the reference's stable sigmoid (src/qmat.h:31-35):
    // exp only of -|x| (never overflows); 1/(1+e) for x >= 0, e/(1+e) below.
    // Hardware exp2 and reciprocal (~1 ulp each), like the reference's own
    // -ffast-math build; every kernel applies this same function.
    const float e = __expf(-fabsf(v));
    const float r = __builtin_amdgcn_rcpf(1.0f + e);
    return v * (v >= 0.0f ? r : e * r);
}

// ---------------------------------------------------------------------------
// Activation split of one chunk, in the A-operand layout: lane (r = l&31,
// hh = l>>5) holds elements 16u + 8hh .. +7 of half-step u for row m. The
// chunk's largest magnitude is shared by the two lanes of a row through one
// xor shuffle (every lane of the wave must call this).
struct XChunk {
    half8 h[HSTEPS], l[HSTEPS];
    float s8[HSTEPS];  // sum of the lane's 8 scaled values of half-step u, in order
    float p;           // 2^-sh: the chunk's fold factor for this row
};

// f16(x0 - h.lo), f16(x1 - h.hi) as one packed pair: x - h is exact in f32
// (h is x rounded to f16), and v_fma_mixlo / v_fma_mixhi form it with h read as f16 in place
// and rounds it to f16 once: the value of (_Float16)(x - (float)h), in two
// instructions per pair instead of six.
__device__ __forceinline__ uint32_t lo_pair(uint32_t hpair, float x0, float x1) {
    uint32_t r;
    asm volatile("v_fma_mixlo_f16 %0, %1, -1.0, %2 op_sel_hi:[1,0,0]" : "=v"(r) : "v"(hpair), "v"(x0));
    asm volatile("v_fma_mixhi_f16 %0, %1, -1.0, %2 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
                 : "+v"(r)
                 : "v"(hpair), "v"(x1));
    return r;
}

// the split of NU half-steps' values v[u][j] with shift sh
template <int NU>
__device__ __forceinline__ void split_part(const float (&v)[NU][8], int sh, half8 (&h)[NU], half8 (&l)[NU],
                                           float (&s8)[NU]) {
#pragma unroll
    for (int u = 0; u < NU; u++) {
        float acc = 0.0f;
        float xs[8];
#pragma unroll
        for (int j = 0; j < 8; j++) {
            xs[j] = ldexpf(v[u][j], sh);
            h[u][j] = (_Float16)xs[j];
            acc += xs[j];
        }
        s8[u] = acc;
        uint32_t hw[4], lw[4];
        __builtin_memcpy(hw, &h[u], 16);
#pragma unroll
        for (int t = 0; t < 4; t++) lw[t] = lo_pair(hw[t], xs[2 * t], xs[2 * t + 1]);
        __builtin_memcpy(&l[u], lw, 16);
    }
}

// the split of one chunk's values v[u][j] (element 16u + 8hh + j of row m)
__device__ __forceinline__ void split_vals(const float (&v)[HSTEPS][8], XChunk &o) {
    float amax = 0.0f;
#pragma unroll
    for (int u = 0; u < HSTEPS; u++)
#pragma unroll
        for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[u][j]));
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const int sh = chunk_shift(amax);
    o.p = ldexpf(1.0f, -sh);
    split_part<HSTEPS>(v, sh, o.h, o.l, o.s8);
}

// VEC: K % 8 == 0 and 16-byte aligned rows (each lane's 8 elements are
// wholly inside or wholly past K), two float4 loads per half-step
template <bool VEC>
__device__ __forceinline__ void load_chunk(const float *__restrict__ x, int M, int K, int m, int c, int hh,
                                           float (&v)[HSTEPS][8]) {
    const bool live = m < M;
    const float *row = x + (size_t)(live ? m : 0) * K;
#pragma unroll
    for (int u = 0; u < HSTEPS; u++) {
        const int k0 = 128 * c + 16 * u + 8 * hh;
        if constexpr (VEC) {
            float4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
            if (live && k0 < K) {
                a = *(const float4 *)(row + k0);
                b = *(const float4 *)(row + k0 + 4);
            }
            v[u][0] = a.x; v[u][1] = a.y; v[u][2] = a.z; v[u][3] = a.w;
            v[u][4] = b.x; v[u][5] = b.y; v[u][6] = b.z; v[u][7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[u][j] = (live && k0 + j < K) ? row[k0 + j] : 0.0f;
        }
    }
}

template <bool VEC>
__device__ __forceinline__ void split_chunk(const float *__restrict__ x, int M, int K, int m, int c, int hh,
                                            XChunk &o) {
    float v[HSTEPS][8];
    load_chunk<VEC>(x, M, K, m, c, hh, v);
    split_vals(v, o);
}

// ---------------------------------------------------------------------------
// Weight fragments of WN column groups: per-chunk headers and per-kstep words.
// Formats whose integer sub-block factors fold into the decoded weights (the
// FHdr traits): a chunk's MFMAs then accumulate straight through its four
// ksteps, and the factors d (and the mins, through one more MFMA) apply once
// per chunk instead of once per sub-block
template <int QT> constexpr bool fold_fmt() {
    return QT == QT_Q2_K || QT == QT_Q3_K || QT == QT_Q4_K || QT == QT_Q5_K;
}
template <int QT, bool FOLD = fold_fmt<QT>()> struct KHdr { using T = typename Fmt<QT>::Hdr; };
template <int QT> struct KHdr<QT, true> { using T = typename Fmt<QT>::FHdr; };

template <int QT, int WN> struct BH { typename KHdr<QT>::T h[WN]; };
template <int QT, int WN> struct BK { typename Fmt<QT>::RawK r[WN]; };

template <int QT, int WN>
__device__ __forceinline__ void load_bh(const DevW &W, int Kc, const int (&gn)[WN], int c, int lane, BH<QT, WN> &b) {
#pragma unroll
    for (int j = 0; j < WN; j++) {
        if constexpr (fold_fmt<QT>()) Fmt<QT>::load_fhdr(W, Kc, gn[j], c, lane, b.h[j]);
        else Fmt<QT>::load_hdr(W, Kc, gn[j], c, lane, b.h[j]);
    }
}
template <int QT, int WN>
__device__ __forceinline__ void load_bk(const DevW &W, int Kc, const int (&gn)[WN], int c, int s, int lane,
                                        BK<QT, WN> &b) {
#pragma unroll
    for (int j = 0; j < WN; j++) Fmt<QT>::load_k(W, Kc, gn[j], c, s, lane, b.r[j]);
}

// A fragments of one kstep for WM row groups: the two f16 terms of its two
// half-steps
template <int WM> struct AK {
    half8 h[WM][2], l[WM][2];
};

// The exact product of one kstep into the chunk accumulator. Folded formats:
// acc += xh*(q f) + xl*(q f) for both half-steps, MFMA after MFMA; the others:
// t = the kstep's MFMAs from zero, acc = fma(sc, t, acc) per sub-block. The
// float operations each output sees, and their order, are the same in every
// caller.
//
// A1 (INT8ACT numerics): the activations are int8 values held as f16 (exact),
// one term: the xl MFMAs drop out, and every sum the MFMAs form is an exact
// integer (the kernels keep each accumulation below 2^24 in magnitude).
//
// NE: the per-element f32 work covers accumulator elements e < NE only (the
// GEMV of M rows reads elements 0 .. NE-1: rows drow(e, hh) below M); the
// elements it covers see the same operations at every NE.
template <int QT, int WM, int WN, bool A1 = false, int NE = 16>
__device__ __forceinline__ void kstep(const AK<WM> &a, const BK<QT, WN> &b, const BH<QT, WN> &hd, int s,
                                      f16v (&acc)[WM][WN]) {
    using F = Fmt<QT>;
    if constexpr (fold_fmt<QT>()) {
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const half8 b0 = F::decode_f(b.r[j], s, 0, hd.h[j]), b1 = F::decode_f(b.r[j], s, 1, hd.h[j]);
#pragma unroll
            for (int i = 0; i < WM; i++) {
                acc[i][j] = mfma32(a.h[i][0], b0, acc[i][j]);
                acc[i][j] = mfma32(a.h[i][1], b1, acc[i][j]);
                if constexpr (!A1) {
                    acc[i][j] = mfma32(a.l[i][0], b0, acc[i][j]);
                    acc[i][j] = mfma32(a.l[i][1], b1, acc[i][j]);
                }
            }
        }
    } else if constexpr (QT == QT_F32) {
        static_assert(!A1, "f32 weights have no int8-activation form");
        // f32 weights: resident as (wh, wl) f16 pairs scaled per row by
        // 2^shw_n; acc += xh*wh + xh*wl + xl*wh straight into the chunk
        // accumulator (no per-kstep factor)
#pragma unroll
        for (int kh = 0; kh < 2; kh++)
#pragma unroll
            for (int j = 0; j < WN; j++)
#pragma unroll
                for (int i = 0; i < WM; i++) {
                    acc[i][j] = mfma32(a.h[i][kh], b.r[j].h[kh], acc[i][j]);
                    acc[i][j] = mfma32(a.h[i][kh], b.r[j].l[kh], acc[i][j]);
                    acc[i][j] = mfma32(a.l[i][kh], b.r[j].h[kh], acc[i][j]);
                }
    } else if constexpr (!F::SUB16) {
        static_assert(!F::MINS, "affine formats fold");
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const half8 b0 = F::decode(b.r[j], s, 0), b1 = F::decode(b.r[j], s, 1);
            float sc, mn;
            F::scale(hd.h[j], s, 0, sc, mn);
#pragma unroll
            for (int i = 0; i < WM; i++) {
                f16v t = mfma32(a.h[i][0], b0, zero16());
                t = mfma32(a.h[i][1], b1, t);
                if constexpr (!A1) {
                    t = mfma32(a.l[i][0], b0, t);
                    t = mfma32(a.l[i][1], b1, t);
                }
#pragma unroll
                for (int e = 0; e < NE; e++) acc[i][j][e] = __builtin_fmaf(sc, t[e], acc[i][j][e]);
            }
        }
    } else {
        static_assert(!F::MINS, "affine formats fold");
#pragma unroll
        for (int j = 0; j < WN; j++) {
            half8 b0, b1;
            if constexpr (QT == QT_Q6_K) {   // the same values, fewer instructions
                b0 = F::decode_fast(b.r[j], s, 0);
                b1 = F::decode_fast(b.r[j], s, 1);
            } else {
                b0 = F::decode(b.r[j], s, 0);
                b1 = F::decode(b.r[j], s, 1);
            }
            float sc0, mn0, sc1, mn1;
            F::scale(hd.h[j], s, 0, sc0, mn0);
            F::scale(hd.h[j], s, 1, sc1, mn1);
#pragma unroll
            for (int i = 0; i < WM; i++) {
                f16v t0 = mfma32(a.h[i][0], b0, zero16());
                if constexpr (!A1) t0 = mfma32(a.l[i][0], b0, t0);
                f16v t1 = mfma32(a.h[i][1], b1, zero16());
                if constexpr (!A1) t1 = mfma32(a.l[i][1], b1, t1);
#pragma unroll
                for (int e = 0; e < NE; e++) {
                    acc[i][j][e] = __builtin_fmaf(sc0, t0[e], acc[i][j][e]);
                    acc[i][j][e] = __builtin_fmaf(sc1, t1[e], acc[i][j][e]);
                }
            }
        }
    }
}

// The affine folded formats' row sums as the A operand of the chunk's mins
// MFMA: sub-block sum x_j (NS per chunk: the 16-element sums (first 8 in
// order) + (next 8), for 32-element sub-blocks two of them added) scaled by
// 2^-5 (|x_j| < 2^20, so the result fits f16) and split into f16 hi_j + lo_j;
// lane half 0 carries hi_j in slot j, half 1 lo_j, slots >= NS are zero. The
// mins product is then sum_j (hi_j + lo_j) * m_j = 2^-5 * sum_j x_j m_j.
__device__ __forceinline__ _Float16 xm_part(float xsum, int hh) {
    const float v = xsum * 0.03125f;
    const _Float16 hi = (_Float16)v;
    return hh ? (_Float16)(v - (float)hi) : hi;
}
template <int NS>
__device__ __forceinline__ half8 xm_frag(const float (&s8)[HSTEPS], int hh) {
    float s16[HSTEPS];
#pragma unroll
    for (int u = 0; u < HSTEPS; u++) s16[u] = s8[u] + __shfl_xor(s8[u], 32);
    half8 r;
#pragma unroll
    for (int j = 0; j < 8; j++) {
        if (j < NS) r[j] = xm_part(NS == 8 ? s16[j] : s16[2 * j] + s16[2 * j + 1], hh);
        else r[j] = (_Float16)0.0f;
    }
    return r;
}

// End of a chunk of a folded format: acc (= sum of x * q f over the chunk)
// becomes d * acc - dm * (mins product), the chunk result the fold takes
template <int QT, int NE = 16>
__device__ __forceinline__ void fold_finish(const half8 &xm, const typename KHdr<QT>::T &H, f16v &acc) {
    if constexpr (Fmt<QT>::MINS) {
        const f16v t2 = mfma32(xm, H.mb, zero16());
#pragma unroll
        for (int e = 0; e < NE; e++) acc[e] = __builtin_fmaf(-H.dm, t2[e], H.d * acc[e]);
    } else {
#pragma unroll
        for (int e = 0; e < NE; e++) acc[e] = H.d * acc[e];
    }
}

// the per-row weight shift of the f32 format (0 for the quantized ones)
template <int QT>
__device__ __forceinline__ int wshift(const DevW &W, int n) {
    if constexpr (QT == QT_F32) return (int)W.h2[n];
    return 0;
}

__device__ __forceinline__ f16v load_rows16(const float *b) {
    // the lane's 16 D-layout rows from a [32]-row float vector (b at row 4*hh)
    f16v r;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 v = *(const float4 *)(b + 8 * q);
        r[4 * q + 0] = v.x; r[4 * q + 1] = v.y; r[4 * q + 2] = v.z; r[4 * q + 3] = v.w;
    }
    return r;
}

// ---------------------------------------------------------------------------
// Global -> LDS copies (global_load_lds: no VGPRs; the LDS destination is
// wave-uniform, lane l writes bytes [l*size, (l+1)*size) of each piece).
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) const void glob_void;

// src is wave-uniform: the address is an SGPR base + the lane's 32-bit offset
// (+ an immediate), so the copies need no per-lane 64-bit address math
template <int BYTES>
__device__ __forceinline__ void dma(const uint8_t *src, uint8_t *dst, int lane) {
    const glob_void *g = (const glob_void *)src;
    if constexpr (BYTES == 0) {
        return;
    } else if constexpr (BYTES % 1024 == 0) {
#pragma unroll
        for (int k = 0; k < BYTES / 1024; k++)
            __builtin_amdgcn_global_load_lds((const glob_void *)((const __attribute__((address_space(1))) uint8_t *)g +
                                                                 k * 1024 + (uint32_t)lane * 16u),
                                             (lds_void *)(dst + k * 1024), 16, 0, 0);
    } else if constexpr (BYTES % 256 == 0) {
#pragma unroll
        for (int k = 0; k < BYTES / 256; k++)
            __builtin_amdgcn_global_load_lds((const glob_void *)((const __attribute__((address_space(1))) uint8_t *)g +
                                                                 k * 256 + (uint32_t)lane * 4u),
                                             (lds_void *)(dst + k * 256), 4, 0, 0);
    } else {
        static_assert(BYTES == 128, "staged region size");
        if (lane < 32)
            __builtin_amdgcn_global_load_lds((const glob_void *)((const __attribute__((address_space(1))) uint8_t *)g +
                                                                 (uint32_t)lane * 4u),
                                             (lds_void *)dst, 4, 0, 0);
    }
}

// the lane's 16 D-layout rows from a staged [32]-row float vector
__device__ __forceinline__ f16v lds_rows16(const uint8_t *v, int hh) {
    f16v r;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const float4 x = *(const float4 *)(v + (8 * q + 4 * hh) * 4);
        r[4 * q + 0] = x.x; r[4 * q + 1] = x.y; r[4 * q + 2] = x.z; r[4 * q + 3] = x.w;
    }
    return r;
}

template <int N> __device__ __forceinline__ void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// LDS stage of k_gemm: SPS ksteps (half a chunk; one kstep for f32 weights,
// whose two f16 planes make a half-chunk stage 48 KiB) of everything the
// workgroup reads, for its 2 row groups and 4 column groups. Planes of 32 or
// more bytes per lane and chunk stage the stage's own part; narrower ones the
// whole (column group, chunk) block.
// BD: the weight planes go global -> registers instead of through LDS (each
// wave reads only its own column groups' planes, so LDS brings no reuse)
template <int QT, bool A1 = false, int NCG = 4, int NRG = 2, bool BD = false> struct StageLayout {
    using F = Fmt<QT>;
    static constexpr int SPS = QT == QT_F32 ? 1 : 2;              // ksteps per stage
    static constexpr int NST = KSTEPS / SPS;                      // stages per chunk
    static constexpr int TERMS = A1 ? 1 : 2;                      // activation f16 terms
    static constexpr int AR = SPS * 2048 * TERMS;                 // activation bytes per row group
    template <int B> static constexpr int plane() { return B == 0 ? 0 : (B >= 32 ? SPS * 16 * B : 64 * B); }
    template <int B> static __device__ int plane_off(int q) { return B >= 32 ? q * SPS * 16 * B : 0; }
    static constexpr int A = 0;                                   // [NRG rg][2 SPS u][TERMS][1 KiB]
    static constexpr int B0S = BD ? 0 : plane<F::B0>(), B1S = BD ? 0 : plane<F::B1>();
    static constexpr int P0 = A + NRG * AR;                       // [NCG cg][B0S]
    static constexpr int P1 = P0 + NCG * B0S;                     // [NCG cg][B1S]
    static constexpr int HB = P1 + NCG * B1S;                     // [NCG cg][F::HB]
    static constexpr int H2 = HB + NCG * F::HB;                   // [NCG cg][F::H2]
    static constexpr int PF = H2 + NCG * F::H2;                   // [NRG rg][32 floats]
    static constexpr int XS = PF + NRG * 128;                     // [NRG rg][64 lanes][16 B] mins A operand
    static constexpr int BYTES = XS + (F::MINS ? NRG * 1024 : 0);
};

// Where a product's result goes: EPI_Y stores y (SiLU applied when act);
// EPI_PREP (the first product of the FFN) applies SiLU and, instead of
// storing the f32 intermediate, prepares it as the second product's input —
// the workgroup's 128 output columns are exactly one 128-element chunk of
// the second product's K, so the chunk's shift, split and sums are formed
// here by split_part, the same function the preparation pass runs, on the
// same f32 values (bit-identical to storing y and preparing it).
enum { EPI_Y = 0, EPI_PREP = 1, EPI_PART = 2 };
// EPI_PART (launches with few tiles): workgroup (tile, split) runs one range
// of chunks and stores each chunk's result to part[c][Mpad][Np] instead of
// folding it; k_gemm_fold then folds them in chunk order from zero, with the
// prepared input's fold factors: the operations the fold in registers runs.
struct PrepOut {
    uint8_t *xp, *xm;
    float *xpf;
    int Kc, xsum;   // mins A operands (xm_frag): 0 none, 1 of 8 sub-blocks, 2 of 4
};

// workgroups per CU the register budget is sized for: as many as the LDS
// ring allows (three double-buffered workgroups: 25-27 KiB stages, 24 KiB
// one-kstep stages for f32 weights; four of 32-row tiles, three for f32
// weights), two for Q6_K (its eight per-half-step f32 factors need more
// registers), and two for the split-K form of the
// formats whose chunk-result stores would otherwise spill (INT4; Q5_K with
// int8 activations, whose chunk halves join in int32)
#ifndef GQ_V
#define GQ_V 0
#endif
#ifndef GQ_OCC
#define GQ_OCC 3
#endif
// The products' output epilogue (k_gemm_fold's; k_gemm's spells it out): act
// 1 SiLU; act 2 and 3 accumulate into y, y = fmaf(1 or 1/2, v, y) (the
// residual adds x += tmp and x += tmp / 2 of the encoder layer, with their
// operations); otherwise v.
__device__ __forceinline__ float epi_out(int act, float v, const float *yp) {
    if (act == 1) return silu_f(v);
    if (act >= 2) return fmaf(act == 3 ? 0.5f : 1.0f, v, *yp);
    return v;
}

template <int QT, int EPI, bool A1 = false, int WN = 1, int WM = 2> constexpr int gemm_occ() {
    if (QT == QT_Q8_0 && !A1 && WN == 1 && WM == 2 && EPI != EPI_PART) return GQ_OCC;
    if (WN > 1) return 2;
    if (WM == 1) return QT == QT_Q6_K || QT == QT_F32 ? 3 : 4;
    if (EPI == EPI_PART && (QT == QT_INT4 || (A1 && QT == QT_Q5_K))) return 2;
    return QT == QT_Q6_K ? 2 : 3;
}

// ---------------------------------------------------------------------------
// Large-M GEMM. Workgroup = 4 waves side by side over N, tile 64 x 128: row
// groups G0, G0+1 and column groups GC0..GC0+3; wave w computes both row
// groups against column group GC0+w (2 x 1 tiles of 32x32).
// Everything the MFMAs read goes through LDS in half-chunk stages,
// double-buffered: the next half's stage lands while the current one
// computes (a ring of three, two halves of lead, fits only twice per CU and
// measured 10-15% slower: occupancy hides the copy latency better). The copies are global_load_lds (no VGPRs hold prefetched data),
// shared out so that wave w brings its own column group's plane bytes and
// headers and a quarter of the activation pieces. Small LDS and VGPR
// footprints let two or three workgroups share a CU: their waves fill each
// other's stalls and overlap one's VALU epilogue with another's MFMAs.
// grid = tilesM * tilesN workgroups.
// A1: INT8ACT numerics (int8 activations as single f16 terms, xpf = their
// scales); Q5_K then sums each chunk as two exact halves (its products reach
// 127 * 1953, so a whole chunk could pass 2^24) joined in int32.
// WN: column groups per wave (1: tile 64 x 128 per workgroup; 2: 64 x 256,
// each wave 64 x 64, which halves the activation reads from LDS per MFMA).
// WM: row groups per wave and workgroup (2: tiles of 64 rows; 1: of 32 rows,
// twice the workgroups for products of few row bands).
template <int QT, int EPI, bool A1 = false, int WN = 1, int WM = 2>
__global__ __launch_bounds__(256, (gemm_occ<QT, EPI, A1, WN, WM>())) void k_gemm(GemmJobs J, const uint8_t *__restrict__ xp,
                                                 const uint8_t *__restrict__ xm,
                                                 const float *__restrict__ xpf,
                                                 int M, int act, int tilesM, int tilesN, PrepOut po,
                                                 float *__restrict__ part, int ksplit, int ngrp) {
    using F = Fmt<QT>;
    // the weight planes go straight to registers, one stage ahead (measured
    // 3-6% faster than through LDS on every format: less LDS traffic), except
    // in the split-K form (its chunk-result stores leave no registers for
    // them: with them it spilled, and 4096->1024 at 750 rows took 129 us, not
    // 50) and, for f32 weights, in the FFN's fused form (its epilogue's LDS
    // tile needs the larger stages)
    constexpr bool BD = EPI != EPI_PART && (QT != QT_F32 || EPI == EPI_Y);
    using L = StageLayout<QT, A1, 4 * WN, WM, BD>;
    typename F::RawK rb[2][WN][L::SPS];   // BD: the weight planes of the stage in flight and the current one
    static_assert(!(A1 && EPI == EPI_PREP), "the fused FFN hand-off is EXACT only");
    static_assert((WN == 1 && WM == 2) || EPI != EPI_PREP, "the fused FFN hand-off takes 64 x 128 tiles");
    constexpr bool HALVES = A1 && QT == QT_Q5_K;
    constexpr int WPR = 4 / WM;   // waves copying one row group's activations
    __shared__ __attribute__((aligned(16))) uint8_t sbuf[2][L::BYTES];
    // XCD-aware tile order: workgroups are dealt to the 8 XCDs round-robin
    // (bid % 8), each XCD with its own L2. Give every XCD a contiguous run of
    // tiles in row-band-major order, so that the N tiles of a row band — which
    // all read the same activations, the largest operand — share one L2
    // instead of fetching the band from HBM once per XCD.
    // Several products of one input (J.n jobs) share the row bands: the tiles
    // of band tm are (job, column tile) pairs, so one XCD runs all of a band's
    // products and reads its activations into its L2 once.
    // With EPI_PART, a band's splits follow each other (band, split, tile).
    // Without a K split, the order is N-group-major with ngrp groups of
    // column tiles (ngrp divides nj * tilesN), band-major inside a group: an
    // XCD's run then covers the bands of one group only, so the group's
    // slice of the weights can stay in its L2 while the bands stream past
    // (the host picks ngrp from the operand sizes; 1 = plain band-major).
    const int KS = EPI == EPI_PART ? ksplit : 1;
    const int nj = J.n, nt = nj * tilesN, ntiles = nt * tilesM * KS, bid = blockIdx.x;
    const int q = ntiles / 8, rem = ntiles % 8, xcd = bid % 8, loc = bid / 8;
    const int t = xcd < rem ? xcd * (q + 1) + loc : rem * (q + 1) + (xcd - rem) * q + loc;
    int tm, ks, tr;
    if (EPI == EPI_PART) {
        tm = t / (nt * KS);
        const int ts = t - tm * nt * KS;
        ks = ts / nt;
        tr = ts - ks * nt;
    } else {
        const int ntg = nt / ngrp, per = tilesM * ntg;
        const int g = t / per, r = t - g * per;
        tm = r / ntg;
        tr = g * ntg + (r - tm * ntg);
        ks = 0;
    }
    const int job = tr / tilesN, tn = tr - job * tilesN;
    const DevW W = job == 0 ? J.W[0] : (job == 1 ? J.W[1] : J.W[2]);
    float *__restrict__ y = job == 0 ? J.y[0] : (job == 1 ? J.y[1] : J.y[2]);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hh = lane >> 5, col = lane & 31;
    const int Kc = W.Kp / 128;
    const int G0 = tm * WM, GC0 = tn * 4 * WN;   // wave w: column groups GC0 + WN w + j
    const int cps = (Kc + KS - 1) / KS;
    const int c0 = EPI == EPI_PART ? ks * cps : 0, c1 = EPI == EPI_PART ? min(c0 + cps, Kc) : Kc;

    auto stage = [&](int c, int q, uint8_t *B) {
        const int rg = wave / WPR, pw = wave % WPR;
        dma<L::AR / WPR>(xp + (((size_t)(G0 + rg) * Kc + c) * 8 * L::TERMS + 2 * L::SPS * L::TERMS * q) * 1024 +
                             (size_t)pw * (L::AR / WPR),
                         B + L::A + rg * L::AR + pw * (L::AR / WPR), lane);
#pragma unroll
        for (int j = 0; j < WN; j++) {
            const int gc = GC0 + WN * wave + j, slot = WN * wave + j;
            if constexpr (BD) {
#pragma unroll
                for (int sl = 0; sl < L::SPS; sl++) F::load_k(W, Kc, gc, c, L::SPS * q + sl, lane, rb[q & 1][j][sl]);
            } else {
                dma<L::B0S>(W.p0 + ((size_t)gc * Kc + c) * 64 * F::B0 + L::template plane_off<F::B0>(q),
                            B + L::P0 + slot * L::B0S, lane);
                if constexpr (F::B1 > 0)
                    dma<L::B1S>(W.p1 + ((size_t)gc * Kc + c) * 64 * F::B1 + L::template plane_off<F::B1>(q),
                                B + L::P1 + slot * L::B1S, lane);
            }
            if constexpr (F::HB > 0) dma<F::HB>(F::hb_src(W, Kc, gc, c), B + L::HB + slot * F::HB, lane);
            if constexpr (F::H2 > 0) dma<F::H2>(F::h2_src(W, Kc, gc, c), B + L::H2 + slot * F::H2, lane);
        }
        if (wave < WM) {
            dma<128>((const uint8_t *)(xpf + ((size_t)(G0 + wave) * Kc + c) * 32), B + L::PF + wave * 128, lane);
            // the mins operand is read at the chunk's end, from its last stage
            if constexpr (F::MINS)
                if (q == L::NST - 1) dma<1024>(xm + ((size_t)(G0 + wave) * Kc + c) * 1024, B + L::XS + wave * 1024, lane);
        }
    };

    auto compute = [&](const uint8_t *B, int q, const BH<QT, WN> &hd, f16v (&acc)[WM][WN]) {
#if GQ_V & 1
        AK<WM> aa[L::SPS];
#pragma unroll
        for (int sl = 0; sl < L::SPS; sl++)
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int kh = 0; kh < 2; kh++) {
                    const uint8_t *pp = B + L::A + i * L::AR + ((2 * sl + kh) * L::TERMS) * 1024 + lane * 16;
                    aa[sl].h[i][kh] = *(const half8 *)pp;
                    if constexpr (!A1) aa[sl].l[i][kh] = *(const half8 *)(pp + 1024);
                }
#endif
#pragma unroll
        for (int sl = 0; sl < L::SPS; sl++) {
            const int s = L::SPS * q + sl;
#if GQ_V & 1
            const AK<WM> &a = aa[sl];
#else
            AK<WM> a;
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int kh = 0; kh < 2; kh++) {
                    const uint8_t *pp = B + L::A + i * L::AR + ((2 * sl + kh) * L::TERMS) * 1024 + lane * 16;
                    a.h[i][kh] = *(const half8 *)pp;
                    if constexpr (!A1) a.l[i][kh] = *(const half8 *)(pp + 1024);
                }
#endif
            BK<QT, WN> b;
            // (one-kstep stages hold only kstep s: its local index is 0)
#pragma unroll
            for (int j = 0; j < WN; j++) {
                if constexpr (BD) b.r[j] = rb[q & 1][j][sl];
                else
                    F::k_lds(B + L::P0 + (WN * wave + j) * L::B0S, B + L::P1 + (WN * wave + j) * L::B1S,
                             L::SPS == 1 ? 0 : s, lane, b.r[j]);
            }
            kstep<QT, WM, WN, A1>(a, b, hd, s, acc);
#if GQ_V & 2
            if constexpr (QT == QT_Q8_0 && !A1 && WN == 1 && WM == 2) {
#pragma unroll
                for (int g = 0; g < 8; g++) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // MFMA
                    __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);   // VALU
                }
            }
#endif
        }
    };

    f16v total[WM][WN];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int j = 0; j < WN; j++) total[i][j] = zero16();
    if (EPI != EPI_PART || c0 < c1) stage(c0, 0, sbuf[0]);
    for (int c = c0; c < c1; c++) {
        BH<QT, WN> hd;
        f16v acc[WM][WN];
        int half0[HALVES ? WM : 1][HALVES ? WN : 1][HALVES ? 16 : 1];
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int j = 0; j < WN; j++) acc[i][j] = zero16();
        // NST (even) stages per chunk, alternating buffers: stage 0 of every
        // chunk is in sbuf[0], the last in sbuf[1]
#pragma unroll
        for (int q = 0; q < L::NST; q++) {
            // the stage (issued one stage ago) has landed for every wave, and
            // every wave is done reading the buffer the next stage overwrites
            wait_vm<0>();
            __syncthreads();
            if (q + 1 < L::NST) stage(c, q + 1, sbuf[(q + 1) & 1]);
            else if (c + 1 < c1) stage(c + 1, 0, sbuf[0]);
            if (q == 0) {
                // the chunk's factors, from its headers (staged with every stage)
#pragma unroll
                for (int j = 0; j < WN; j++) {
                    const int slot = WN * wave + j;
                    if constexpr (fold_fmt<QT>())
                        F::fhdr_lds(sbuf[0] + L::HB + slot * F::HB, sbuf[0] + L::H2 + slot * F::H2, c, lane, hd.h[j]);
                    else
                        F::hdr_lds(sbuf[0] + L::HB + slot * F::HB, sbuf[0] + L::H2 + slot * F::H2, c, lane, hd.h[j]);
                }
            }
            compute(sbuf[q & 1], q, hd, acc);
            if constexpr (HALVES) {
                if (q == L::NST / 2 - 1) {
#pragma unroll
                    for (int i = 0; i < WM; i++)
#pragma unroll
                        for (int j = 0; j < WN; j++)
#pragma unroll
                            for (int e = 0; e < 16; e++) {
                                half0[i][j][e] = (int)acc[i][j][e];
                                acc[i][j][e] = 0.0f;
                            }
                }
            }
        }
        if constexpr (HALVES) {
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int j = 0; j < WN; j++)
#pragma unroll
                    for (int e = 0; e < 16; e++) acc[i][j][e] = (float)(half0[i][j][e] + (int)acc[i][j][e]);
        }
        if constexpr (fold_fmt<QT>()) {
#pragma unroll
            for (int i = 0; i < WM; i++) {
                half8 xmv = {};
                if constexpr (F::MINS) xmv = *(const half8 *)(sbuf[1] + L::XS + i * 1024 + lane * 16);
#pragma unroll
                for (int j = 0; j < WN; j++) fold_finish<QT>(xmv, hd.h[j], acc[i][j]);
            }
        }
        if constexpr (EPI == EPI_PART) {
            const size_t Mp = (size_t)tilesM * 32 * WM;
#pragma unroll
            for (int j = 0; j < WN; j++) {
                float *pc = part + ((size_t)job * Kc + c) * Mp * W.Np + 32 * (GC0 + WN * wave + j) + col;
#pragma unroll
                for (int i = 0; i < WM; i++)
#pragma unroll
                    for (int e = 0; e < 16; e++) pc[(size_t)(32 * (G0 + i) + drow(e, hh)) * W.Np] = acc[i][j][e];
            }
            continue;
        }
#pragma unroll
        for (int i = 0; i < WM; i++) {
            const f16v pv = lds_rows16(sbuf[1] + L::PF + i * 128, hh);
#pragma unroll
            for (int j = 0; j < WN; j++)
#pragma unroll
                for (int e = 0; e < 16; e++) total[i][j][e] = __builtin_fmaf(pv[e], acc[i][j][e], total[i][j][e]);
        }
    }
    wait_vm<0>();
    if constexpr (EPI == EPI_PART) return;
    if constexpr (EPI == EPI_PREP) {
        // the 64 x 128 SiLU tile through LDS (row stride 132 floats: 16-byte
        // aligned rows), then wave w splits half-steps 4*(w>>1) .. +3 of row
        // group w&1; the chunk's row maxima meet in LDS first
        constexpr int RS = 132;
        static_assert(2 * L::BYTES >= (64 * RS + 128) * 4, "LDS tile");
        float *T = (float *)&sbuf[0][0];
        float *amx = T + 64 * RS;  // [2 row groups][2 halves][32 rows]
        const int shw = wshift<QT>(W, 32 * (GC0 + wave) + col);  // (the pad columns hold 0)
        __syncthreads();
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                float v = total[i][0][e];
                if constexpr (QT == QT_F32) v = ldexpf(v, -shw);
                T[(32 * i + drow(e, hh)) * RS + 32 * wave + col] = silu_f(v);
            }
        __syncthreads();
        const int rg = wave & 1, uh = wave >> 1, G = G0 + rg;
        float v[4][8];
        float amax = 0.0f;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const float *src = T + (32 * rg + col) * RS + 16 * (4 * uh + u) + 8 * hh;
            const float4 a0 = *(const float4 *)src, a1 = *(const float4 *)(src + 4);
            v[u][0] = a0.x; v[u][1] = a0.y; v[u][2] = a0.z; v[u][3] = a0.w;
            v[u][4] = a1.x; v[u][5] = a1.y; v[u][6] = a1.z; v[u][7] = a1.w;
#pragma unroll
            for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[u][j]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 32));
        if (hh == 0) amx[(2 * rg + uh) * 32 + col] = amax;
        __syncthreads();
        const int sh = chunk_shift(fmaxf(amx[(2 * rg) * 32 + col], amx[(2 * rg + 1) * 32 + col]));
        half8 xh[4], xl[4];
        float s8[4];
        split_part<4>(v, sh, xh, xl, s8);
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int uu = 4 * uh + u;
            uint8_t *o = po.xp + ((((size_t)G * po.Kc + tn) * HSTEPS + uu) * 2) * 1024;
            *(half8 *)(o + lane * 16) = xh[u];
            *(half8 *)(o + (64 + lane) * 16) = xl[u];
        }
        if (po.xsum) {
            // this wave's sub-blocks of the mins operand (xm_frag's slots,
            // the same arithmetic): half-steps 4uh .. 4uh+3
            float s16[4];
#pragma unroll
            for (int u = 0; u < 4; u++) s16[u] = s8[u] + __shfl_xor(s8[u], 32);
            uint8_t *rec = po.xm + (((size_t)G * po.Kc + tn) * 64 + lane) * 16;
            if (po.xsum == 1) {   // 16-element sub-blocks 4uh .. 4uh+3
                half4v v;
#pragma unroll
                for (int u = 0; u < 4; u++) v[u] = xm_part(s16[u], hh);
                *(half4v *)(rec + 8 * uh) = v;
            } else {              // 32-element sub-blocks 2uh, 2uh+1; slots 4..7 zero
                const half2v v = {xm_part(s16[0] + s16[1], hh), xm_part(s16[2] + s16[3], hh)};
                *(half2v *)(rec + 4 * uh) = v;
                if (uh == 1) *(uint2 *)(rec + 8) = make_uint2(0u, 0u);
            }
        }
        if (hh == 0 && uh == 0) po.xpf[((size_t)G * po.Kc + tn) * 32 + col] = ldexpf(1.0f, -sh);
        return;
    }
#pragma unroll
    for (int j = 0; j < WN; j++) {
        const int n = 32 * (GC0 + WN * wave + j) + col;
        if (n >= W.n) continue;
        const int shw = wshift<QT>(W, n);
        if (act >= 2) {
            // the residual adds: every value of y this lane adds to is loaded
            // first, so the loads are in flight together
            float r[WM][16];
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = min(32 * (G0 + i) + drow(e, hh), M - 1);
                    r[i][e] = y[(size_t)m * W.n + n];
                }
            const float a = act == 3 ? 0.5f : 1.0f;
#pragma unroll
            for (int i = 0; i < WM; i++)
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = 32 * (G0 + i) + drow(e, hh);
                    if (m >= M) continue;
                    float v = total[i][j][e];
                    if constexpr (QT == QT_F32) v = ldexpf(v, -shw);
                    y[(size_t)m * W.n + n] = fmaf(a, v, r[i][e]);
                }
            continue;
        }
#pragma unroll
        for (int i = 0; i < WM; i++)
#pragma unroll
            for (int e = 0; e < 16; e++) {
                const int m = 32 * (G0 + i) + drow(e, hh);
                if (m >= M) continue;
                float v = total[i][j][e];
                if constexpr (QT == QT_F32) v = ldexpf(v, -shw);
                y[(size_t)m * W.n + n] = act ? silu_f(v) : v;
            }
    }
}

// The fold of EPI_PART's chunk results: y[m][n] from part[job][c][m][n], c
// in order from zero, with factor xpf[m/32][c][m%32] (what k_gemm stages as
// the chunk's fold factors), then k_gemm's own epilogue. Thread = (row m, four
// columns), blockIdx.y = job; the loads go out eight chunks at a time.
template <int QT>
__global__ __launch_bounds__(256) void k_gemm_fold(GemmJobs J, const float *__restrict__ part,
                                                   const float *__restrict__ xpf, int M, int Mp, int act) {
    const int job = blockIdx.y;
    const DevW W = job == 0 ? J.W[0] : (job == 1 ? J.W[1] : J.W[2]);
    float *__restrict__ y = job == 0 ? J.y[0] : (job == 1 ? J.y[1] : J.y[2]);
    const int n4 = W.Np / 4;
    const int idx = blockIdx.x * 256 + threadIdx.x;
    const int m = idx / n4, n = 4 * (idx - m * n4);
    if (m >= M) return;
    const int Kc = W.Kp / 128;
    const float *pf = xpf + (size_t)(m >> 5) * Kc * 32 + (m & 31);
    const float *pp = part + (size_t)job * Kc * Mp * W.Np + (size_t)m * W.Np + n;
    float total[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int c0 = 0; c0 < Kc; c0 += 8) {
        float4 pv[8];
        float fv[8];
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (c0 + u < Kc) {
                pv[u] = *(const float4 *)(pp + (size_t)(c0 + u) * Mp * W.Np);
                fv[u] = pf[(c0 + u) * 32];
            }
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (c0 + u < Kc) {
                total[0] = __builtin_fmaf(fv[u], pv[u].x, total[0]);
                total[1] = __builtin_fmaf(fv[u], pv[u].y, total[1]);
                total[2] = __builtin_fmaf(fv[u], pv[u].z, total[2]);
                total[3] = __builtin_fmaf(fv[u], pv[u].w, total[3]);
            }
    }
#pragma unroll
    for (int j = 0; j < 4; j++) {
        if (n + j >= W.n) return;
        float v = total[j];
        if constexpr (QT == QT_F32) v = ldexpf(v, -wshift<QT>(W, n + j));
        float *yp = y + (size_t)m * W.n + n + j;
        *yp = epi_out(act, v, yp);
    }
}

// ---------------------------------------------------------------------------
// Small-M GEMV (M <= 16), no preparation pass: each wave splits its chunks of
// x in registers (split_chunk, the same function k_prep runs) and applies
// them to WNG 32-column groups; the NW waves of a workgroup take chunks
// c = w, w+NW, ...; the chunk results of rows 0..15 and their fold factors
// meet in LDS and are folded in chunk order from zero — the sequence k_gemm
// runs in registers.
//
// A launch may carry up to three products of one input (jobs of the same
// format and shape: the workgroups of job i follow those of job i-1), and for
// M = 1 each wave may form its chunks of the input row itself: the layer norm
// of x, or the merge of attention splits (GPro).

// The input row of a one-row product built by each wave for its own chunks,
// with no workgroup barrier (the row's statistics are formed by every wave
// alone): lane l forms elements 128c + 2l, +1 of chunk c, and the wave moves
// them to the A-fragment layout through its own 128 floats of LDS. All the
// row's loads for the wave's first chunk go out before that chunk's weight
// loads: vector loads complete in issue order, so the row is formed while the
// weight bytes are still on their way.
//
//   GPRO_LN   (float)(((double)x - mean) * (double)inv) * w + b with inv =
//             (float)(1 / sqrt(var + 1e-5)), mean and var over the K values in
//             double, two passes (decoder_aed.c:21-28)
//   GPRO_COMB the attention splits of the element's head merged:
//             sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M), in split order
constexpr int PRO_XB = 8;   // chunks of x per batch of the layer-norm sums (1024 values)
constexpr int PRO_MB = 8;   // attention splits per batch of the merge
static_assert(PRO_XB == PRO_MB, "the two kinds share their load registers");
struct WaveRow {
    // GPRO_LN: a = the first PRO_XB chunks of x (float2 per lane and chunk),
    // then mu and inv; GPRO_COMB: n = the keys, a / b = (m, l) and the lane's
    // two partial outputs of the chunk's first PRO_MB splits
    float2 a[PRO_MB], b[PRO_MB];
    double mu;
    float inv;
    bool have;
    int n;
    float2 xc, wc, bc;   // (GPRO_LN) this chunk's own operands
};

__device__ __forceinline__ float2 ld2(const float *p) { return *(const float2 *)p; }

// issued once per wave, before anything else of the row
__device__ __forceinline__ void wave_row_begin(const GPro &pro, int K, int lane, WaveRow &r) {
    r.have = false;
    if (pro.kind == GPRO_LN) {
#pragma unroll
        for (int u = 0; u < PRO_XB; u++) {
            const int e = 128 * u + 2 * lane;
            r.a[u] = e < K ? ld2(pro.x + e) : float2{0.0f, 0.0f};
        }
    } else {
        r.n = pro.n_fixed > 0 ? pro.n_fixed : pro.st[0] + 1;
    }
}

// chunk c's own loads (before its weight loads)
__device__ __forceinline__ void wave_row_issue(const GPro &pro, int K, int c, int lane, WaveRow &r) {
    const int e = 128 * c + 2 * lane;
    const bool live = e < K;
    if (pro.kind == GPRO_LN) {
        r.xc = live ? ld2(pro.x + e) : float2{0.0f, 0.0f};
        r.wc = live ? ld2(pro.w + e) : float2{0.0f, 0.0f};
        r.bc = live ? ld2(pro.b + e) : float2{0.0f, 0.0f};
    } else {
        const int dk = K / pro.H, h = live ? e / dk : 0, f = live ? e - h * dk : 0;
        const float *ml = pro.ml + (size_t)h * pro.nsplit * 2;
        const float *op = pro.opart + (size_t)h * pro.nsplit * dk + f;
#pragma unroll
        for (int u = 0; u < PRO_MB; u++) {
            const bool ok = live && u < pro.nsplit;
            r.a[u] = ok ? ld2(ml + 2 * u) : float2{-INFINITY, 0.0f};
            r.b[u] = ok ? ld2(op + (size_t)u * dk) : float2{0.0f, 0.0f};
        }
    }
}

// a double moved between lanes by one DPP pattern (its two halves)
template <int CTRL>
__device__ __forceinline__ double dpp_d(double x) {
    const long long b = __double_as_longlong(x);
    const int lo = __builtin_amdgcn_update_dpp(0, (int)b, CTRL, 0xF, 0xF, false);
    const int hi = __builtin_amdgcn_update_dpp(0, (int)(b >> 32), CTRL, 0xF, 0xF, false);
    return __longlong_as_double(((long long)hi << 32) | (unsigned)lo);
}
// The wave's sum in every lane: within each row of 16 lanes by DPP (swap
// neighbours, swap pairs, mirror within 8, mirror within 16: each step adds
// two values symmetrically, so every lane holds the same sum), then across
// the four rows.
__device__ __forceinline__ double wave_sum(double v) {
    v += dpp_d<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp_d<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp_d<0x141>(v);   // row_half_mirror
    v += dpp_d<0x140>(v);   // row_mirror
    v += __shfl_xor(v, 16, 64);
    v += __shfl_xor(v, 32, 64);
    return v;
}

// the lane's two elements of chunk c (zero past K)
__device__ __forceinline__ float2 wave_row_values(const GPro &pro, int K, int c, int lane, WaveRow &r) {
    const int e = 128 * c + 2 * lane;
    const bool live = e < K;
    if (pro.kind == GPRO_LN) {
        if (!r.have) {
            // two passes in double, as ln(): the mean, then the sum of (x - mean)^2
            double s = 0.0;
#pragma unroll
            for (int u = 0; u < PRO_XB; u++) s += (double)r.a[u].x + (double)r.a[u].y;
            for (int c0 = PRO_XB; 128 * c0 < K; c0 += PRO_XB)   // K > 1024: further batches
#pragma unroll
                for (int u = 0; u < PRO_XB; u++) {
                    const int ee = 128 * (c0 + u) + 2 * lane;
                    const float2 v = ee < K ? ld2(pro.x + ee) : float2{0.0f, 0.0f};
                    s += (double)v.x + (double)v.y;
                }
            r.mu = wave_sum(s) / K;
            double q = 0.0;
#pragma unroll
            for (int u = 0; u < PRO_XB; u++)
                if (128 * u + 2 * lane < K) {
                    const double d0 = (double)r.a[u].x - r.mu, d1 = (double)r.a[u].y - r.mu;
                    q += d0 * d0 + d1 * d1;
                }
            for (int c0 = PRO_XB; 128 * c0 < K; c0 += PRO_XB)
#pragma unroll
                for (int u = 0; u < PRO_XB; u++) {
                    const int ee = 128 * (c0 + u) + 2 * lane;
                    if (ee < K) {
                        const float2 v = ld2(pro.x + ee);
                        const double d0 = (double)v.x - r.mu, d1 = (double)v.y - r.mu;
                        q += d0 * d0 + d1 * d1;
                    }
                }
            r.inv = (float)(1.0 / sqrt(wave_sum(q) / K + 1e-5));
            r.have = true;
        }
        if (!live) return float2{0.0f, 0.0f};
        const float t0 = (float)(((double)r.xc.x - r.mu) * (double)r.inv);
        const float t1 = (float)(((double)r.xc.y - r.mu) * (double)r.inv);
        return float2{t0 * r.wc.x + r.bc.x, t1 * r.wc.y + r.bc.y};
    }
    const int dk = K / pro.H, h = live ? e / dk : 0, f = live ? e - h * dk : 0;
    const int ns = min(mh_att_splits_dev(r.n), pro.nsplit);
    float Mx = -INFINITY;
#pragma unroll
    for (int u = 0; u < PRO_MB; u++)
        if (u < ns) Mx = fmaxf(Mx, r.a[u].x);
    const float *ml = pro.ml + (size_t)h * pro.nsplit * 2;
    const float *op = pro.opart + (size_t)h * pro.nsplit * dk + f;
    for (int s0 = PRO_MB; s0 < ns; s0++) Mx = fmaxf(Mx, ml[2 * s0]);
    float L = 0.0f, o0 = 0.0f, o1 = 0.0f;
#pragma unroll
    for (int u = 0; u < PRO_MB; u++)
        if (u < ns) {
            const float w = expf(r.a[u].x - Mx);
            L += r.a[u].y * w;
            o0 += r.b[u].x * w;
            o1 += r.b[u].y * w;
        }
    for (int s0 = PRO_MB; s0 < ns; s0 += PRO_MB) {   // further splits, PRO_MB loads at a time
        float2 mv[PRO_MB], ov[PRO_MB];
#pragma unroll
        for (int u = 0; u < PRO_MB; u++) {
            mv[u] = s0 + u < ns ? ld2(ml + 2 * (s0 + u)) : float2{-INFINITY, 0.0f};
            ov[u] = s0 + u < ns ? ld2(op + (size_t)(s0 + u) * dk) : float2{0.0f, 0.0f};
        }
#pragma unroll
        for (int u = 0; u < PRO_MB; u++)
            if (s0 + u < ns) {
                const float w = expf(mv[u].x - Mx);
                L += mv[u].y * w;
                o0 += ov[u].x * w;
                o1 += ov[u].y * w;
            }
    }
    if (!live) return float2{0.0f, 0.0f};
    return float2{o0 / L, o1 / L};
}

// The epilogue operands of a one-row product (the decoder's), loaded when the
// kernel starts so that their latency is not at its end: bias[n], res[0][n].
struct EpiPre {
    float b, r;
};
__device__ __forceinline__ EpiPre epi_pre(const DevW &W, int n, int M, int hh, const GEpi &ep) {
    EpiPre p{0.0f, 0.0f};
    if (M == 1 && hh == 0 && n < W.n) {
        if (ep.bias) p.b = ep.bias[n];
        if (ep.res) p.r = ep.res[n];
    }
    return p;
}

// y = act(W x + b) + res for output column n and the lane's 8 rows, in the
// order of the reference's mv() and its callers (decoder_aed.c:15-19, 207-210);
// for M = 1, b and res from pre; elements e < NE hold rows
template <int QT, int NE = 8>
__device__ __forceinline__ void gemv_store(const DevW &W, int n, int M, int hh, const float (&total)[8],
                                           const GEpi &ep, const EpiPre &pre, float *y) {
    if (n >= W.n) return;
    const int shw = wshift<QT>(W, n);
#pragma unroll
    for (int e = 0; e < NE; e++) {
        const int m = drow(e, hh);
        if (m >= M) continue;
        float v = total[e];
        if constexpr (QT == QT_F32) v = ldexpf(v, -shw);
        if (ep.bias) v = v + (M == 1 ? pre.b : ep.bias[n]);
        if (ep.act == 1) v = silu_f(v);
        else if (ep.act == 2) v = v < 0.0f ? 0.0f : v;
        if (ep.res) v = (M == 1 ? pre.r : ep.res[(size_t)m * W.n + n]) + v;
        y[(size_t)m * W.n + n] = v;
    }
}

// the GEMV of workgroup bx of one product (shared by k_gemv and k_gemv_jobs).
// NE: accumulator elements carried (1 for M = 1, 8 for M <= 16): rows
// drow(e, hh) for e < NE cover every row below M.
template <int QT, int NW, int WNG, bool VEC, bool PRO, int NE>
__device__ __forceinline__ void gemv_body(const DevW &W, const float *__restrict__ x, int M, float *y,
                                          const GEpi &ep, const GPro &pro, int bx) {
    extern __shared__ float part[];  // [Kc][WNG][8][64] chunk results, pf [Kc][16], prologue row [Kp]
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hh = lane >> 5, col = lane & 31;
    const int Kc = W.Kp / 128;
    float *pf = part + (size_t)Kc * WNG * 8 * 64;
    float *xs = pf + (size_t)Kc * 16;
    int gn[WNG];
#pragma unroll
    for (int j = 0; j < WNG; j++) gn[j] = bx * WNG + j;
    BH<QT, WNG> hd;
    BK<QT, WNG> bk[KSTEPS];
    auto load = [&](int c) {
        load_bh<QT, WNG>(W, Kc, gn, c, lane, hd);
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) load_bk<QT, WNG>(W, Kc, gn, c, s, lane, bk[s]);
    };
    // (the waves w < WNG store column group w)
    const EpiPre pre = wave < WNG ? epi_pre(W, 32 * (bx * WNG + wave) + col, M, hh, ep) : EpiPre{0.0f, 0.0f};
    WaveRow wr;
    if constexpr (PRO) wave_row_begin(pro, W.k, lane, wr);
    for (int c = wave; c < Kc; c += NW) {
        // x's chunk (a few KiB, in L2) goes out before the weights: vector
        // loads complete in issue order, so the split can start as soon as
        // x lands, while the weight bytes are still on their way
        float xv[HSTEPS][8];
        if constexpr (!PRO) load_chunk<VEC>(x, M, W.k, col, c, hh, xv);
        else wave_row_issue(pro, W.k, c, lane, wr);
        __builtin_amdgcn_sched_barrier(0);
        load(c);
        __builtin_amdgcn_sched_barrier(0);
        XChunk xc;
        if constexpr (PRO) {
            // M = 1: row 0, formed by this wave; its 128 values go to the
            // A-fragment layout (lanes 0 and 32) through the chunk's own LDS
            const float2 val = wave_row_values(pro, W.k, c, lane, wr);
            *(float2 *)(xs + 128 * c + 2 * lane) = val;
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            float v[HSTEPS][8];
#pragma unroll
            for (int u = 0; u < HSTEPS; u++)
#pragma unroll
                for (int j = 0; j < 8; j++) v[u][j] = col == 0 ? xs[128 * c + 16 * u + 8 * hh + j] : 0.0f;
            split_vals(v, xc);
        } else {
            split_vals(xv, xc);
        }
        if (hh == 0 && col < 16) pf[c * 16 + col] = xc.p;
        f16v acc[1][WNG];
#pragma unroll
        for (int j = 0; j < WNG; j++) acc[0][j] = zero16();
#pragma unroll
        for (int s = 0; s < KSTEPS; s++) {
            AK<1> a;
#pragma unroll
            for (int kh = 0; kh < 2; kh++) {
                a.h[0][kh] = xc.h[2 * s + kh];
                a.l[0][kh] = xc.l[2 * s + kh];
            }
            kstep<QT, 1, WNG, false, NE>(a, bk[s], hd, s, acc);
        }
        if constexpr (fold_fmt<QT>()) {
            // the mins operand from this chunk's own sums, as the preparation forms it
            half8 xmv = {};
            if constexpr (Fmt<QT>::MINS) xmv = xm_frag<Fmt<QT>::SUB16 ? 8 : 4>(xc.s8, hh);
#pragma unroll
            for (int j = 0; j < WNG; j++) fold_finish<QT, NE>(xmv, hd.h[j], acc[0][j]);
        }
#pragma unroll
        for (int j = 0; j < WNG; j++)
#pragma unroll
            for (int e = 0; e < NE; e++) part[((c * WNG + j) * 8 + e) * 64 + lane] = acc[0][j][e];
    }
    __syncthreads();
    for (int j = wave; j < WNG; j += NW) {
        float total[8];
#pragma unroll
        for (int e = 0; e < 8; e++) total[e] = 0.0f;
        for (int c = 0; c < Kc; c++)
#pragma unroll
            for (int e = 0; e < NE; e++)
                total[e] = __builtin_fmaf(pf[c * 16 + drow(e, hh)], part[((c * WNG + j) * 8 + e) * 64 + lane], total[e]);
        gemv_store<QT, NE>(W, 32 * gn[j] + col, M, hh, total, ep, pre, y);
    }
}

// Split-K GEMV for long K over few column groups (K >= 2048, N <= 2048: 32
// to 64 workgroups would each run many chunks in turn, one memory latency per
// chunk). Part 1: workgroup (column group bx, split ks) runs chunks
// ks*NW .. ks*NW+NW-1, one per wave, and writes each chunk's result rows
// (the values gemv_body keeps in LDS) to part[bx][c][8][64] and the fold
// factors to pfg[c][16]. Part 2 (k_gemv_fold) folds them in chunk order from
// zero: the same operations, so the rows are bit-identical to gemv_body's.
template <int QT, int NW, bool VEC, int NE>
__global__ __launch_bounds__(NW * 64) void k_gemv_part(DevW W, const float *__restrict__ x, int M,
                                                       float *__restrict__ part, float *__restrict__ pfg) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hh = lane >> 5, col = lane & 31;
    const int Kc = W.Kp / 128, c = blockIdx.y * NW + wave, bx = blockIdx.x;
    if (c >= Kc) return;   // (no barrier follows)
    const int gn[1] = {bx};
    BH<QT, 1> hd;
    BK<QT, 1> bk[KSTEPS];
    // x first: its loads complete before the weights' (issue order)
    float xv[HSTEPS][8];
    load_chunk<VEC>(x, M, W.k, col, c, hh, xv);
    __builtin_amdgcn_sched_barrier(0);
    load_bh<QT, 1>(W, Kc, gn, c, lane, hd);
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) load_bk<QT, 1>(W, Kc, gn, c, s, lane, bk[s]);
    __builtin_amdgcn_sched_barrier(0);
    XChunk xc;
    split_vals(xv, xc);
    if (bx == 0 && hh == 0 && col < 16) pfg[c * 16 + col] = xc.p;
    f16v acc[1][1];
    acc[0][0] = zero16();
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) {
        AK<1> a;
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            a.h[0][kh] = xc.h[2 * s + kh];
            a.l[0][kh] = xc.l[2 * s + kh];
        }
        kstep<QT, 1, 1, false, NE>(a, bk[s], hd, s, acc);
    }
    if constexpr (fold_fmt<QT>()) {
        half8 xmv = {};
        if constexpr (Fmt<QT>::MINS) xmv = xm_frag<Fmt<QT>::SUB16 ? 8 : 4>(xc.s8, hh);
        fold_finish<QT, NE>(xmv, hd.h[0], acc[0][0]);
    }
    float *o = part + ((size_t)bx * Kc + c) * 8 * 64;
#pragma unroll
    for (int e = 0; e < NE; e++) o[e * 64 + lane] = acc[0][0][e];
}

template <int QT>
__global__ __launch_bounds__(64) void k_gemv_fold(DevW W, const float *__restrict__ part,
                                                  const float *__restrict__ pfg, int M, float *y, GEpi ep) {
    const int lane = threadIdx.x, hh = lane >> 5, col = lane & 31, bx = blockIdx.x;
    const int Kc = W.Kp / 128;
    const EpiPre pre = epi_pre(W, 32 * bx + col, M, hh, ep);
    const float *pp = part + (size_t)bx * Kc * 8 * 64;
    // The fma chain of each row runs in chunk order from zero; what varies is
    // how far its loads go out ahead of it.
    float total[8];
#pragma unroll
    for (int e = 0; e < 8; e++) total[e] = 0.0f;
    if (M <= 2) {
        // one or two live rows (on the lanes of half 0): a row at a time, 32
        // chunks' loads together
#pragma unroll
        for (int e = 0; e < 2; e++) {
            const int row = drow(e, hh);
            if (row >= M) continue;
            for (int c0 = 0; c0 < Kc; c0 += 32) {
                float pv[32], fv[32];
#pragma unroll
                for (int u = 0; u < 32; u++)
                    if (c0 + u < Kc) {
                        pv[u] = pp[((size_t)(c0 + u) * 8 + e) * 64 + lane];
                        fv[u] = pfg[(c0 + u) * 16 + row];
                    }
#pragma unroll
                for (int u = 0; u < 32; u++)
                    if (c0 + u < Kc) total[e] = __builtin_fmaf(fv[u], pv[u], total[e]);
            }
        }
    } else {
        // all rows, eight chunks' loads at a time (Kc is even: Kp of 256)
        int c = 0;
        for (; c + 8 <= Kc; c += 8) {
            float pv[8][8], fv[8][8];
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int e = 0; e < 8; e++) {
                    pv[u][e] = pp[((size_t)(c + u) * 8 + e) * 64 + lane];
                    fv[u][e] = pfg[(c + u) * 16 + drow(e, hh)];
                }
#pragma unroll
            for (int u = 0; u < 8; u++)
#pragma unroll
                for (int e = 0; e < 8; e++) total[e] = __builtin_fmaf(fv[u][e], pv[u][e], total[e]);
        }
        for (; c < Kc; c++)
#pragma unroll
            for (int e = 0; e < 8; e++)
                total[e] = __builtin_fmaf(pfg[c * 16 + drow(e, hh)], pp[((size_t)c * 8 + e) * 64 + lane], total[e]);
    }
    gemv_store<QT>(W, 32 * bx + col, M, hh, total, ep, pre, y);
}

// one product: the compact argument block of the encoder and decoder GEMVs
template <int QT, int NW, int WNG, bool VEC, int NE>
__global__ __launch_bounds__(NW * 64) void k_gemv(DevW W, const float *__restrict__ x, int M, float *y, GEpi ep) {
    gemv_body<QT, NW, WNG, VEC, false, NE>(W, x, M, y, ep, GPro{}, blockIdx.x);
}

// up to three products of one prologue-built row (the decoder step)
template <int QT, int NW, int WNG>
__global__ __launch_bounds__(NW * 64) void k_gemv_jobs(GJobs J, GPro pro) {
    const int gpj = J.W[0].Np / 32 / WNG;   // workgroups per job
    const int job = blockIdx.x / gpj, bx = blockIdx.x - job * gpj;
    const DevW W = job == 0 ? J.W[0] : (job == 1 ? J.W[1] : J.W[2]);
    float *y = job == 0 ? J.y[0] : (job == 1 ? J.y[1] : J.y[2]);
    const GEpi ep = job == 0 ? J.ep[0] : (job == 1 ? J.ep[1] : J.ep[2]);
    gemv_body<QT, NW, WNG, false, true, 1>(W, nullptr, 1, y, ep, pro, bx);
}

// ---------------------------------------------------------------------------
// Activation preparation for k_gemm: workgroups of NWP waves per 32-row
// group (the launch uses one wave per chunk); a wave splits its chunks with
// split_chunk and stores
//   xp   A fragments of (xh, xl), zero beyond M and K   [G][chunk][u][term][64][16 B]
//   xm   the affine folded formats' mins A operand (xm_frag) of 8 (want_xsum
//        1) or 4 (want_xsum 2) sub-blocks       [G][chunk][64][16 B]
//   xpf  per row group, chunk and row: the fold factor 2^-sh  [G][chunk][32]
template <bool VEC, int NWP>
__global__ __launch_bounds__(64 * NWP) void k_prep(const float *__restrict__ x, int M, int K, int Kp,
                                              uint8_t *__restrict__ xp, uint8_t *__restrict__ xm,
                                              float *__restrict__ xpf, int want_xsum) {
    const int G = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int r = lane & 31, hh = lane >> 5, m = 32 * G + r;
    const int Kc = Kp / 128;
    // workgroup (G, y): chunks NWP y .. NWP y + NWP-1, one per wave (enough
    // waves to fill the chip at encoder sizes: M/32 row groups alone are fewer
    // than the CUs)
    for (int c = NWP * blockIdx.y + wave; c < Kc; c += NWP * gridDim.y) {
        XChunk xc;
        split_chunk<VEC>(x, M, K, m, c, hh, xc);
#pragma unroll
        for (int u = 0; u < HSTEPS; u++) {
            const size_t off = ((((size_t)G * Kc + c) * HSTEPS + u) * 2) * 64 * 16;
            *(half8 *)(xp + off + lane * 16) = xc.h[u];
            *(half8 *)(xp + off + (64 + lane) * 16) = xc.l[u];
        }
        if (want_xsum) {
            const half8 v = want_xsum == 1 ? xm_frag<8>(xc.s8, hh) : xm_frag<4>(xc.s8, hh);
            *(half8 *)(xm + (((size_t)G * Kc + c) * 64 + lane) * 16) = v;
        }
        if (hh == 0) xpf[((size_t)G * Kc + c) * 32 + r] = xc.p;
    }
}

// ---------------------------------------------------------------------------
// INT8ACT numerics: the reference's small-T int8 path (src/qmat.c:508-552),
// for every M. Activations are quantized per row exactly as
// quantize_act_int8 (qmat.c:186-202); v_mfma_i32_32x32x32_i8 forms the exact
// integer sum of one 32-block per instruction; the f32 combine follows the
// reference's order:
//   INT8   y = ((float)s * ws) * sx           (s over the whole row)
//   INT4   acc = acc + (float)ig * sg per group of 32, in order; y = acc * sx
//   Q8_0/Q4_0  the same with the block factor d (the oracle's block semantics)
// Int8 activation layout: [row group][kstep][64][16 B]; each lane's 16 bytes
// are half-steps 2s then 2s+1, each as dwords {e0,e4,e1,e5} {e2,e6,e3,e7} of
// elements 8hh..8hh+7 — the byte order of the weight planes, so weight bytes
// (or nibbles expanded with two masks) feed the MFMA unchanged.
typedef int i4v __attribute__((ext_vector_type(4)));
typedef int i16v __attribute__((ext_vector_type(16)));

__device__ __forceinline__ i16v mfma_i8(i4v a, i4v b, i16v c) {
    return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ int act_q8(float v, float inv) {
    const float t = __fmul_rn(v, inv);
    int q = (int)(t >= 0.0f ? __fadd_rn(t, 0.5f) : __fsub_rn(t, 0.5f));
    return q > 127 ? 127 : (q < -127 ? -127 : q);
}

// Otherwise two launches, each with work for the whole chip: the row scales (one wave
// per row: sx = amax / 127 and its factor 127 / amax, both rounded once, as
// quantize_act_int8 forms them), then the int8 values (one wave per 32-row
// group and kstep, the MFMA A-fragment layout).
// One pass for K <= 4096 with 16-byte rows: a wave per row holds the whole
// row in registers. Lane l owns NSL of the row's 16-byte fragment slots
// (slot q = l + 64 t: kstep q / 2, half hh = q % 2, elements 32 s + 8 hh ..
// +7 and 32 s + 16 + 8 hh .. +7), loads them, takes the row maximum over the
// wave, then quantizes and stores exactly those slots. A workgroup holds 8
// consecutive rows: the 8 lanes of one 128-byte line of a fragment are its
// rows r .. r + 7, so every line is written by one workgroup.
template <int NSL>
__global__ __launch_bounds__(512) void k_prep_i8_row(const float *__restrict__ x, int M, int K, int Kp, int Mpad,
                                                     uint8_t *__restrict__ qx, float *__restrict__ sx) {
    const int m = blockIdx.x * 8 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (m >= Mpad) return;
    const int S = Kp / 32, G = m >> 5, r = m & 31;
    const bool live_row = m < M;
    const float *row = x + (size_t)(live_row ? m : 0) * K;
    float v[NSL][16];
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < NSL; t++) {
        const int q = lane + 64 * t, s = q >> 1, hh = q & 1;
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            const int k0 = 32 * s + 16 * kh + 8 * hh;
            float4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
            if (live_row && q < 2 * S && k0 < K) {
                a = *(const float4 *)(row + k0);
                b = *(const float4 *)(row + k0 + 4);
            }
            v[t][8 * kh + 0] = a.x; v[t][8 * kh + 1] = a.y; v[t][8 * kh + 2] = a.z; v[t][8 * kh + 3] = a.w;
            v[t][8 * kh + 4] = b.x; v[t][8 * kh + 5] = b.y; v[t][8 * kh + 6] = b.z; v[t][8 * kh + 7] = b.w;
        }
    }
#pragma unroll
    for (int t = 0; t < NSL; t++)
#pragma unroll
        for (int j = 0; j < 16; j++) amax = fmaxf(amax, fabsf(v[t][j]));
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float iv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    if (lane == 0) sx[m] = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 0.0f;
    const bool live = live_row && iv > 0.0f;
    static const int kWord[8] = {0, 0, 1, 1, 0, 0, 1, 1};
    static const int kByte[8] = {0, 2, 0, 2, 1, 3, 1, 3};
#pragma unroll
    for (int t = 0; t < NSL; t++) {
        const int q = lane + 64 * t, s = q >> 1, hh = q & 1;
        if (q >= 2 * S) continue;
        uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            const int k0 = 32 * s + 16 * kh + 8 * hh;
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int qv = (live && k0 + j < K) ? act_q8(v[t][8 * kh + j], iv) : 0;
                w[2 * kh + kWord[j]] |= ((uint32_t)qv & 0xffu) << (8 * kByte[j]);
            }
        }
        *(uint4 *)(qx + (((size_t)G * S + s) * 64 + r + 32 * hh) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void k_rowscale_i8(const float *__restrict__ x, int M, int K, int Mpad,
                                                     float *__restrict__ sx, float *__restrict__ inv) {
    const int m = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (m >= Mpad) return;
    float amax = 0.0f;
    if (m < M) {
        const float *row = x + (size_t)m * K;
        if constexpr (VEC) {   // K % 8 == 0, 16-byte rows: four 16-byte loads per lane at a time
            for (int j0 = 4 * lane; j0 < K; j0 += 1024) {
                float4 v[4];
#pragma unroll
                for (int u = 0; u < 4; u++) {
                    const int j = j0 + 256 * u;
                    v[u] = j < K ? *(const float4 *)(row + j) : float4{0.f, 0.f, 0.f, 0.f};
                }
#pragma unroll
                for (int u = 0; u < 4; u++)
                    amax = fmaxf(fmaxf(fmaxf(amax, fabsf(v[u].x)), fmaxf(fabsf(v[u].y), fabsf(v[u].z))), fabsf(v[u].w));
            }
        } else {
#pragma unroll 4
            for (int j = lane; j < K; j += 64) amax = fmaxf(amax, fabsf(row[j]));
        }
    }
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    if (lane == 0) {
        inv[m] = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
        sx[m] = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 0.0f;
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void k_quant_i8(const float *__restrict__ x, int M, int K, int Kp,
                                                  uint8_t *__restrict__ qx, const float *__restrict__ inv) {
    const int G = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int S = Kp / 32, s = blockIdx.y * 4 + wave;
    if (s >= S) return;
    const int r = lane & 31, hh = lane >> 5, m = 32 * G + r;
    const float iv = inv[m];
    const bool live = m < M && iv > 0.0f;
    const float *row = x + (size_t)(m < M ? m : 0) * K;
    static const int kWord[8] = {0, 0, 1, 1, 0, 0, 1, 1};
    static const int kByte[8] = {0, 2, 0, 2, 1, 3, 1, 3};
    uint32_t w[4] = {0, 0, 0, 0};
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
        const int k0 = 32 * s + 16 * kh + 8 * hh;
        float v[8];
        if constexpr (VEC) {   // the lane's 8 elements in two 16-byte loads
            float4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
            if (live && k0 < K) {
                a = *(const float4 *)(row + k0);
                b = *(const float4 *)(row + k0 + 4);
            }
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
            v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        } else {
#pragma unroll
            for (int j = 0; j < 8; j++) v[j] = (live && k0 + j < K) ? row[k0 + j] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int q = (live && k0 + j < K) ? act_q8(v[j], iv) : 0;
            w[2 * kh + kWord[j]] |= ((uint32_t)q & 0xffu) << (8 * kByte[j]);
        }
    }
    *(uint4 *)(qx + (((size_t)G * S + s) * 64 + lane) * 16) = make_uint4(w[0], w[1], w[2], w[3]);
}

// ---------------------------------------------------------------------------
// INT8ACT activations for the ggml block formats, as the A1 GEMM reads them:
//   xp   int8 values as single f16 terms (exact)   [G][chunk][u][64][16 B]
//   xpf  the activation scale of each row and chunk [G][chunk][32]
//   xm   the affine formats' mins A operand from the exact integer sums of
//        the int8 values (xm_frag, want_xsum 1 / 2)  [G][chunk][64][16 B]
// PA1_ROW (Q8_0, Q4_0): one scale per row, quantized exactly as
//   quantize_act_int8 (src/qmat.c:186-202), the reference's int8 path.
// PA1_SB (the K-quants): one scale per 256-element super-block, quantized as
//   ingot's q4_k_quantize_activation (third_party/ingot/src/kernels.c:719-750):
//   scale = amax/127, q = round-to-nearest-even(x * (127/amax)), saturated.
enum { PA1_ROW = 0, PA1_SB = 1 };

__device__ __forceinline__ int act_q8_rne(float v, float inv) {
    const int q = __float2int_rn(__fmul_rn(v, inv));
    return q > 127 ? 127 : (q < -128 ? -128 : q);
}

// the lane's 8 values of half-step u of chunk c (zero past M or K)
template <bool VEC>
__device__ __forceinline__ void load8(const float *row, bool live, int K, int k0, float (&v)[8]) {
    if constexpr (VEC) {
        float4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
        if (live && k0 < K) {
            a = *(const float4 *)(row + k0);
            b = *(const float4 *)(row + k0 + 4);
        }
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; j++) v[j] = (live && k0 + j < K) ? row[k0 + j] : 0.0f;
    }
}

// one chunk's quantized values of the lane into the A1 layout, their 8-element
// sums into s8 (exact integers)
__device__ __forceinline__ void a1_store(uint8_t *xp, int G, int Kc, int c, int lane, const int (&q)[HSTEPS][8],
                                         float (&s8)[HSTEPS]) {
#pragma unroll
    for (int u = 0; u < HSTEPS; u++) {
        half8 h;
        int sum = 0;
#pragma unroll
        for (int j = 0; j < 8; j++) {
            h[j] = (_Float16)(float)q[u][j];
            sum += q[u][j];
        }
        s8[u] = (float)sum;
        *(half8 *)(xp + ((((size_t)G * Kc + c) * HSTEPS + u) * 64 + lane) * 16) = h;
    }
}

__device__ __forceinline__ void a1_store_xm(uint8_t *xm, int G, int Kc, int c, int lane, int hh,
                                            const float (&s8)[HSTEPS], int want_xsum) {
    if (!want_xsum) return;
    const half8 v = want_xsum == 1 ? xm_frag<8>(s8, hh) : xm_frag<4>(s8, hh);
    *(half8 *)(xm + (((size_t)G * Kc + c) * 64 + lane) * 16) = v;
}

// PA1_SB: workgroup (row group G, super-block b) = one wave over chunks 2b, 2b+1
template <bool VEC>
__global__ __launch_bounds__(64) void k_prep_a1_sb(const float *__restrict__ x, int M, int K, int Kp,
                                                   uint8_t *__restrict__ xp, uint8_t *__restrict__ xm,
                                                   float *__restrict__ xpf, int want_xsum) {
    const int G = blockIdx.x, b = blockIdx.y, lane = threadIdx.x;
    const int r = lane & 31, hh = lane >> 5, m = 32 * G + r;
    const int Kc = Kp / 128;
    const bool live = m < M;
    const float *row = x + (size_t)(live ? m : 0) * K;
    float v[2][HSTEPS][8];
    float amax = 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int u = 0; u < HSTEPS; u++) {
            load8<VEC>(row, live, K, 256 * b + 128 * h + 16 * u + 8 * hh, v[h][u]);
#pragma unroll
            for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[h][u][j]));
        }
    amax = fmaxf(amax, __shfl_xor(amax, 32));
    const bool nz = amax > 0.0f;
    const float inv = nz ? __fdiv_rn(127.0f, amax) : 0.0f;
    const float scale = nz ? __fdiv_rn(amax, 127.0f) : 0.0f;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int c = 2 * b + h;
        int q[HSTEPS][8];
#pragma unroll
        for (int u = 0; u < HSTEPS; u++)
#pragma unroll
            for (int j = 0; j < 8; j++) q[u][j] = nz ? act_q8_rne(v[h][u][j], inv) : 0;
        float s8[HSTEPS];
        a1_store(xp, G, Kc, c, lane, q, s8);
        a1_store_xm(xm, G, Kc, c, lane, hh, s8, want_xsum);
        if (hh == 0) xpf[((size_t)G * Kc + c) * 32 + r] = scale;
    }
}

// PA1_ROW: workgroup = one 32-row group; 16 waves find the row maxima (two
// rows each), then take the chunks in turn
constexpr int PREP_I8_NW = 16;
template <bool VEC>
__global__ __launch_bounds__(PREP_I8_NW * 64) void k_prep_a1_row(const float *__restrict__ x, int M, int K, int Kp,
                                                                 uint8_t *__restrict__ xp, float *__restrict__ xpf) {
    __shared__ float invs[32], sxs[32];
    const int G = blockIdx.x, lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    constexpr int RPW = 32 / PREP_I8_NW;
    for (int rr = 0; rr < RPW; rr++) {
        const int m = 32 * G + RPW * wave + rr;
        float amax = 0.0f;
        if (m < M) {
            const float *row = x + (size_t)m * K;
#pragma unroll 4
            for (int j = lane; j < K; j += 64) amax = fmaxf(amax, fabsf(row[j]));
        }
        for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
        if (lane == 0) {
            invs[RPW * wave + rr] = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
            sxs[RPW * wave + rr] = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 0.0f;
        }
    }
    __syncthreads();
    const int r = lane & 31, hh = lane >> 5, m = 32 * G + r;
    const float inv = invs[r], sx = sxs[r];
    const bool live = m < M && inv > 0.0f;
    const float *row = x + (size_t)(m < M ? m : 0) * K;
    const int Kc = Kp / 128;
    for (int c = wave; c < Kc; c += PREP_I8_NW) {
        int q[HSTEPS][8];
#pragma unroll
        for (int u = 0; u < HSTEPS; u++) {
            float v[8];
            load8<VEC>(row, live, K, 128 * c + 16 * u + 8 * hh, v);
#pragma unroll
            for (int j = 0; j < 8; j++) q[u][j] = (live && 128 * c + 16 * u + 8 * hh + j < K) ? act_q8(v[j], inv) : 0;
        }
        float s8[HSTEPS];
        a1_store(xp, G, Kc, c, lane, q, s8);
        if (hh == 0) xpf[((size_t)G * Kc + c) * 32 + r] = sx;
    }
}

// PA1_ROW in one pass for K <= 4096 with 16-byte rows (as k_prep_i8_row): a
// wave per row holds the row in registers. Lane l owns NSL of the row's
// 16-byte fragment slots (slot q = l + 64 t: chunk q / 16, half-step
// (q / 2) % 8, half q % 2: 8 elements), takes the row maximum over the wave,
// then stores those slots; lanes l < Kc (and l + 64 ...) store the chunk
// scales. A workgroup holds 8 consecutive rows, so every 128-byte line of a
// fragment is written by one workgroup.
template <int NSL>
__global__ __launch_bounds__(512) void k_prep_a1_row1(const float *__restrict__ x, int M, int K, int Kp, int Mpad,
                                                      uint8_t *__restrict__ xp, float *__restrict__ xpf) {
    const int m = blockIdx.x * 8 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (m >= Mpad) return;
    const int Kc = Kp / 128, NQ = Kp / 8, G = m >> 5, r = m & 31;
    const bool live_row = m < M;
    const float *row = x + (size_t)(live_row ? m : 0) * K;
    float v[NSL][8];
    float amax = 0.0f;
#pragma unroll
    for (int t = 0; t < NSL; t++) {
        const int q = lane + 64 * t, k0 = 8 * q;   // slot q's elements: 128 c + 16 u + 8 hh = 8 q
        float4 a = {0.f, 0.f, 0.f, 0.f}, b = a;
        if (live_row && q < NQ && k0 < K) {
            a = *(const float4 *)(row + k0);
            b = *(const float4 *)(row + k0 + 4);
        }
        v[t][0] = a.x; v[t][1] = a.y; v[t][2] = a.z; v[t][3] = a.w;
        v[t][4] = b.x; v[t][5] = b.y; v[t][6] = b.z; v[t][7] = b.w;
#pragma unroll
        for (int j = 0; j < 8; j++) amax = fmaxf(amax, fabsf(v[t][j]));
    }
    for (int off = 32; off > 0; off >>= 1) amax = fmaxf(amax, __shfl_xor(amax, off));
    const float inv = amax > 0.0f ? __fdiv_rn(127.0f, amax) : 0.0f;
    const float sx = amax > 0.0f ? __fdiv_rn(amax, 127.0f) : 0.0f;
    const bool live = live_row && inv > 0.0f;
#pragma unroll
    for (int t = 0; t < NSL; t++) {
        const int q = lane + 64 * t;
        if (q >= NQ) continue;
        const int c = q >> 4, u = (q >> 1) & 7, hh = q & 1, k0 = 8 * q;
        half8 h;
#pragma unroll
        for (int j = 0; j < 8; j++) h[j] = (_Float16)(float)((live && k0 + j < K) ? act_q8(v[t][j], inv) : 0);
        *(half8 *)(xp + ((((size_t)G * Kc + c) * HSTEPS + u) * 64 + r + 32 * hh) * 16) = h;
    }
    for (int c = lane; c < Kc; c += 64) xpf[((size_t)G * Kc + c) * 32 + r] = sx;
}

// 4 waves per workgroup, one 32-column group each, WM row groups per wave.
template <int QT, int WM>
__global__ __launch_bounds__(256) void k_gemm_i8(DevW W, const uint8_t *__restrict__ qx,
                                                 const float *__restrict__ sx, float *__restrict__ y,
                                                 int M, int act) {
    constexpr bool NIB = QT == QT_INT4 || QT == QT_Q4_0;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int hh = lane >> 5, col = lane & 31;
    const int G = blockIdx.x * 4 + wave;  // weight column group
    const int Kc = W.Kp / 128, S = W.Kp / 32;
    int gm[WM];
#pragma unroll
    for (int i = 0; i < WM; i++) gm[i] = blockIdx.y * WM + i;
    i16v si[WM];
    f16v acc[WM];
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            si[i][e] = 0;
            acc[i][e] = 0.0f;
        }
    i16v zi;
#pragma unroll
    for (int e = 0; e < 16; e++) zi[e] = 0;
    const i4v minus8 = {(int)0xF8F8F8F8u, (int)0xF8F8F8F8u, (int)0xF8F8F8F8u, (int)0xF8F8F8F8u};
    // the kstep's plane words, loaded one kstep ahead of their use
    auto ldw = [&](int ks) -> uint4 {
        const size_t tile = (size_t)G * Kc + (ks >> 2);
        const int s = ks & 3;
        if constexpr (NIB) {
            const uint2 v = *(const uint2 *)(W.p0 + ((tile * 2 + (s >> 1)) * 64 + lane) * 16 + 8 * (s & 1));
            return make_uint4(v.x, v.y, 0u, 0u);
        } else {
            return *(const uint4 *)(W.p0 + ((tile * 4 + s) * 64 + lane) * 16);
        }
    };
    uint4 nxt = ldw(0);
    for (int ks = 0; ks < S; ks++) {
        const int c = ks >> 2, s = ks & 3;
        const size_t tile = (size_t)G * Kc + c;
        const uint4 v = nxt;
        if (ks + 1 < S) nxt = ldw(ks + 1);
        uint32_t b[4];
        if constexpr (NIB) {
            b[0] = v.x & 0x0F0F0F0Fu;
            b[1] = (v.x >> 4) & 0x0F0F0F0Fu;
            b[2] = v.y & 0x0F0F0F0Fu;
            b[3] = (v.y >> 4) & 0x0F0F0F0Fu;
        } else {
            b[0] = v.x; b[1] = v.y; b[2] = v.z; b[3] = v.w;
            if constexpr (QT == QT_Q8_0) {   // the plane is offset binary: back to int8
#pragma unroll
                for (int i = 0; i < 4; i++) b[i] ^= 0x80808080u;
            }
        }
        float d = 0.f;
        if constexpr (QT == QT_Q8_0 || QT == QT_Q4_0) {
            const uint32_t hd = *(const uint32_t *)(W.h + (tile * 32 + col) * 8 + 4 * (s >> 1));
            d = h2f((hd >> (16 * (s & 1))) & 0xffff);
        } else if constexpr (QT == QT_INT4) {
            d = W.h2[(tile * 32 + col) * 4 + s];
        }
        const i4v bb = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
#pragma unroll
        for (int i = 0; i < WM; i++) {
            const i4v a = *(const i4v *)(qx + (((size_t)gm[i] * S + ks) * 64 + lane) * 16);
            if constexpr (QT == QT_INT8) {
                si[i] = mfma_i8(a, bb, si[i]);
            } else {
                // nibble formats: sum (n - 8) * q = sum q * (-8) + sum n * q
                const i16v t = mfma_i8(a, bb, NIB ? mfma_i8(a, minus8, zi) : zi);
#pragma unroll
                for (int e = 0; e < 16; e++) acc[i][e] = __fadd_rn(acc[i][e], __fmul_rn((float)t[e], d));
            }
        }
    }
    const int n = 32 * G + col;
    if (n >= W.n) return;
    const float ws = QT == QT_INT8 ? W.h2[n] : 0.0f;
#pragma unroll
    for (int i = 0; i < WM; i++)
#pragma unroll
        for (int e = 0; e < 16; e++) {
            const int m = 32 * gm[i] + drow(e, hh);
            if (m >= M) continue;
            float v;
            if constexpr (QT == QT_INT8) v = __fmul_rn(__fmul_rn((float)si[i][e], ws), sx[m]);
            else v = __fmul_rn(acc[i][e], sx[m]);
            y[(size_t)m * W.n + n] = act ? silu_f(v) : v;
        }
}

// The qmat INT8 product at encoder sizes: one int32 sum per output over all
// of K (qmat.c:464-500), so the main loop is MFMAs only. Workgroup = 4 waves
// side by side over N: tile TR row groups x 4 CW column groups of 32, wave w
// takes every row group against column groups CW w .. CW w + CW - 1. The
// loop runs in steps of SK ksteps:
//   * the activations, which all four waves read, go global -> registers
//     two steps ahead, then into one of two LDS slots at the end of the step
//     before their use (one barrier per step);
//   * each wave's weight fragments are its own (no reuse between waves), so
//     they go global -> registers one step ahead and never touch LDS.
// Only ordinary loads are used, so the compiler's own waits before each use
// count exactly what is still in flight (with global_load_lds it cannot, and
// waits for everything). Row groups past the prepared rows and column groups
// past Np load a valid neighbour's bytes (no output reads them), and the
// loads past the last step reload it, so every step issues the same loads.
// Every fragment is the MFMA's own 1 KiB lane-order block ([group][kstep][64]
// [16 B]): coalesced 16-byte loads, conflict-free 16-byte LDS accesses.
// Tiles go to the XCDs in contiguous band-major runs (as k_gemm), so a row
// band's column tiles share one L2. The sums are exact integers: the result
// has the bits of k_gemm_i8.
template <int TR, int CW, int SK>
__global__ __launch_bounds__(256, 2) void k_gemm_i8t(DevW W, const uint8_t *__restrict__ qx,
                                                     const float *__restrict__ sx, float *__restrict__ y, int M,
                                                     int act, int tilesM, int tilesN) {
    constexpr int TC = 4 * CW;                  // tile in column groups
    constexpr int STB = TR * SK * 1024;         // LDS slot: [TR][SK][1 KiB] activations
    constexpr int PPW = TR * SK / 4;            // activation fragments per wave and step
    constexpr int LDSB = 2 * STB > 4 * 32 * 36 * 4 ? 2 * STB : 4 * 32 * 36 * 4;   // two slots; the epilogue's tiles
    static_assert(TR * SK % 4 == 0, "step shape");
    __shared__ __attribute__((aligned(16))) uint8_t sbuf[LDSB];
    const int ntiles = tilesM * tilesN, bid = blockIdx.x;
    const int q8 = ntiles / 8, rem = ntiles % 8, xcd = bid % 8, loc = bid / 8;
    const int t = xcd < rem ? xcd * (q8 + 1) + loc : rem * (q8 + 1) + (xcd - rem) * q8 + loc;
    const int tm = t / tilesN, tn = t - tm * tilesN;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int hh = lane >> 5, col = lane & 31;
    const int S = W.Kp / 32, NS = S / SK;
    const int G0 = tm * TR, GC0 = tn * TC + CW * wave;
    const int Gend = (M + 63) / 64 * 2, GCend = W.Np / 32;   // prepared row groups (M padded to 64); column groups

    const uint8_t *bsrc[CW];
#pragma unroll
    for (int j = 0; j < CW; j++) bsrc[j] = W.p0 + (size_t)min(GC0 + j, GCend - 1) * S * 1024 + lane * 16;
    const uint8_t *asrc[PPW];
    int aoff[PPW];   // LDS offset of the wave's fragment u within a slot
#pragma unroll
    for (int u = 0; u < PPW; u++) {
        const int pc = wave * PPW + u, grp = pc / SK, sl = pc % SK;
        asrc[u] = qx + ((size_t)min(G0 + grp, Gend - 1) * S + sl) * 1024 + lane * 16;
        aoff[u] = (grp * SK + sl) * 1024 + lane * 16;
    }
    auto load_b = [&](int st, i4v(&b)[CW][SK]) {
        st = min(st, NS - 1);
#pragma unroll
        for (int j = 0; j < CW; j++)
#pragma unroll
            for (int k = 0; k < SK; k++) b[j][k] = *(const i4v *)(bsrc[j] + (size_t)(SK * st + k) * 1024);
    };
    auto load_a = [&](int st, i4v(&r)[PPW]) {
        st = min(st, NS - 1);
#pragma unroll
        for (int u = 0; u < PPW; u++) r[u] = *(const i4v *)(asrc[u] + (size_t)SK * st * 1024);
    };
    auto put_a = [&](const i4v(&r)[PPW], uint8_t *B) {
#pragma unroll
        for (int u = 0; u < PPW; u++) *(i4v *)(B + aoff[u]) = r[u];
    };

    i16v acc[TR][CW];
#pragma unroll
    for (int i = 0; i < TR; i++)
#pragma unroll
        for (int j = 0; j < CW; j++)
#pragma unroll
            for (int e = 0; e < 16; e++) acc[i][j][e] = 0;
    i4v bb0[CW][SK], bb1[CW][SK], ra0[PPW], ra1[PPW];
    load_b(0, bb0);
    load_a(0, ra0);
    load_a(1, ra1);
    put_a(ra0, sbuf);
    __syncthreads();
    // step st: b = B(st), ra = A(st + 1) (written to slot (st + 1) & 1 at
    // the end), rn receives A(st + 2), bn receives B(st + 1)
    auto step = [&](int st, const i4v(&b)[CW][SK], i4v(&bn)[CW][SK], const i4v(&ra)[PPW], i4v(&rn)[PPW]) {
        load_b(st + 1, bn);
        load_a(st + 2, rn);
        __builtin_amdgcn_sched_barrier(0);   // (the loads go out before the step's MFMAs)
        const uint8_t *B = sbuf + (st & 1) * STB;
        // kstep k + 1's activation fragments are read before kstep k's MFMAs
        // (with one wave per SIMD nothing else hides the LDS latency)
        i4v a[2][TR];
#pragma unroll
        for (int i = 0; i < TR; i++) a[0][i] = *(const i4v *)(B + (i * SK) * 1024 + lane * 16);
#pragma unroll
        for (int k = 0; k < SK; k++) {
            if (k + 1 < SK) {
#pragma unroll
                for (int i = 0; i < TR; i++) a[(k + 1) & 1][i] = *(const i4v *)(B + (i * SK + k + 1) * 1024 + lane * 16);
            }
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int i = 0; i < TR; i++)
#pragma unroll
                for (int j = 0; j < CW; j++) acc[i][j] = mfma_i8(a[k & 1][i], b[j][k], acc[i][j]);
            __builtin_amdgcn_sched_barrier(0);
        }
        // slot (st + 1) & 1 was last read at step st - 1, before the barrier
        // that ended it
        put_a(ra, sbuf + ((st + 1) & 1) * STB);
        __syncthreads();
    };
    for (int st = 0; st < NS; st += 2) {
        step(st, bb0, bb1, ra1, ra0);
        if (st + 1 < NS) step(st + 1, bb1, bb0, ra0, ra1);
    }
    // epilogue: y = (acc * ws[n]) * sx[m] (SiLU when act). Each 32 x 32
    // block goes through the wave's own 4 KiB of LDS (row stride 36 floats)
    // and out as rows of 32 columns in 16-byte stores, 8 lanes per row;
    // without 16-byte alignment (y, or N not a multiple of 4), element by
    // element.
    const bool vec = (W.n & 3) == 0 && ((uintptr_t)y & 15) == 0;
    float *T = (float *)sbuf + wave * 32 * 36;   // (the last step ended with a barrier)
#pragma unroll
    for (int i = 0; i < TR; i++) {
        float sxr[16];
#pragma unroll
        for (int e = 0; e < 16; e++) sxr[e] = sx[min(32 * (G0 + i) + drow(e, hh), M - 1)];
#pragma unroll
        for (int j = 0; j < CW; j++) {
            const int n = 32 * (GC0 + j) + col;
            const float ws = W.h2[min(n, W.n - 1)];
            if (vec) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const float v = __fmul_rn(__fmul_rn((float)acc[i][j][e], ws), sxr[e]);
                    T[drow(e, hh) * 36 + col] = act ? silu_f(v) : v;
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                const int nc = 32 * (GC0 + j) + 4 * (lane & 7);
#pragma unroll
                for (int r0 = 0; r0 < 32; r0 += 8) {
                    const int r = r0 + (lane >> 3), m = 32 * (G0 + i) + r;
                    const float4 v = *(const float4 *)(T + r * 36 + 4 * (lane & 7));
                    if (m < M && nc < W.n) *(float4 *)(y + (size_t)m * W.n + nc) = v;
                }
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                __builtin_amdgcn_wave_barrier();
                __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            } else if (n < W.n) {
#pragma unroll
                for (int e = 0; e < 16; e++) {
                    const int m = 32 * (G0 + i) + drow(e, hh);
                    if (m >= M) continue;
                    const float v = __fmul_rn(__fmul_rn((float)acc[i][j][e], ws), sxr[e]);
                    y[(size_t)m * W.n + n] = act ? silu_f(v) : v;
                }
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Dequantization from the resident layout: one wave per (column group, chunk).
// Values are formed exactly as the reference decoders form them.
template <int QT>
__global__ __launch_bounds__(64) void k_dequant(DevW W, float *__restrict__ out) {
    using F = Fmt<QT>;
    const int lane = threadIdx.x, c = blockIdx.x, G = blockIdx.y;
    const int Kc = W.Kp / 128;
    typename F::Hdr hd;
    F::load_hdr(W, Kc, G, c, lane, hd);
    const int n = 32 * G + (lane & 31), hh = lane >> 5;
    if (n >= W.n) return;
#pragma unroll
    for (int s = 0; s < KSTEPS; s++) {
        typename F::RawK raw;
        F::load_k(W, Kc, G, c, s, lane, raw);
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            const half8 q = F::decode(raw, s, kh);
            float sc, mn;
            F::scale(hd, s, F::SUB16 ? kh : 0, sc, mn);
#pragma unroll
            for (int j = 0; j < 8; j++) {
                const int k = 128 * c + 32 * s + 16 * kh + 8 * hh + j;
                if (k >= W.k) continue;
                const float qv = (float)q[j];
                float v;
                if constexpr (F::MINS) v = __fsub_rn(__fmul_rn(sc, qv), mn);
                else v = __fmul_rn(sc, qv);
                out[(size_t)n * W.k + k] = v;
            }
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

#include <type_traits>

#include "launch.h"

// A plain streaming read of `n4` float4 (the one-launch floor a memory-bound
// kernel of the same bytes is measured against: no compute, nothing written
// unless the data sum to a value they never do). Four loads per thread per
// round, all issued before their sums.
__device__ float g_read_sink;
__global__ __launch_bounds__(256) void k_read_floor(const float4 *__restrict__ p, size_t n4) {
    const size_t stride = (size_t)gridDim.x * 256;
    float s = 0.0f;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n4; i += 4 * stride) {
        float4 v[4];
#pragma unroll
        for (int u = 0; u < 4; u++) v[u] = i + u * stride < n4 ? p[i + u * stride] : float4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int u = 0; u < 4; u++) s += (v[u].x + v[u].y) + (v[u].z + v[u].w);
    }
    if (s == -1.2345e-37f) g_read_sink = s;
}

template <typename F>
static hipError_t allow_lds(F *f) {
    // dynamic LDS beyond 64 KiB: gfx950 has 160 KiB, less the prologue's static
    // scratch (about 5 KiB); the largest GEMV request is about 130 KiB
    return hipFuncSetAttribute((const void *)f, hipFuncAttributeMaxDynamicSharedMemorySize, 154 * 1024);
}

template <int QT, int NW, int WNG, bool VEC, bool PRO>
static hipError_t launch_gemv1(const GJobs &J, const float *x, int M, const GPro &pro, hipStream_t st) {
    const DevW &W = J.W[0];
    const int Kc = W.Kp / 128;
    const size_t lds = ((size_t)Kc * WNG * 8 * 64 + (size_t)Kc * 16 + (PRO ? (size_t)W.Kp : 0)) * sizeof(float);
    // set once per instantiation; a function-local static's initialisation is
    // thread-safe, so concurrent first calls wait for the one that runs it
    static const hipError_t attr = []() {
        if constexpr (PRO) {
            return allow_lds(k_gemv_jobs<QT, NW, WNG>);
        } else {
            hipError_t e = allow_lds(k_gemv<QT, NW, WNG, VEC, 1>);
            if (e == hipSuccess) e = allow_lds(k_gemv<QT, NW, WNG, VEC, 4>);
            if (e == hipSuccess) e = allow_lds(k_gemv<QT, NW, WNG, VEC, 8>);
            return e;
        }
    }();
    if (attr != hipSuccess) return attr;
    if constexpr (PRO) {
        hipLaunchKernelGGL((k_gemv_jobs<QT, NW, WNG>), dim3(W.Np / 32 / WNG * J.n), dim3(NW * 64), lds, st, J, pro);
    } else {
        if (J.n != 1) return hipErrorInvalidValue;
        // accumulator elements the M rows need (rows drow(e, hh) < M)
        if (M == 1)
            hipLaunchKernelGGL((k_gemv<QT, NW, WNG, VEC, 1>), dim3(W.Np / 32 / WNG), dim3(NW * 64), lds, st, W, x, M,
                               J.y[0], J.ep[0]);
        else if (M <= 8)
            hipLaunchKernelGGL((k_gemv<QT, NW, WNG, VEC, 4>), dim3(W.Np / 32 / WNG), dim3(NW * 64), lds, st, W, x, M,
                               J.y[0], J.ep[0]);
        else
            hipLaunchKernelGGL((k_gemv<QT, NW, WNG, VEC, 8>), dim3(W.Np / 32 / WNG), dim3(NW * 64), lds, st, W, x, M,
                               J.y[0], J.ep[0]);
    }
    return hipGetLastError();
}

// WITH_PRO / WITH_SCALAR: whether the row-forming form and the form for
// unaligned x (element loads) exist at this shape (callers route around them)
template <int QT, int NW, int WNG, bool WITH_PRO = true, bool WITH_SCALAR = true>
static hipError_t launch_gemv(const GJobs &J, const float *x, int M, int vec, const GPro &pro, hipStream_t st) {
    if constexpr (WITH_PRO) {
        if (pro.kind != GPRO_NONE) return launch_gemv1<QT, NW, WNG, false, true>(J, x, M, pro, st);
    } else {
        if (pro.kind != GPRO_NONE) return hipErrorInvalidValue;
    }
    if (vec) return launch_gemv1<QT, NW, WNG, true, false>(J, x, M, pro, st);
    if constexpr (WITH_SCALAR) return launch_gemv1<QT, NW, WNG, false, false>(J, x, M, pro, st);
    return hipErrorInvalidValue;
}

// column groups per GEMV workgroup: two for wide outputs, so that each chunk
// of x is split once for both
static int gemv_wng(const DevW &W) {
    const int Kc = W.Kp / 128, groups = W.Np / 32;
    if (groups >= 256 && Kc <= 32) return 2;
    return 1;
}

template <int QT>
static hipError_t gemv_t(const GJobs &J, const float *x, int M, int vec, const GPro &pro, hipStream_t st) {
    const DevW &W = J.W[0];
    const int Kc = W.Kp / 128, wng = gemv_wng(W);
    // (f32 weights form their row with one column group per wave: the two
    // f16 planes of two groups beside the row registers spill)
    constexpr bool PRO2 = QT != QT_F32;
    if (wng == 2 && (PRO2 || pro.kind == GPRO_NONE)) {
        if (Kc >= 8) return launch_gemv<QT, 8, 2, PRO2>(J, x, M, vec, pro, st);
        return launch_gemv<QT, 4, 2, PRO2>(J, x, M, vec, pro, st);
    }
    // K >= 4096 over few column groups: 16 waves take two chunks each rather
    // than 8 taking four (each chunk's loads wait a full memory latency);
    // within the 128 registers a 1024-thread workgroup allows, except the
    // formats whose GEMV needs more (Q2_K spilled 60 registers there), the
    // row-forming form (its per-wave row registers) and unaligned x (Q8_0's
    // element loads spilled 4)
    if constexpr (QT != QT_F32 && QT != QT_Q2_K && QT != QT_Q4_K && QT != QT_Q5_K && QT != QT_Q6_K)
        if (Kc >= 32 && pro.kind == GPRO_NONE && vec) return launch_gemv<QT, 16, 1, false, false>(J, x, M, vec, pro, st);
    if (Kc >= 8) return launch_gemv<QT, 8, 1>(J, x, M, vec, pro, st);
    return launch_gemv<QT, 4, 1>(J, x, M, vec, pro, st);
}

// K split for a launch of few tiles (at most one workgroup per CU otherwise,
// each running its chunks as one long dependent chain): enough (tile, split)
// workgroups for three per CU, none of them empty. 1: no split. It pays when
// the chain it shortens is long (16 chunks or more) or the chunk results the
// fold reads back are few (outputs of at most 512K elements over all jobs);
// measured on 1024 -> 1024 at M = 750 (8 chunks, 786K outputs), and on three
// such products at M = 256, it does not.
static int gemm_ksplit(int Kc, int tiles, size_t outs) {
    if (tiles > 256 || Kc < 2 || (Kc < 16 && outs > ((size_t)512 << 10))) return 1;
    if ((size_t)Kc * outs > ((size_t)64 << 20)) return 1;   // workspace above 256 MiB: unsplit
    int s = (768 + tiles - 1) / tiles;
    if (s > Kc) s = Kc;
    const int cps = (Kc + s - 1) / s;
    return (Kc + cps - 1) / cps;
}

size_t mh_gemm_ws_floats(const DevW &W, int M, int jobs) {
    const int Kc = W.Kp / 128, tilesM = mh_mpad(M) / 64;
    const size_t outs = (size_t)jobs * tilesM * 64 * W.Np;   // over all jobs
    if (W.Np % 128 != 0 || gemm_ksplit(Kc, jobs * tilesM * (W.Np / 128), outs) == 1) return 0;
    return (size_t)Kc * outs;
}

// Weight bytes per element of the resident layout (planes and headers)
template <int QT> constexpr float w_bpe() {
    return QT == QT_F32 ? 4.0f : QT == QT_INT8 ? 1.0f : QT == QT_INT4 ? 0.5625f : QT == QT_Q4_0 ? 0.5625f
         : QT == QT_Q8_0 ? 1.0625f : QT == QT_Q2_K ? 0.33f : QT == QT_Q3_K ? 0.43f : QT == QT_Q4_K ? 0.5625f
         : QT == QT_Q5_K ? 0.6875f : 0.82f;
}

// Column-tile groups of the tile order (k_gemm's ngrp): the count in {1, 2, 4}
// that minimises a model of the L2 misses. Each XCD runs about 96 tiles at a
// time (32 CUs x 3) out of an L2 of 4 MB. A group's weight slice that fits
// beside the bands in flight is read once per XCD; one that does not is read
// again for every round of tiles. Every extra group reads the activations
// once more.
static int gemm_ngroups(float wbytes, float abytes, int tilesM, int nt) {
    const float l2 = 4.0f * 1048576.0f, conc = 96.0f;
    const float band = abytes / (float)tilesM, rounds = fmaxf(1.0f, (float)tilesM * nt / 8.0f / conc);
    int best = 1;
    float best_cost = 0.0f;
    for (int S = 1; S <= 4; S *= 2) {
        if (nt % S) continue;
        const float wslice = wbytes / S, bands_in_flight = fminf((float)tilesM, conc * S / nt);
        const bool fits = wslice + bands_in_flight * band <= l2;
        const float cost = S * abytes + 8.0f * wslice * (fits ? 1.0f : rounds);
        if (S == 1 || cost < best_cost) best = S, best_cost = cost;
    }
    return best;
}

// 32 x 128 workgroup tiles when the 64 x 128 ones give at most two per CU;
// measured on 750 rows: 1024->4096 (384 tiles) 25.9 -> 23.4 us, 1024->1024
// (96) 17.7 -> 13.3 us; at 6000 rows 1024->1024 (752) 36 -> 40 us and at 1500
// rows 1024->4096 (768) 36.6 -> 39.7 us, so there the 64-row tiles stay. The
// same bits either way.
static bool gemm_narrow(int grid) { return grid <= 512; }

// 64 x 256 workgroup tiles (two column groups per wave, two workgroups per
// CU) for the folded affine K-quants and f32 weights in EXACT numerics when
// there are enough of them: measured at 12000 rows, Q4_K 1024->4096 294 ->
// 278 us, Q2_K 4096->1024 280 -> 264 us (Q5_K 1%; Q3_K, Q8_0 and the A1 forms
// slower); f32 weights 1024->4096 at 6000 rows 176 -> 164 us.
template <int QT, bool A1> constexpr bool wide_fmt() {
    return !A1 && (QT == QT_Q2_K || QT == QT_Q4_K || QT == QT_Q5_K || QT == QT_F32);
}
template <int QT, bool A1>
static bool gemm_wide(const DevW &W, int tilesM, int jobs) {
    // K of two chunks: each tile's start-up is a large part of its work, and the
    // 64 x 128 tiles, three workgroups per CU, hide it better (f32 weights,
    // 256 -> 256 at 480 000 rows: 301 -> 294 us; at 120 000 rows 78 -> 75.5 us)
    if (!wide_fmt<QT, A1>() || W.Np % 256 != 0 || W.Kp < 512) return false;
    const int tw = tilesM * (W.Np / 256) * jobs;
    if (tw < 512) return false;
    // f32 weights: only when the wide tiles (two workgroups per CU) fill their
    // rounds as well as the 64 x 128 ones (three per CU): 2560 -> 1024 at 12 000
    // rows is 752 wide tiles, 1.47 rounds, 228 us, against 198 us in 1504
    // narrow tiles, 1.96 rounds. (Q2_K 4096 -> 1024 at 12 000 rows, the same 752
    // tiles, measured faster wide: 280 -> 264 us; the rule on the Q2_K, Q4_K and
    // Q5_K layer sets: 290-317 against 302-332 TOPS.)
    if (QT == QT_F32) {
        auto fill = [](int t, int slots) { return (double)t / (double)((t + slots - 1) / slots * slots); };
        if (fill(tw, 512) < fill(2 * tw, 768)) return false;
    }
    return true;
}

template <int QT, bool A1>
static hipError_t gemm_launch(const GemmJobs &J, const uint8_t *xp, const float *xs16, const float *xpf, int M,
                              int act, const PrepOut *po, float *ws, hipStream_t st) {
    const DevW &W = J.W[0];
    const int mpad = mh_mpad(M);
    if (mpad % 64 != 0 || W.Np % 128 != 0 || J.n < 1 || J.n > 3) return hipErrorInvalidValue;
    for (int i = 1; i < J.n; i++)
        if (J.W[i].Np != W.Np || J.W[i].Kp != W.Kp || J.W[i].n != W.n) return hipErrorInvalidValue;
    const int tilesM = mpad / 64, tilesN = W.Np / 128, grid = J.n * tilesM * tilesN;
    const int ngrp = gemm_ngroups(w_bpe<QT>() * W.Np * W.Kp * J.n, (A1 ? 2.0f : 4.0f) * mpad * W.Kp, tilesM,
                                  J.n * tilesN);
    if (po) {
        if constexpr (A1) {
            return hipErrorInvalidValue;
        } else {
            if (po->Kc != tilesN || J.n != 1) return hipErrorInvalidValue;
            hipLaunchKernelGGL((k_gemm<QT, EPI_PREP>), dim3(grid), dim3(256), 0, st, J, xp, (const uint8_t *)xs16,
                               xpf, M, 1, tilesM, tilesN, *po, nullptr, 1, ngrp);
            return hipGetLastError();
        }
    }
    const int ks = ws ? gemm_ksplit(W.Kp / 128, grid, (size_t)J.n * mpad * W.Np) : 1;
    if (ks > 1) {
        hipLaunchKernelGGL((k_gemm<QT, EPI_PART, A1>), dim3(grid * ks), dim3(256), 0, st, J, xp,
                           (const uint8_t *)xs16, xpf, M, act, tilesM, tilesN, PrepOut{}, ws, ks, 1);
        const int threads = M * (W.Np / 4);
        hipLaunchKernelGGL((k_gemm_fold<QT>), dim3((threads + 255) / 256, J.n), dim3(256), 0, st, J, (const float *)ws,
                           xpf, M, mpad, act);
    } else if (gemm_narrow(grid)) {
        hipLaunchKernelGGL((k_gemm<QT, EPI_Y, A1, 1, 1>), dim3(2 * grid), dim3(256), 0, st, J, xp,
                           (const uint8_t *)xs16, xpf, M, act, 2 * tilesM, tilesN, PrepOut{}, nullptr, 1, ngrp);
    } else if (gemm_wide<QT, A1>(W, tilesM, J.n)) {
        if constexpr (wide_fmt<QT, A1>()) {   // (the other formats never instantiate it)
            const int tN2 = W.Np / 256, ng2 = gemm_ngroups(w_bpe<QT>() * W.Np * W.Kp * J.n,
                                                          (A1 ? 2.0f : 4.0f) * mpad * W.Kp, tilesM, J.n * tN2);
            hipLaunchKernelGGL((k_gemm<QT, EPI_Y, A1, 2>), dim3(J.n * tilesM * tN2), dim3(256), 0, st, J, xp,
                               (const uint8_t *)xs16, xpf, M, act, tilesM, tN2, PrepOut{}, nullptr, 1, ng2);
        }
    } else {
        hipLaunchKernelGGL((k_gemm<QT, EPI_Y, A1>), dim3(grid), dim3(256), 0, st, J, xp, (const uint8_t *)xs16, xpf,
                           M, act, tilesM, tilesN, PrepOut{}, nullptr, 1, ngrp);
    }
    return hipGetLastError();
}

// a1: the INT8ACT form (int8 activations from mh_launch_prep_a1); the qmat
// formats INT8 / INT4 and f32 weights have none
template <int QT>
static hipError_t gemm_t(const GemmJobs &J, const uint8_t *xp, const float *xs16, const float *xpf, int M,
                         int act, const PrepOut *po, float *ws, hipStream_t st, bool a1 = false) {
    if constexpr (QT == QT_F32 || QT == QT_INT8 || QT == QT_INT4) {
        if (a1) return hipErrorInvalidValue;
        return gemm_launch<QT, false>(J, xp, xs16, xpf, M, act, po, ws, st);
    } else {
        if (a1) return gemm_launch<QT, true>(J, xp, xs16, xpf, M, act, po, ws, st);
        return gemm_launch<QT, false>(J, xp, xs16, xpf, M, act, po, ws, st);
    }
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

hipError_t mh_launch_gemv_jobs(int qtype, const GJobs &J, const float *x, int M, int vec, const GPro &pro,
                               hipStream_t st) {
    if (J.n < 1 || J.n > 3 || (pro.kind != GPRO_NONE && (M != 1 || J.W[0].k > 4096)) ||
        (pro.kind == GPRO_NONE && J.n != 1))
        return hipErrorInvalidValue;
    for (int i = 1; i < J.n; i++)
        if (J.W[i].Np != J.W[0].Np || J.W[i].Kp != J.W[0].Kp || J.W[i].k != J.W[0].k) return hipErrorInvalidValue;
    MH_DISPATCH(gemv_t, qtype, J, x, M, vec, pro, st)
}

// the split-K GEMV: K >= 2048 over at most 64 column groups (N <= 2048)
static bool gemv_split(const DevW &W) { return W.Kp / 128 >= 16 && W.Np / 32 <= 64; }

size_t mh_gemv_ws_floats(const DevW &W) {
    const size_t Kc = W.Kp / 128;
    return gemv_split(W) ? (size_t)(W.Np / 32) * Kc * 512 + Kc * 16 : 0;
}

template <int QT>
static hipError_t gemv_split_t(const DevW &W, const float *x, int M, int vec, float *y, GEpi ep, float *ws,
                               hipStream_t st) {
    constexpr int NW = 4;
    const int Kc = W.Kp / 128, G = W.Np / 32;
    float *part = ws, *pfg = ws + (size_t)G * Kc * 512;
    const dim3 grid(G, (Kc + NW - 1) / NW);
    // chunk results of the rows below M only (the fold reads no other row)
    auto part_k = [&](auto ne) {
        constexpr int NE = decltype(ne)::value;
        if (vec)
            hipLaunchKernelGGL((k_gemv_part<QT, NW, true, NE>), grid, dim3(NW * 64), 0, st, W, x, M, part, pfg);
        else
            hipLaunchKernelGGL((k_gemv_part<QT, NW, false, NE>), grid, dim3(NW * 64), 0, st, W, x, M, part, pfg);
    };
    if (M == 1) part_k(std::integral_constant<int, 1>{});
    else if (M <= 8) part_k(std::integral_constant<int, 4>{});
    else part_k(std::integral_constant<int, 8>{});
    hipLaunchKernelGGL((k_gemv_fold<QT>), dim3(G), dim3(64), 0, st, W, part, pfg, M, y, ep);
    return hipGetLastError();
}

hipError_t mh_launch_gemv_epi(int qtype, const DevW &W, const float *x, int M, int vec, float *y, GEpi ep,
                              float *ws, hipStream_t st) {
    if (ws && gemv_split(W)) {
        MH_DISPATCH(gemv_split_t, qtype, W, x, M, vec, y, ep, ws, st)
    }
    GJobs J{};
    J.W[0] = J.W[1] = J.W[2] = W;
    J.y[0] = y;
    J.ep[0] = ep;
    J.n = 1;
    return mh_launch_gemv_jobs(qtype, J, x, M, vec, GPro{}, st);
}

hipError_t mh_launch_gemv(int qtype, const DevW &W, const float *x, int M, int vec, float *y, int act,
                          float *ws, hipStream_t st) {
    return mh_launch_gemv_epi(qtype, W, x, M, vec, y, GEpi{act, nullptr, nullptr}, ws, st);
}

hipError_t mh_launch_gemm(int qtype, const DevW &W, const uint8_t *xp, const float *xs16,
                          const float *xpf, float *y, int M, int act, float *ws, hipStream_t st, bool a1) {
    GemmJobs J{};
    J.W[0] = J.W[1] = J.W[2] = W;
    J.y[0] = J.y[1] = J.y[2] = y;
    J.n = 1;
    MH_DISPATCH(gemm_t, qtype, J, xp, xs16, xpf, M, act, nullptr, ws, st, a1)
}

hipError_t mh_launch_gemm_jobs(int qtype, const GemmJobs &J, const uint8_t *xp, const float *xs16,
                               const float *xpf, int M, float *ws, hipStream_t st, bool a1) {
    MH_DISPATCH(gemm_t, qtype, J, xp, xs16, xpf, M, 0, nullptr, ws, st, a1)
}

hipError_t mh_launch_gemm_prep_out(int qtype, const DevW &W, const uint8_t *xp, const float *xs16,
                                   const float *xpf, int M, uint8_t *oxp, float *oxs16, float *oxpf, int oKc,
                                   int oxsum, hipStream_t st) {
    const PrepOut po{oxp, (uint8_t *)oxs16, oxpf, oKc, oxsum};
    GemmJobs J{};
    J.W[0] = J.W[1] = J.W[2] = W;
    J.n = 1;
    MH_DISPATCH(gemm_t, qtype, J, xp, xs16, xpf, M, 1, &po, nullptr, st)
}

hipError_t mh_launch_read_floor(const void *p, size_t bytes, hipStream_t st) {
    const size_t n4 = bytes / 16;
    if (n4 == 0) return hipSuccess;
    // enough threads for four float4 each per round, at most 2048 workgroups
    const size_t wgs = (n4 + 4 * 256 - 1) / (4 * 256);
    hipLaunchKernelGGL(k_read_floor, dim3((unsigned)(wgs < 2048 ? wgs : 2048)), dim3(256), 0, st,
                       (const float4 *)p, n4);
    return hipGetLastError();
}

hipError_t mh_launch_prep(const float *x, int M, int K, int Kp, int Mpad, uint8_t *xp, float *xs16,
                          float *xpf, int want_xsum, int vec, hipStream_t st) {
    constexpr int NWP = 1;
    const dim3 grid(Mpad / 32, (Kp / 128 + NWP - 1) / NWP);
    if (vec)
        hipLaunchKernelGGL((k_prep<true, NWP>), grid, dim3(64 * NWP), 0, st, x, M, K, Kp, xp, (uint8_t *)xs16, xpf, want_xsum);
    else
        hipLaunchKernelGGL((k_prep<false, NWP>), grid, dim3(64 * NWP), 0, st, x, M, K, Kp, xp, (uint8_t *)xs16, xpf, want_xsum);
    return hipGetLastError();
}

template <int QT>
static hipError_t launch_dq(const DevW &W, float *out, hipStream_t st) {
    if constexpr (QT == QT_F32) {
        return hipErrorInvalidValue;
    } else {
        hipLaunchKernelGGL((k_dequant<QT>), dim3(W.Kp / 128, W.Np / 32), dim3(64), 0, st, W, out);
        return hipGetLastError();
    }
}

hipError_t mh_launch_dequant(int qtype, const DevW &W, float *out, hipStream_t st) {
    MH_DISPATCH(launch_dq, qtype, W, out, st)
}

bool mh_i8_supported(int qtype) { return qtype != QT_F32; }

int mh_i8_kind(int qtype) {
    if (qtype == QT_INT8 || qtype == QT_INT4) return MH_I8_QMAT;
    if (qtype == QT_Q8_0 || qtype == QT_Q4_0) return MH_I8_ROW;
    return MH_I8_SB;
}

hipError_t mh_launch_prep_a1(int kind, const float *x, int M, int K, int Kp, int Mpad, uint8_t *xp, float *xs16,
                             float *xpf, int want_xsum, hipStream_t st) {
    const bool vec = K % 8 == 0 && ((uintptr_t)x & 15) == 0;
    if (kind == MH_I8_ROW) {
        if (vec && Kp <= 4096) {
            const dim3 g(Mpad / 8);
            if (Kp <= 512) hipLaunchKernelGGL(k_prep_a1_row1<1>, g, dim3(512), 0, st, x, M, K, Kp, Mpad, xp, xpf);
            else if (Kp <= 1024) hipLaunchKernelGGL(k_prep_a1_row1<2>, g, dim3(512), 0, st, x, M, K, Kp, Mpad, xp, xpf);
            else if (Kp <= 2048) hipLaunchKernelGGL(k_prep_a1_row1<4>, g, dim3(512), 0, st, x, M, K, Kp, Mpad, xp, xpf);
            else hipLaunchKernelGGL(k_prep_a1_row1<8>, g, dim3(512), 0, st, x, M, K, Kp, Mpad, xp, xpf);
        } else if (vec)
            hipLaunchKernelGGL(k_prep_a1_row<true>, dim3(Mpad / 32), dim3(PREP_I8_NW * 64), 0, st, x, M, K, Kp, xp, xpf);
        else
            hipLaunchKernelGGL(k_prep_a1_row<false>, dim3(Mpad / 32), dim3(PREP_I8_NW * 64), 0, st, x, M, K, Kp, xp, xpf);
    } else if (kind == MH_I8_SB) {
        if (Kp % 256 != 0) return hipErrorInvalidValue;
        const dim3 grid(Mpad / 32, Kp / 256);
        if (vec)
            hipLaunchKernelGGL(k_prep_a1_sb<true>, grid, dim3(64), 0, st, x, M, K, Kp, xp, (uint8_t *)xs16, xpf, want_xsum);
        else
            hipLaunchKernelGGL(k_prep_a1_sb<false>, grid, dim3(64), 0, st, x, M, K, Kp, xp, (uint8_t *)xs16, xpf, want_xsum);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t mh_launch_prep_i8(const float *x, int M, int K, int Kp, int Mpad, uint8_t *qx, float *sx, float *inv,
                             hipStream_t st) {
    const dim3 gq(Mpad / 32, (Kp / 32 + 3) / 4);
    const bool vec = K % 8 == 0 && ((uintptr_t)x & 15) == 0;
    if (vec && Kp <= 4096) {
        const dim3 g(Mpad / 8);
        if (Kp <= 1024) hipLaunchKernelGGL(k_prep_i8_row<1>, g, dim3(512), 0, st, x, M, K, Kp, Mpad, qx, sx);
        else if (Kp <= 2048) hipLaunchKernelGGL(k_prep_i8_row<2>, g, dim3(512), 0, st, x, M, K, Kp, Mpad, qx, sx);
        else hipLaunchKernelGGL(k_prep_i8_row<4>, g, dim3(512), 0, st, x, M, K, Kp, Mpad, qx, sx);
    } else if (vec) {
        hipLaunchKernelGGL(k_rowscale_i8<true>, dim3(Mpad / 4), dim3(256), 0, st, x, M, K, Mpad, sx, inv);
        hipLaunchKernelGGL(k_quant_i8<true>, gq, dim3(256), 0, st, x, M, K, Kp, qx, inv);
    } else {
        hipLaunchKernelGGL(k_rowscale_i8<false>, dim3(Mpad / 4), dim3(256), 0, st, x, M, K, Mpad, sx, inv);
        hipLaunchKernelGGL(k_quant_i8<false>, gq, dim3(256), 0, st, x, M, K, Kp, qx, inv);
    }
    return hipGetLastError();
}

template <int QT, int WM>
static hipError_t launch_i8(const DevW &W, const uint8_t *qx, const float *sx, float *y, int M, int act,
                            hipStream_t st) {
    const int mpad = mh_mpad(M);
    if (mpad % (32 * WM) != 0) return hipErrorInvalidValue;
    hipLaunchKernelGGL((k_gemm_i8<QT, WM>), dim3(W.Np / 128, mpad / (32 * WM)), dim3(256), 0, st, W, qx, sx, y,
                       M, act);
    return hipGetLastError();
}

// the tiled INT8 product, tile TR x 4 CW groups of 32
template <int TR, int CW>
static hipError_t launch_i8t(const DevW &W, const uint8_t *qx, const float *sx, float *y, int M, int act,
                             hipStream_t st) {
    const int tilesM = (mh_mpad(M) / 32 + TR - 1) / TR, tilesN = (W.Np / 32 + 4 * CW - 1) / (4 * CW);
    hipLaunchKernelGGL((k_gemm_i8t<TR, CW, 4>), dim3(tilesM * tilesN), dim3(256), 0, st, W, qx, sx, y, M, act,
                       tilesM, tilesN);
    return hipGetLastError();
}

// work on the busiest CU, in tile units of 32 x 32, for tiles of tr x tc
// groups dealt over the 256 CUs
static long i8t_makespan(int M, int Np, int tr, int tc) {
    const long tiles = (long)((mh_mpad(M) / 32 + tr - 1) / tr) * ((Np / 32 + tc - 1) / tc);
    return (tiles + 255) / 256 * tr * tc;
}

template <int QT>
static hipError_t gemm_i8_t(const DevW &W, const uint8_t *qx, const float *sx, float *y, int M, int act,
                            hipStream_t st) {
    if (QT == QT_INT8 && M > 64) {
        // 96 x 256 or 64 x 256 tiles, whichever leaves less on the busiest CU
        if (i8t_makespan(M, W.Np, 3, 8) <= i8t_makespan(M, W.Np, 2, 8))
            return launch_i8t<3, 2>(W, qx, sx, y, M, act, st);
        return launch_i8t<2, 2>(W, qx, sx, y, M, act, st);
    }
    if (M <= 64 || mh_mpad(M) % 64 != 0) return launch_i8<QT, 1>(W, qx, sx, y, M, act, st);
    return launch_i8<QT, 2>(W, qx, sx, y, M, act, st);
}

hipError_t mh_launch_gemm_i8(int qtype, const DevW &W, const uint8_t *qx, const float *sx, float *y, int M,
                             int act, hipStream_t st) {
    switch (qtype) {
    case QT_INT8: return gemm_i8_t<QT_INT8>(W, qx, sx, y, M, act, st);
    case QT_INT4: return gemm_i8_t<QT_INT4>(W, qx, sx, y, M, act, st);
    case QT_Q8_0: return gemm_i8_t<QT_Q8_0>(W, qx, sx, y, M, act, st);
    case QT_Q4_0: return gemm_i8_t<QT_Q4_0>(W, qx, sx, y, M, act, st);
    }
    return hipErrorInvalidValue;
}

hipError_t mh_launch_silu(float *x, size_t n, hipStream_t st) {
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_silu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, x, n);
    return hipGetLastError();
}
