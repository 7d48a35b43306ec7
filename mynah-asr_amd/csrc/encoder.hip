// encoder.hip — the steps of one FastConformer encoder layer around its
// products and its attention core (src/encoder.c:485-521 and the batched form
// :901-946): the layer norms with the residual add that precedes each of
// them, the GLU, and the depthwise convolution with its conv norm and SiLU
// (conv_module, :413-462).
//
//   k_add_ln    x += alpha * res (when res), then out = LN(x) per row
//               (layer_norm_f, :25-37; the adds of :495, 502, 507, 511)
//   k_add_ln_prep  the same, its output written as the products' prepared
//               input (EXACT numerics) instead of f32 rows
//   k_glu       g = a * sigmoid(b) over the two halves of each row  :426-432
//   k_dwconv    depthwise conv over time within each segment (causal: left
//               pad k-1; else 'same'), + dw_b, then the folded batch norm
//               x * scale + shift and SiLU when scale is given     :434-459
//   k_dwconv_tile  the same on LDS tiles of 32 rows, optionally forming the
//               GLU as it stages its input
//
// and of the dw_striding subsampling in front of the layers
// (src/subsampling.c:208-268, 109-200), with activations channel-last,
// [segment][time][freq][channel], so that its pointwise convolutions and its
// final linear are this unit's products:
//   k_conv_in_dw  the full 3x3 stride-2 conv of the mel features, 1 -> C
//               channels, + bias, ReLU (:222-226), fused into the first
//               depthwise 3x3 stride-2 conv, + bias (:231-236)
//   k_dw_s2     the depthwise 3x3 stride-2 conv, + bias; its input takes
//               the previous pointwise conv's bias and ReLU on load  :237-244
//   k_flatten   the last pointwise conv's bias and ReLU, then the
//               channel-major flatten [t][c * F' + f] of :249-257
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "fmt.h"
#include "launch.h"

namespace {

// the reference's stable sigmoid (src/qmat.h:31-35): exp only of -|x|
__device__ __forceinline__ float sigmoid_f(float x) {
    if (x >= 0.0f) return 1.0f / (1.0f + expf(-x));
    const float e = expf(x);
    return e / (1.0f + e);
}

// One wave per row of d = 256 V4 floats (lane l holds elements 4l + 256u ..
// +3): x += alpha res (stored; res may be null), then the layer norm into
// v. Sums in double in two passes, as layer_norm_f: mean, then the sum of
// (x - mean)^2; inv = (float)(1 / sqrt(var + 1e-5)); v = ((x - (float)mean)
// * inv) * w + b in f32.
template <int V4>
__device__ __forceinline__ void add_ln_row(float *xr, const float *__restrict__ rr, float alpha,
                                           const float *__restrict__ w, const float *__restrict__ b, int lane,
                                           float4 (&v)[V4]) {
    constexpr int d = 256 * V4;
    float4 wv[V4], bv[V4];
#pragma unroll
    for (int u = 0; u < V4; u++) {
        const int i = 4 * lane + 256 * u;
        v[u] = *(const float4 *)(xr + i);
        wv[u] = *(const float4 *)(w + i);
        bv[u] = *(const float4 *)(b + i);
    }
    if (rr) {
#pragma unroll
        for (int u = 0; u < V4; u++) {
            const float4 a = *(const float4 *)(rr + 4 * lane + 256 * u);
            v[u].x = fmaf(alpha, a.x, v[u].x);
            v[u].y = fmaf(alpha, a.y, v[u].y);
            v[u].z = fmaf(alpha, a.z, v[u].z);
            v[u].w = fmaf(alpha, a.w, v[u].w);
            *(float4 *)(xr + 4 * lane + 256 * u) = v[u];
        }
    }
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < V4; u++) s += ((double)v[u].x + (double)v[u].y) + ((double)v[u].z + (double)v[u].w);
    for (int o = 32; o > 0; o >>= 1) s += __shfl_xor(s, o, 64);
    const double mu = s / d;
    double q = 0.0;
#pragma unroll
    for (int u = 0; u < V4; u++) {
        const double c0 = (double)v[u].x - mu, c1 = (double)v[u].y - mu;
        const double c2 = (double)v[u].z - mu, c3 = (double)v[u].w - mu;
        q += (c0 * c0 + c1 * c1) + (c2 * c2 + c3 * c3);
    }
    for (int o = 32; o > 0; o >>= 1) q += __shfl_xor(q, o, 64);
    const float inv = (float)(1.0 / sqrt(q / d + 1e-5));
    const float muf = (float)mu;
#pragma unroll
    for (int u = 0; u < V4; u++) {
        v[u].x = ((v[u].x - muf) * inv) * wv[u].x + bv[u].x;
        v[u].y = ((v[u].y - muf) * inv) * wv[u].y + bv[u].y;
        v[u].z = ((v[u].z - muf) * inv) * wv[u].z + bv[u].z;
        v[u].w = ((v[u].w - muf) * inv) * wv[u].w + bv[u].w;
    }
}

// out = LN(x += alpha res), one wave per row. out may be x.
template <int V4>
__global__ __launch_bounds__(256) void k_add_ln(float *x, const float *__restrict__ res, float alpha,
                                                const float *__restrict__ w, const float *__restrict__ b,
                                                float *out, int rows) {
    constexpr int d = 256 * V4;
    const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    if (r >= rows) return;
    float4 v[V4];
    add_ln_row<V4>(x + (size_t)r * d, res ? res + (size_t)r * d : nullptr, alpha, w, b, lane, v);
    float *orow = out + (size_t)r * d;
#pragma unroll
    for (int u = 0; u < V4; u++) *(float4 *)(orow + 4 * lane + 256 * u) = v[u];
}

// LN(x += alpha res) as the products' prepared input in EXACT numerics, in
// place of the f32 rows: the split of each row's 128-element chunks that the
// products' preparation forms (the same values: shift sh from the chunk's
// largest magnitude, hi = f16(v 2^sh), lo = f16(v 2^sh - hi), fold factor
// 2^-sh), in its layout
//   xp   [row group G][chunk][half-step u][hi, lo][64 slots][16 B], slot r + 32 hh
//        holding chunk elements 16u + 8hh .. +7 of row 32G + r
//   xpf  [G][chunk][32]
// Lane l's float4 u is chunk 2u + l / 32, elements 4 (l % 32) .. +3: half-step
// (l % 32) / 4, half hh = (l / 2) % 2, the 8-byte half l % 2 of the slot. A
// workgroup holds 8 consecutive rows (8 waves): for each (chunk, half-step,
// term, hh) their slots are one 128-byte line of xp. The pieces go to LDS
// first, in that line order, so that the stores to xp are whole lines (a
// wave's store covers 8 of them). Rows rows .. Mpad-1 are the zero rows the
// preparation pads with (fold factor 1).
template <int V4>
__global__ __launch_bounds__(512) void k_add_ln_prep(float *x, const float *__restrict__ res, float alpha,
                                                     const float *__restrict__ w, const float *__restrict__ b,
                                                     int rows, uint8_t *__restrict__ xp, float *__restrict__ xpf) {
    constexpr int d = 256 * V4, Kc = d / 128, NL = Kc * 32;   // lines of the workgroup
    __shared__ uint4 stage[NL * 8];
    const int wave = threadIdx.x >> 6, m = blockIdx.x * 8 + wave, lane = threadIdx.x & 63;
    const int G = m >> 5, r = m & 31, l32 = lane & 31;
    float4 v[V4];
    if (m < rows) {
        add_ln_row<V4>(x + (size_t)m * d, res ? res + (size_t)m * d : nullptr, alpha, w, b, lane, v);
    } else {
#pragma unroll
        for (int u = 0; u < V4; u++) v[u] = float4{0.f, 0.f, 0.f, 0.f};
    }
    const int hu = l32 >> 2, hh = (l32 >> 1) & 1;
#pragma unroll
    for (int u = 0; u < V4; u++) {
        const int c = 2 * u + (lane >> 5);
        float a = fmaxf(fmaxf(fabsf(v[u].x), fabsf(v[u].y)), fmaxf(fabsf(v[u].z), fabsf(v[u].w)));
#pragma unroll
        for (int o = 16; o > 0; o >>= 1) a = fmaxf(a, __shfl_xor(a, o, 64));
        const int sh = chunk_shift(a);
        const float xs[4] = {ldexpf(v[u].x, sh), ldexpf(v[u].y, sh), ldexpf(v[u].z, sh), ldexpf(v[u].w, sh)};
        _Float16 hv[4], lv[4];
#pragma unroll
        for (int j = 0; j < 4; j++) {
            hv[j] = (_Float16)xs[j];
            lv[j] = (_Float16)(xs[j] - (float)hv[j]);
        }
        uint2 hw, lw;
        __builtin_memcpy(&hw, hv, 8);
        __builtin_memcpy(&lw, lv, 8);
        // line ((c * 8 + hu) * 2 + term) * 2 + hh, slot wave (the row within the 8)
        uint8_t *o = (uint8_t *)stage + (((((c * 8 + hu) * 2) * 2 + hh) * 8 + wave) * 16 + 8 * (lane & 1));
        *(uint2 *)o = hw;
        *(uint2 *)(o + 2 * 8 * 16) = lw;
        if (l32 == 0) xpf[((size_t)G * Kc + c) * 32 + r] = ldexpf(1.0f, -sh);
    }
    __syncthreads();
    // line L = (q * 2 + hh), q = (c * 8 + hu) * 2 + term, lies at xp offset
    // (G * Kc * 16 + q) * 1024 + hh * 512 + (8-row block) * 128
    const int rb = (blockIdx.x & 3) * 128;
    uint8_t *gx = xp + (size_t)(blockIdx.x >> 2) * Kc * 16 * 1024 + rb;
#pragma unroll
    for (int i = threadIdx.x; i < NL * 8; i += 512) {
        const int L = i >> 3, sl = i & 7;
        *(uint4 *)(gx + (size_t)(L >> 1) * 1024 + (L & 1) * 512 + sl * 16) = stage[i];
    }
}

// g[r, i] = h[r, i] * sigmoid(h[r, d + i]); thread = 4 elements
__global__ __launch_bounds__(256) void k_glu(const float *__restrict__ h, float *__restrict__ g, size_t rows,
                                             int d) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x, d4 = d / 4;
    if (idx >= rows * d4) return;
    const size_t r = idx / d4, i = 4 * (idx - r * d4);
    const float4 a = *(const float4 *)(h + r * 2 * d + i), b = *(const float4 *)(h + r * 2 * d + d + i);
    const float4 o = {a.x * sigmoid_f(b.x), a.y * sigmoid_f(b.y), a.z * sigmoid_f(b.z), a.w * sigmoid_f(b.w)};
    *(float4 *)(g + r * d + i) = o;
}

// x * sigmoid(x) with the stable sigmoid (mynah_asr_silu)
__device__ __forceinline__ float silu_e(float x) { return x * sigmoid_f(x); }

// c[t, i] = dw_b[i] + sum_j w[i, j] * g[t - pc + j, i] over the taps inside
// the segment (in tap order from j0), then, with scale: silu(c * scale +
// shift). Thread = (row, 4 channels); the weights in the reference's order
// w[i][j] (the fallback for shapes the tiled form does not take).
__global__ __launch_bounds__(256) void k_dwconv(const float *__restrict__ g, const float *__restrict__ w,
                                                const float *__restrict__ bias, const float *__restrict__ scale,
                                                const float *__restrict__ shift, float *__restrict__ out, int T,
                                                int nseq, int d, int k, int pc) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int d4 = d / 4;
    if (idx >= (size_t)nseq * T * d4) return;
    const int row = (int)(idx / d4), i = 4 * (int)(idx - (size_t)row * d4);
    const int s = row / T, t = row - s * T;
    const float *gs = g + (size_t)s * T * d;
    float4 o = bias ? *(const float4 *)(bias + i) : float4{0.f, 0.f, 0.f, 0.f};
    const int j0 = t - pc < 0 ? pc - t : 0, j1 = t - pc + k > T ? T - t + pc : k;
    for (int j = j0; j < j1; j++) {
        const float4 src = *(const float4 *)(gs + (size_t)(t - pc + j) * d + i);
        const float *wj = w + (size_t)i * k + j;
        const float4 wv = {wj[0], wj[k], wj[2 * k], wj[3 * k]};
        o.x = fmaf(wv.x, src.x, o.x);
        o.y = fmaf(wv.y, src.y, o.y);
        o.z = fmaf(wv.z, src.z, o.z);
        o.w = fmaf(wv.w, src.w, o.w);
    }
    if (scale) {
        const float4 sc = *(const float4 *)(scale + i), sh = *(const float4 *)(shift + i);
        o.x = silu_e(fmaf(o.x, sc.x, sh.x));
        o.y = silu_e(fmaf(o.y, sc.y, sh.y));
        o.z = silu_e(fmaf(o.z, sc.z, sh.z));
        o.w = silu_e(fmaf(o.w, sc.w, sh.w));
    }
    *(float4 *)(out + (size_t)row * d + i) = o;
}

// The same in tiles: a workgroup = DW_R rows of one segment x 256 channels.
// The rows t0 - pc .. t0 + DW_R - 1 - pc + k - 1 of g (zero outside the
// segment) and the k taps are staged in LDS once, so each input row is read
// from memory once per tile instead of once per tap; thread = (4 channels,
// every 4th row of the tile). Per output the operations and their order are
// those of k_dwconv (taps outside the segment skipped, not added as zeros).
// GLU: g is formed from pw1's output h [rows][2d] as it is staged (k_glu's
// operations; the halo rows' values are formed again by the next tile).
constexpr int DW_R = 32;
// PREP: the output rows are written as the EXACT products' prepared input
// (xp, xpf, for M = nseq T rows padded to 64, as k_add_ln_prep writes it)
// instead of into out: per (row, 128-channel chunk: 32 lanes) the split the
// preparation forms, held in registers until the tile is done, then staged
// in the input rows' LDS so the stores run along rows.
template <bool GLU, bool PREP>
__global__ __launch_bounds__(256) void k_dwconv_tile(const float *__restrict__ g, const float *__restrict__ w,
                                                     const float *__restrict__ bias, const float *__restrict__ scale,
                                                     const float *__restrict__ shift, float *__restrict__ out,
                                                     int T, int d, int k, int pc, uint8_t *__restrict__ xp,
                                                     float *__restrict__ xpf) {
    // [DW_R + k - 1][64] rows of g, then [k][64] taps; PREP, once the tile is
    // done: the staged slots [DW_R rows][2 chunks][8 half-steps][2 terms][2
    // halves] over the rows, the fold factors [DW_R][2] over the taps
    extern __shared__ float4 dws[];
    uint2 ph[PREP ? DW_R / 4 : 1], pl[PREP ? DW_R / 4 : 1];
    float pf[PREP ? DW_R / 4 : 1];
    const int tid = threadIdx.x, q = tid & 63, t0 = blockIdx.x * DW_R, c0 = blockIdx.y * 256;
    const int nrow = DW_R + k - 1;
    const int gw = GLU ? 2 * d : d;   // the input's row width
    const float *gs = g + (size_t)blockIdx.z * T * gw + c0;
    float4 *taps = dws + nrow * 64;
    for (int i = tid; i < nrow * 64; i += 256) {
        const int t = t0 - pc + (i >> 6);
        float4 o = {0.f, 0.f, 0.f, 0.f};
        if (t >= 0 && t < T) {
            const float *p = gs + (size_t)t * gw + 4 * (i & 63);
            o = *(const float4 *)p;
            if constexpr (GLU) {
                const float4 b = *(const float4 *)(p + d);
                o = float4{o.x * sigmoid_f(b.x), o.y * sigmoid_f(b.y), o.z * sigmoid_f(b.z), o.w * sigmoid_f(b.w)};
            }
        }
        dws[i] = o;
    }
    // the taps of w [d][k] written tap-major (each tap of 4 channels one
    // float4): thread = channel c0 + tid, its k taps
    {
        float *tf = (float *)taps;
        const float *wc = w + (size_t)(c0 + tid) * k;
        for (int j = 0; j < k; j++) tf[j * 256 + tid] = wc[j];
    }
    __syncthreads();
    const int i = c0 + 4 * q;
    const float4 b0 = bias ? *(const float4 *)(bias + i) : float4{0.f, 0.f, 0.f, 0.f};
    float4 sc = {0.f, 0.f, 0.f, 0.f}, sh = sc;
    if (scale) {
        sc = *(const float4 *)(scale + i);
        sh = *(const float4 *)(shift + i);
    }
    float *os = out + (size_t)blockIdx.z * T * d + i;
#pragma unroll
    for (int u = 0; u < DW_R / 4; u++) {
        const int rr = (tid >> 6) + 4 * u, t = t0 + rr;
        if (t >= T) break;
        const int j0 = t - pc < 0 ? pc - t : 0, j1 = t - pc + k > T ? T - t + pc : k;
        float4 o = b0;
        for (int j = j0; j < j1; j++) {
            const float4 src = dws[(rr + j) * 64 + q], wv = taps[j * 64 + q];
            o.x = fmaf(wv.x, src.x, o.x);
            o.y = fmaf(wv.y, src.y, o.y);
            o.z = fmaf(wv.z, src.z, o.z);
            o.w = fmaf(wv.w, src.w, o.w);
        }
        if (scale) {
            o.x = silu_e(fmaf(o.x, sc.x, sh.x));
            o.y = silu_e(fmaf(o.y, sc.y, sh.y));
            o.z = silu_e(fmaf(o.z, sc.z, sh.z));
            o.w = silu_e(fmaf(o.w, sc.w, sh.w));
        }
        if constexpr (PREP) {
            // lanes 32 cl .. 32 cl + 31 hold chunk cl's 128 channels of row t
            float a = fmaxf(fmaxf(fabsf(o.x), fabsf(o.y)), fmaxf(fabsf(o.z), fabsf(o.w)));
#pragma unroll
            for (int off = 16; off > 0; off >>= 1) a = fmaxf(a, __shfl_xor(a, off, 64));
            const int shf = chunk_shift(a);
            const float xs[4] = {ldexpf(o.x, shf), ldexpf(o.y, shf), ldexpf(o.z, shf), ldexpf(o.w, shf)};
            _Float16 hv[4], lv[4];
#pragma unroll
            for (int j = 0; j < 4; j++) {
                hv[j] = (_Float16)xs[j];
                lv[j] = (_Float16)(xs[j] - (float)hv[j]);
            }
            __builtin_memcpy(&ph[u], hv, 8);
            __builtin_memcpy(&pl[u], lv, 8);
            pf[u] = ldexpf(1.0f, -shf);
        } else {
            *(float4 *)(os + (size_t)t * d) = o;
        }
    }
    if constexpr (PREP) {
        __syncthreads();   // every wave is done with the input rows and the taps
        float4 *stage = dws;
        float *fold = (float *)taps;
        {
            const int l32 = q & 31, cl = q >> 5, hu = l32 >> 2, hh = (l32 >> 1) & 1;
#pragma unroll
            for (int u = 0; u < DW_R / 4; u++) {
                const int rr = (tid >> 6) + 4 * u;
                if (t0 + rr >= T) break;
                uint8_t *o8 = (uint8_t *)(stage + (((rr * 2 + cl) * 8 + hu) * 2) * 2 + hh) + 8 * (l32 & 1);
                *(uint2 *)o8 = ph[u];
                *(uint2 *)(o8 + 2 * 16) = pl[u];   // term 1: two slots on
                if (l32 == 0) fold[rr * 2 + cl] = pf[u];
            }
        }
        __syncthreads();
        const int Kc = d / 128;
        const size_t mb = (size_t)blockIdx.z * T;
        // 2048 slots; consecutive threads run along the 32 rows
        for (int p = tid; p < DW_R * 64; p += 256) {
            const int rr = p & 31, rest = p >> 5;
            const int cl = rest >> 5, hu = (rest >> 2) & 7, term = (rest >> 1) & 1, hh = rest & 1;
            const int t = t0 + rr;
            if (t < T) {
                const size_t m = mb + t;
                const int chunk = 2 * blockIdx.y + cl;
                *(float4 *)(xp + ((((m >> 5) * Kc + chunk) * 8 + hu) * 2 * 64 + term * 64 + (m & 31) + 32 * hh) * 16) =
                    stage[(((rr * 2 + cl) * 8 + hu) * 2 + term) * 2 + hh];
            }
        }
        if (tid < 64) {
            const int rr = tid & 31, cl = tid >> 5, t = t0 + rr;
            if (t < T) {
                const size_t m = mb + t;
                xpf[((m >> 5) * Kc + 2 * blockIdx.y + cl) * 32 + (m & 31)] = fold[rr * 2 + cl];
            }
        }
        // the rows past M up to the 64-row padding: zeros (fold factor 1), as
        // the preparation pads; by the last tile of the last segment
        if (blockIdx.z == gridDim.z - 1 && blockIdx.x == gridDim.x - 1) {
            const size_t M = (size_t)gridDim.z * T, Mp = (M + 63) / 64 * 64;
            for (size_t i = tid; i < (Mp - M) * 64; i += 256) {
                const size_t m = M + (i >> 6);
                const int rest = (int)(i & 63), cl = rest >> 5, hu = (rest >> 2) & 7, term = (rest >> 1) & 1,
                          hh = rest & 1;
                const int chunk = 2 * blockIdx.y + cl;
                *(float4 *)(xp + ((((m >> 5) * Kc + chunk) * 8 + hu) * 2 * 64 + term * 64 + (m & 31) + 32 * hh) * 16) =
                    float4{0.f, 0.f, 0.f, 0.f};
                if (rest == 0 || rest == 32) xpf[((m >> 5) * Kc + chunk) * 32 + (m & 31)] = 1.0f;
            }
        }
    }
}

// The first two stages in one pass: out[s][to][fo][c] = the depthwise 3x3
// stride-2 conv (+ b1) of y = relu(conv_in(x) + b0), the 1 -> C 3x3 stride-2
// conv of the mel features (subsampling.c:222-226, 231-236). y is formed
// where a depthwise tap reads it and never stored (at config 5 it would be
// 2 GB written and read back). Per tap the operations are those of the
// conv alone (nine fmas from zero in tap order, + b0, ReLU) and of the
// depthwise conv (a product, then eight fmas, + b1 last); a tap outside
// y's [T1, F1] reads zero (the depthwise conv's pad), and a mel sample
// outside [T, F] reads zero (the first conv's pad).
//
// One wave per output row (s, to), its lanes over the channels 4 at a time,
// sliding along fo: the 3 x 3 window of y a depthwise output reads stays in
// registers, and each step forms y's two new columns (y column 2 of one
// step is column 0 of the next). The mel samples are wave-uniform and read
// through the scalar cache; each lane holds its channels' 2 x 9 taps.
// Weights tap-major, w0[j][C] and w1[j][C].
__global__ __launch_bounds__(256) void k_conv_in_dw(const float *__restrict__ x, const float *__restrict__ w0,
                                                    const float *__restrict__ b0, const float *__restrict__ w1,
                                                    const float *__restrict__ b1, float *__restrict__ out, int nseq,
                                                    int T, int F, int T1, int F1, int To, int Fo, int C, int pl) {
    const int wrow = __builtin_amdgcn_readfirstlane((int)blockIdx.x * 4 + (int)(threadIdx.x >> 6));
    if (wrow >= nseq * To) return;
    const int lane = threadIdx.x & 63;
    const int to = wrow % To, s = wrow / To;
    const float *xs = x + (size_t)s * T * F;
    for (int c = 4 * lane; c < C; c += 256) {
        float4 wa[9], wb[9];
#pragma unroll
        for (int j = 0; j < 9; j++) {
            wa[j] = *(const float4 *)(w0 + (size_t)j * C + c);
            wb[j] = *(const float4 *)(w1 + (size_t)j * C + c);
        }
        const float4 bb0 = *(const float4 *)(b0 + c), bb1 = *(const float4 *)(b1 + c);
        // y at (t1 = 2 to - pl + r, f1): relu(b0 + conv_in), zero outside [T1, F1]
        auto yat = [&](int r, int f1) {
            const int t1 = 2 * to - pl + r;
            float4 y = {0.f, 0.f, 0.f, 0.f};
            if (t1 >= 0 && t1 < T1 && f1 >= 0 && f1 < F1) {
                float4 ci = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int dt = 0; dt < 3; dt++)
#pragma unroll
                    for (int df = 0; df < 3; df++) {
                        const int t = 2 * t1 - pl + dt, f = 2 * f1 - pl + df;
                        const float v = t >= 0 && t < T && f >= 0 && f < F ? xs[(size_t)t * F + f] : 0.0f;
                        const float4 wv = wa[3 * dt + df];
                        ci.x = fmaf(wv.x, v, ci.x);
                        ci.y = fmaf(wv.y, v, ci.y);
                        ci.z = fmaf(wv.z, v, ci.z);
                        ci.w = fmaf(wv.w, v, ci.w);
                    }
                y = float4{fmaxf(ci.x + bb0.x, 0.0f), fmaxf(ci.y + bb0.y, 0.0f), fmaxf(ci.z + bb0.z, 0.0f),
                           fmaxf(ci.w + bb0.w, 0.0f)};
            }
            return y;
        };
        float4 yw[3][3];
#pragma unroll
        for (int r = 0; r < 3; r++) yw[r][2] = yat(r, -pl);
        for (int fo = 0; fo < Fo; fo++) {
#pragma unroll
            for (int r = 0; r < 3; r++) {
                yw[r][0] = yw[r][2];
                yw[r][1] = yat(r, 2 * fo - pl + 1);
                yw[r][2] = yat(r, 2 * fo - pl + 2);
            }
            float4 acc = {wb[0].x * yw[0][0].x, wb[0].y * yw[0][0].y, wb[0].z * yw[0][0].z, wb[0].w * yw[0][0].w};
#pragma unroll
            for (int j = 1; j < 9; j++) {
                const float4 wv = wb[j], y = yw[j / 3][j % 3];
                acc.x = fmaf(wv.x, y.x, acc.x);
                acc.y = fmaf(wv.y, y.y, acc.y);
                acc.z = fmaf(wv.z, y.z, acc.z);
                acc.w = fmaf(wv.w, y.w, acc.w);
            }
            *(float4 *)(out + ((size_t)wrow * Fo + fo) * C + c) =
                float4{bb1.x + acc.x, bb1.y + acc.y, bb1.z + acc.z, bb1.w + acc.w};
        }
    }
}

// out[s][to][fo][c] = b[c] + sum w[c][3 dt + df] in[s][2 to - pl + dt][2 fo - pl + df][c],
// in the reference's term order (the nine products summed left to right,
// subsampling.c:96-98); with pb, each input value is relu(in + pb[c]) first.
// The weights tap-major, wt[j][c].
__global__ __launch_bounds__(256) void k_dw_s2(const float *__restrict__ in, const float *__restrict__ pb,
                                               const float *__restrict__ wt, const float *__restrict__ b,
                                               float *__restrict__ out, int nseq, int T, int F, int To, int Fo,
                                               int C, int pl) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int C4 = C / 4;
    if (idx >= (size_t)nseq * To * Fo * C4) return;
    const size_t row = idx / C4;
    const int c = 4 * (int)(idx - row * C4);
    const int fo = (int)(row % Fo), to = (int)((row / Fo) % To), s = (int)(row / ((size_t)Fo * To));
    const float *is = in + (size_t)s * T * F * C;
    const float4 pbv = pb ? *(const float4 *)(pb + c) : float4{0.f, 0.f, 0.f, 0.f};
    float4 v[9];
#pragma unroll
    for (int dt = 0; dt < 3; dt++)
#pragma unroll
        for (int df = 0; df < 3; df++) {
            const int t = 2 * to - pl + dt, f = 2 * fo - pl + df;
            float4 a = {0.f, 0.f, 0.f, 0.f};
            if (t >= 0 && t < T && f >= 0 && f < F) {
                a = *(const float4 *)(is + ((size_t)t * F + f) * C + c);
                if (pb) {
                    a.x = fmaxf(a.x + pbv.x, 0.0f);
                    a.y = fmaxf(a.y + pbv.y, 0.0f);
                    a.z = fmaxf(a.z + pbv.z, 0.0f);
                    a.w = fmaxf(a.w + pbv.w, 0.0f);
                }
            }
            v[3 * dt + df] = a;
        }
    float4 wv = *(const float4 *)(wt + c);
    float4 acc = {wv.x * v[0].x, wv.y * v[0].y, wv.z * v[0].z, wv.w * v[0].w};
#pragma unroll
    for (int j = 1; j < 9; j++) {
        wv = *(const float4 *)(wt + (size_t)j * C + c);
        acc.x = fmaf(wv.x, v[j].x, acc.x);
        acc.y = fmaf(wv.y, v[j].y, acc.y);
        acc.z = fmaf(wv.z, v[j].z, acc.z);
        acc.w = fmaf(wv.w, v[j].w, acc.w);
    }
    const float4 bb = *(const float4 *)(b + c);
    *(float4 *)(out + row * C + c) = float4{bb.x + acc.x, bb.y + acc.y, bb.z + acc.z, bb.w + acc.w};
}

// flat[s * To + t][c * Fo + f] = relu(in[s][t][f][c] + pb[c]); thread = one
// output element, consecutive threads along f then c (coalesced writes)
__global__ __launch_bounds__(256) void k_flatten(const float *__restrict__ in, const float *__restrict__ pb,
                                                 float *__restrict__ flat, size_t rows, int Fo, int C) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    const size_t CF = (size_t)C * Fo;
    if (idx >= rows * CF) return;
    const size_t r = idx / CF;
    const int j = (int)(idx - r * CF), c = j / Fo, f = j - c * Fo;
    const float v = in[(r * Fo + f) * C + c] + pb[c];
    flat[idx] = v < 0.0f ? 0.0f : v;
}

// wt[j][c] = w[c][j] for w [C][k]: the per-channel taps tap-major
__global__ __launch_bounds__(256) void k_transpose(const float *__restrict__ w, float *__restrict__ wt, int C,
                                                   int k) {
    const int idx = blockIdx.x * 256 + threadIdx.x;
    if (idx >= C * k) return;
    const int j = idx / C, c = idx - j * C;
    wt[idx] = w[(size_t)c * k + j];
}

// y[r][i] = (y[r][i] + b[i]) * scale (the subsampling's linear bias, then
// the layer input scale: encoder.c:958-959)
__global__ __launch_bounds__(256) void k_bias_scale(float *__restrict__ y, const float *__restrict__ b, size_t rows,
                                                    int d, float scale) {
    const size_t idx = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= rows * d) return;
    const int i = (int)(idx % d);
    const float v = y[idx] + b[i];
    y[idx] = scale != 1.0f ? v * scale : v;
}

}  // namespace

// the widths k_add_ln is instantiated for: 256 V4 with V4 = 1..8, 12, 16
bool mh_enc_d_supported(int d) {
    if (d <= 0 || d % 256) return false;
    const int v = d / 256;
    return v <= 8 || v == 12 || v == 16;
}

hipError_t mh_launch_add_ln(float *x, const float *res, float alpha, const float *w, const float *b, float *out,
                            int rows, int d, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (!mh_enc_d_supported(d)) return hipErrorInvalidValue;
    const dim3 grid((rows + 3) / 4), blk(256);
    switch (d / 256) {
    case 1: hipLaunchKernelGGL(k_add_ln<1>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 2: hipLaunchKernelGGL(k_add_ln<2>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 3: hipLaunchKernelGGL(k_add_ln<3>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 4: hipLaunchKernelGGL(k_add_ln<4>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 5: hipLaunchKernelGGL(k_add_ln<5>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 6: hipLaunchKernelGGL(k_add_ln<6>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 7: hipLaunchKernelGGL(k_add_ln<7>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 8: hipLaunchKernelGGL(k_add_ln<8>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 12: hipLaunchKernelGGL(k_add_ln<12>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    case 16: hipLaunchKernelGGL(k_add_ln<16>, grid, blk, 0, st, x, res, alpha, w, b, out, rows); break;
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// d = 256 .. 2048 (wider rows would spill at two waves per SIMD)
bool mh_add_ln_prep_supported(int d) { return d > 0 && d % 256 == 0 && d / 256 <= 8; }

hipError_t mh_launch_add_ln_prep(float *x, const float *res, float alpha, const float *w, const float *b, int rows,
                                 int d, uint8_t *xp, float *xpf, hipStream_t st) {
    if (rows <= 0) return hipSuccess;
    if (!mh_add_ln_prep_supported(d)) return hipErrorInvalidValue;
    const dim3 grid(mh_mpad(rows) / 8), blk(512);
    switch (d / 256) {
#define LNP(V) \
    case V: hipLaunchKernelGGL(k_add_ln_prep<V>, grid, blk, 0, st, x, res, alpha, w, b, rows, xp, xpf); break;
    LNP(1) LNP(2) LNP(3) LNP(4) LNP(5) LNP(6) LNP(7) LNP(8)
#undef LNP
    default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t mh_launch_glu(const float *h, float *g, size_t rows, int d, hipStream_t st) {
    if (!rows) return hipSuccess;
    if (d % 4) return hipErrorInvalidValue;
    const size_t n = rows * (size_t)(d / 4);
    hipLaunchKernelGGL(k_glu, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, h, g, rows, d);
    return hipGetLastError();
}

bool mh_glu_dwconv_supported(int d, int k) {
    return d > 0 && d % 256 == 0 && k > 0 && sizeof(float4) * 64 * (size_t)(DW_R + 2 * k - 1) <= 64 * 1024;
}

hipError_t mh_launch_glu_dwconv(const float *h, const float *w, const float *bias, const float *scale,
                                const float *shift, float *out, int T, int nseq, int d, int k, int causal,
                                uint8_t *xp, float *xpf, hipStream_t st) {
    if (T <= 0 || nseq <= 0) return hipSuccess;
    if (!mh_glu_dwconv_supported(d, k)) return hipErrorInvalidValue;
    const int pc = causal ? k - 1 : (k - 1) / 2;
    const size_t lds = sizeof(float4) * 64 * (size_t)(DW_R + 2 * k - 1);   // >= the staged slots and folds
    const dim3 grid((unsigned)((T + DW_R - 1) / DW_R), d / 256, nseq);
    if (xp) {
        hipLaunchKernelGGL((k_dwconv_tile<true, true>), grid, dim3(256), lds, st, h, w, bias, scale, shift, out, T, d,
                           k, pc, xp, xpf);
    } else {
        hipLaunchKernelGGL((k_dwconv_tile<true, false>), grid, dim3(256), lds, st, h, w, bias, scale, shift, out, T, d,
                           k, pc, nullptr, nullptr);
    }
    return hipGetLastError();
}

hipError_t mh_launch_dwconv(const float *g, const float *w, const float *bias, const float *scale,
                            const float *shift, float *out, int T, int nseq, int d, int k, int causal,
                            hipStream_t st) {
    if (T <= 0 || nseq <= 0) return hipSuccess;
    if (d % 4 || k <= 0) return hipErrorInvalidValue;
    const int pc = causal ? k - 1 : (k - 1) / 2;
    if (mh_glu_dwconv_supported(d, k)) {
        const size_t lds = sizeof(float4) * 64 * (size_t)(DW_R + 2 * k - 1);
        hipLaunchKernelGGL((k_dwconv_tile<false, false>), dim3((unsigned)((T + DW_R - 1) / DW_R), d / 256, nseq),
                           dim3(256), lds, st, g, w, bias, scale, shift, out, T, d, k, pc, nullptr, nullptr);
        return hipGetLastError();
    }
    const size_t n = (size_t)nseq * T * (d / 4);
    hipLaunchKernelGGL(k_dwconv, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, g, w, bias, scale, shift, out,
                       T, nseq, d, k, pc);
    return hipGetLastError();
}

int mh_ss_out_len(int n, int causal) {
    // (n + pl + pr - 3) / 2 + 1 with pads (2, 1) causal, (1, 1) otherwise
    const int p = causal ? 3 : 2;
    return (n + p - 3) / 2 + 1;
}

hipError_t mh_launch_conv_in_dw(const float *x, const float *w0, const float *b0, const float *w1, const float *b1,
                                float *out, int nseq, int T, int F, int C, int causal, hipStream_t st) {
    if (C % 4) return hipErrorInvalidValue;
    const int T1 = mh_ss_out_len(T, causal), F1 = mh_ss_out_len(F, causal);
    const int To = mh_ss_out_len(T1, causal), Fo = mh_ss_out_len(F1, causal);
    if (T1 <= 0 || F1 <= 0 || To <= 0 || Fo <= 0) return hipSuccess;
    const size_t rows = (size_t)nseq * To;   // one wave per output row (s, to)
    if (!rows) return hipSuccess;
    if (rows > 0x7fffffff) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_conv_in_dw, dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, st, x, w0, b0, w1, b1, out, nseq,
                       T, F, T1, F1, To, Fo, C, causal ? 2 : 1);
    return hipGetLastError();
}

hipError_t mh_launch_dw_s2(const float *in, const float *pb, const float *w, const float *b, float *out, int nseq,
                           int T, int F, int C, int causal, hipStream_t st) {
    if (C % 4) return hipErrorInvalidValue;
    const int To = mh_ss_out_len(T, causal), Fo = mh_ss_out_len(F, causal);
    const size_t n = (size_t)nseq * To * Fo * (C / 4);
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_dw_s2, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, pb, w, b, out, nseq, T, F, To,
                       Fo, C, causal ? 2 : 1);
    return hipGetLastError();
}

hipError_t mh_launch_flatten(const float *in, const float *pb, float *flat, size_t rows, int Fo, int C,
                             hipStream_t st) {
    const size_t n = rows * (size_t)C * Fo;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_flatten, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, in, pb, flat, rows, Fo, C);
    return hipGetLastError();
}

hipError_t mh_launch_bias_scale(float *y, const float *b, size_t rows, int d, float scale, hipStream_t st) {
    const size_t n = rows * (size_t)d;
    if (!n) return hipSuccess;
    hipLaunchKernelGGL(k_bias_scale, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, y, b, rows, d, scale);
    return hipGetLastError();
}

hipError_t mh_launch_transpose_taps(const float *w, float *wt, int C, int k, hipStream_t st) {
    if (C * k <= 0) return hipSuccess;
    hipLaunchKernelGGL(k_transpose, dim3((C * k + 255) / 256), dim3(256), 0, st, w, wt, C, k);
    return hipGetLastError();
}
