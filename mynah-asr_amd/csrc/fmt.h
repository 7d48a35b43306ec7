// fmt.h — device-side view of the resident weight layouts (gfx950).
//
// Every weight format is repacked at upload into an "MFMA-native" layout: the
// quant bits each lane of a wave feeds into v_mfma_f32_32x32x16_f16 sit at
// consecutive addresses, so one wave-wide load of 4/8/16 bytes per lane moves a
// contiguous 256 B/512 B/1 KiB block. Nothing is widened: the planes hold the
// same bits as the ggml blocks (or the qmat INT8/INT4 arrays), only reordered
// (Q8_0's bytes with their top bit flipped: offset binary, q + 128).
//
// Geometry shared by every kernel:
//   column group G = 32 weight rows (the B/N side of one MFMA)
//   kstep          = 32 elements of K (one block of the 32-block formats)
//   half-step u    = 16 elements of K (the K of one MFMA); kstep s = u 2s, 2s+1
//   chunk          = 4 ksteps = 8 half-steps = 128 elements of K
//   lane l (0..63): column r = l & 31, half h = l >> 5; in half-step u it
//                   carries chunk elements 16u + 8h + j (j = 0..7) of weight
//                   row 32G + r.
// MFMA operand convention (32x32x16 f16): A = activations (row = l&31, k =
// 8h+j), B = weights (column = l&31, k = 8h+j); D lane l holds column l&31 and
// rows 8i + 4h + jj in element 4i + jj (i, jj = 0..3).
//
// Planes (bytes per lane per chunk = b):  b <= 16: [G][chunk][64][b]
//                                         b  > 16: [G][chunk][b/16][64][16]
// Lane bit layouts inside a plane, chosen so that a pair of elements (2t, 2t+1)
// lands in the two 16-bit halves of a dword with one shift and one mask:
//   bytes  (8 b/elt) : half-step u = dwords 2u, 2u+1; dword 2u holds elements
//                      {0,4,1,5}, dword 2u+1 elements {2,6,3,7} in bytes 0..3
//                      (the order in which a nibble dword expands to bytes,
//                      w & 0x0F0F0F0F and (w >> 4) & 0x0F0F0F0F, so that one
//                      int8 activation layout serves byte and nibble weights);
//                      kstep s is the 16-byte part s
//   nibble (4 b/elt) : half-step u = dword u; element 2t+v at bit 16v + 4t
//   crumb  (2 b/elt) : half-steps 2w, 2w+1 = dword w; element 2t+v of half-step
//                      2w+x at bit 16v + 8x + 2t
//   bit    (1 b/elt) : half-steps 4w..4w+3 = dword w; element 2t+v of half-step
//                      4w+x at bit 16v + 4x + t
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef _Float16 half4v __attribute__((ext_vector_type(4)));
typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f16v __attribute__((ext_vector_type(16)));

enum {
    QT_F32 = 0, QT_INT8 = 1, QT_INT4 = 2, QT_Q4_0 = 18, QT_Q8_0 = 24, QT_Q2_K = 26,
    QT_Q3_K = 27, QT_Q4_K = 28, QT_Q5_K = 29, QT_Q6_K = 30
};

// Resident weight, as the kernels see it.
struct DevW {
    const uint8_t *p0;   // main quant plane
    const uint8_t *p1;   // high-bit plane (Q5_K, Q6_K, Q3_K)
    const uint8_t *h;    // per-(row, block/super-block) header bytes
    const float *h2;     // per-(row, super-block) f32 factors / per-row scale
    int n, k;            // logical shape
    int Np, Kp;          // padded: Np multiple of 128, Kp multiple of 256
};

// The activation split's chunk shift (the products' preparation, and the
// layer norm that prepares its output for them): sh puts the chunk's largest
// magnitude in [2^14, 2^15); 0 for a chunk of zeros.
__device__ __forceinline__ int chunk_shift(float amax) {
    int e = 0;
    if (amax > 0.0f) (void)frexpf(amax, &e);
    return amax > 0.0f ? 15 - e : 0;
}

// XCD-aware order of a 3-D grid. The hardware deals workgroups to the 8 XCDs
// round-robin by flat id (x fastest, then y, then z), and each XCD has its own
// L2. This gives each XCD a contiguous run of logical (x, z, y) triples, x
// fastest, then z, then y, so that workgroups neighbouring in x (then in z)
// run on one XCD and share what they read through its L2. A bijection of the
// grid onto itself.
__device__ __forceinline__ void xcd_order(int &bx, int &by, int &bz) {
    const int gx = gridDim.x, gy = gridDim.y, gz = gridDim.z;
    const int ntot = gx * gy * gz, flat = blockIdx.x + gx * (blockIdx.y + gy * blockIdx.z);
    const int qx = ntot / 8, rx = ntot % 8, xcd = flat % 8, loc = flat / 8;
    const int lg = xcd < rx ? xcd * (qx + 1) + loc : rx * (qx + 1) + (xcd - rx) * qx + loc;
    bx = lg % gx;
    bz = (lg / gx) % gz;
    by = lg / (gx * gz);
}

__device__ __forceinline__ half8 pairs_to_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                                _Float16 bias) {
    // each dword holds two f16 values 1024+code (exact integers); subtract the
    // format's bias with packed f16 adds (exact: operands and result < 2048)
    half2v v0 = __builtin_bit_cast(half2v, a), v1 = __builtin_bit_cast(half2v, b);
    half2v v2 = __builtin_bit_cast(half2v, c), v3 = __builtin_bit_cast(half2v, d);
    const half2v nb = {(_Float16)-bias, (_Float16)-bias};
    v0 += nb; v1 += nb; v2 += nb; v3 += nb;
    half8 r;
    r[0] = v0[0]; r[1] = v0[1]; r[2] = v1[0]; r[3] = v1[1];
    r[4] = v2[0]; r[5] = v2[1]; r[6] = v3[0]; r[7] = v3[1];
    return r;
}

// the same pairs (1024 + code) times an integer sub-block factor f: one
// packed f16 fma per pair, v*f - 1024*f, whose exact value (code*f) is an
// f16 integer below 2048, so the single rounding is exact
__device__ __forceinline__ half8 pairs_to_half8_f(uint32_t a, uint32_t b, uint32_t c, uint32_t d, half2v f) {
    const half2v nb = f * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};   // exact: 2^10 * f
    half2v v0 = __builtin_bit_cast(half2v, a), v1 = __builtin_bit_cast(half2v, b);
    half2v v2 = __builtin_bit_cast(half2v, c), v3 = __builtin_bit_cast(half2v, d);
    v0 = __builtin_elementwise_fma(v0, f, nb);
    v1 = __builtin_elementwise_fma(v1, f, nb);
    v2 = __builtin_elementwise_fma(v2, f, nb);
    v3 = __builtin_elementwise_fma(v3, f, nb);
    half8 r;
    r[0] = v0[0]; r[1] = v0[1]; r[2] = v1[0]; r[3] = v1[1];
    r[4] = v2[0]; r[5] = v2[1]; r[6] = v3[0]; r[7] = v3[1];
    return r;
}

#define MAGIC 0x64006400u
// (a & b) | c as one v_bitop3_b32 (truth table over sources 0xF0, 0xCC, 0xAA:
// (0xF0 & 0xCC) | 0xAA = 0xEA); the compiler would emit an and and an or
__device__ __forceinline__ uint32_t and_or(uint32_t a, uint32_t b, uint32_t c) {
    return __builtin_amdgcn_bitop3_b32(a, b, c, 0xEA);
}
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int t) { return (w >> (4 * t)) & 0x000F000Fu; }
// pair t of half-step u in a crumb dword / a bit dword
__device__ __forceinline__ uint32_t crumb_pair(uint32_t w, int u, int t) {
    return (w >> (8 * (u & 1) + 2 * t)) & 0x00030003u;
}
__device__ __forceinline__ uint32_t bit_pair(uint32_t w, int u, int t) {
    return (w >> (4 * (u & 3) + t)) & 0x00010001u;
}

// int8 bytes -> half8 of their signed values (pairs (0,1) (2,3) (4,5) (6,7))
__device__ __forceinline__ half8 dec_bytes(uint32_t w0, uint32_t w1) {
    const uint32_t a = (w0 & 0x00FF00FFu) ^ 0x64806480u, b = (w1 & 0x00FF00FFu) ^ 0x64806480u;
    const uint32_t c = ((w0 >> 8) & 0x00FF00FFu) ^ 0x64806480u, d = ((w1 >> 8) & 0x00FF00FFu) ^ 0x64806480u;
    return pairs_to_half8(a, b, c, d, (_Float16)1152.0f);
}

// offset-binary bytes (q + 128) -> half8 of q: each f16 pair 1024 + (q + 128)
// assembled by one byte permute with the exponent byte 0x64, then -1152
__device__ __forceinline__ half8 dec_bytes_ob(uint32_t w0, uint32_t w1) {
    const uint32_t E = 0x64646464u;
    const uint32_t a = __builtin_amdgcn_perm(E, w0, 0x04020400u), b = __builtin_amdgcn_perm(E, w1, 0x04020400u);
    const uint32_t c = __builtin_amdgcn_perm(E, w0, 0x04030401u), d = __builtin_amdgcn_perm(E, w1, 0x04030401u);
    return pairs_to_half8(a, b, c, d, (_Float16)1152.0f);
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// a[i] for a runtime i in 0..3 as register selects (a dynamic index into a
// register array would go through scratch memory)
__device__ __forceinline__ uint32_t sel4(const uint32_t (&a)[4], int i) {
    const uint32_t lo = (i & 1) ? a[1] : a[0], hi = (i & 1) ? a[3] : a[2];
    return (i & 2) ? hi : lo;
}

// header slot of (column group G, unit c of `units`, the lane's column)
__device__ __forceinline__ size_t hdr(int G, int units, int c, int lane) {
    return ((size_t)G * units + c) * 32 + (lane & 31);
}

// Per-kstep plane words: B bytes per lane per chunk; kstep s uses
//   B = 64: the 16-byte part s            B = 32: 8 bytes (dwords 2s, 2s+1)
//   B = 16: dword s                       B =  8: dword s >> 1
template <int B> struct KWords { static constexpr int N = B == 64 ? 4 : (B == 32 ? 2 : 1); };

template <int B>
__device__ __forceinline__ void load_kpart(const uint8_t *p, int Kc, int G, int c, int s, int lane,
                                           uint32_t (&w)[KWords<B>::N]) {
    const size_t tile = (size_t)G * Kc + c;
    if constexpr (B == 64) {
        const uint4 v = *(const uint4 *)(p + ((tile * 4 + s) * 64 + lane) * 16);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (B == 32) {
        const uint2 v = *(const uint2 *)(p + ((tile * 2 + (s >> 1)) * 64 + lane) * 16 + 8 * (s & 1));
        w[0] = v.x; w[1] = v.y;
    } else if constexpr (B == 16) {
        w[0] = *(const uint32_t *)(p + (tile * 64 + lane) * 16 + 4 * s);
    } else {
        static_assert(B == 8, "plane width");
        w[0] = *(const uint32_t *)(p + (tile * 64 + lane) * 8 + 4 * (s >> 1));
    }
}

// Staging of a plane for half a chunk (the LDS-staged GEMM): B >= 32 stages
// the half's own 32*B bytes of the (G, chunk) block, narrower planes the whole
// 64*B-byte block. off(h) = byte offset of half h inside the block.
template <int B> struct Stage {
    static constexpr int BYTES = B == 0 ? 0 : (B >= 32 ? 32 * B : 64 * B);
    static __device__ __forceinline__ int off(int h) { return B >= 32 ? h * 32 * B : 0; }
};

// the same words from a staged region r (the half containing kstep s)
template <int B>
__device__ __forceinline__ void lds_kpart(const uint8_t *r, int s, int lane, uint32_t (&w)[KWords<B>::N]) {
    if constexpr (B == 64) {
        const uint4 v = *(const uint4 *)(r + ((s & 1) * 64 + lane) * 16);
        w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
    } else if constexpr (B == 32) {
        const uint2 v = *(const uint2 *)(r + lane * 16 + 8 * (s & 1));
        w[0] = v.x; w[1] = v.y;
    } else if constexpr (B == 16) {
        w[0] = *(const uint32_t *)(r + lane * 16 + 4 * s);
    } else {
        static_assert(B == 8, "plane width");
        w[0] = *(const uint32_t *)(r + lane * 8 + 4 * (s >> 1));
    }
}

// A nibble dword as four f16 pairs, with one shift: pairs 0 and 2 are the low
// nibbles of the bytes of w and w >> 8 (value 1024 + q), pairs 1 and 3 their
// high nibbles left in place (1024 + 16 q, still an exact f16 integer).
struct NibPairs { half2v lo0, hi0, lo1, hi1; };
__device__ __forceinline__ NibPairs nib_pairs(uint32_t w) {
    const uint32_t w8 = w >> 8;
    return {__builtin_bit_cast(half2v, and_or(w, 0x000F000Fu, MAGIC)), __builtin_bit_cast(half2v, and_or(w, 0x00F000F0u, MAGIC)),
            __builtin_bit_cast(half2v, and_or(w8, 0x000F000Fu, MAGIC)),
            __builtin_bit_cast(half2v, and_or(w8, 0x00F000F0u, MAGIC))};
}
__device__ __forceinline__ half8 pack_pairs(half2v v0, half2v v1, half2v v2, half2v v3) {
    half8 r;
    r[0] = v0[0]; r[1] = v0[1]; r[2] = v1[0]; r[3] = v1[1];
    r[4] = v2[0]; r[5] = v2[1]; r[6] = v3[0]; r[7] = v3[1];
    return r;
}
// q - (bias - 1024): exact packed adds, and for the in-place pairs
// (1024 + 16 q) / 16 - (bias - 960) by one packed fma (1/16 is exact)
__device__ __forceinline__ half8 dec_nib(uint32_t w, _Float16 bias) {
    const NibPairs p = nib_pairs(w);
    const half2v nb = {(_Float16)-bias, (_Float16)-bias};
    const half2v r16 = {(_Float16)0.0625f, (_Float16)0.0625f};
    const _Float16 b16 = (_Float16)(960.0f - (float)bias);
    const half2v nb16 = {b16, b16};
    return pack_pairs(p.lo0 + nb, __builtin_elementwise_fma(p.hi0, r16, nb16), p.lo1 + nb,
                      __builtin_elementwise_fma(p.hi1, r16, nb16));
}
// Nibble pairs with extra high bits: pairs 0 and 2 (low nibbles) take them at
// bit 4 (value 1024 + q), pairs 1 and 3 (high nibbles, in place) at bit 8
// (value 1024 + 16 q). hm[t] = MAGIC | pair t's extra bits at that place.
__device__ __forceinline__ NibPairs nib_pairs_hi(uint32_t w, const uint32_t (&hm)[4]) {
    const uint32_t w8 = w >> 8;
    return {__builtin_bit_cast(half2v, and_or(w, 0x000F000Fu, hm[0])),
            __builtin_bit_cast(half2v, and_or(w, 0x00F000F0u, hm[1])),
            __builtin_bit_cast(half2v, and_or(w8, 0x000F000Fu, hm[2])),
            __builtin_bit_cast(half2v, and_or(w8, 0x00F000F0u, hm[3]))};
}
// x << sh for sh >= 0, else x >> -sh (constant after unrolling)
__device__ __forceinline__ uint32_t shift_by(uint32_t x, int sh) { return sh >= 0 ? x << sh : x >> -sh; }
// hm for extra bits of width NB (1: a bit plane, 2: a crumb plane) whose pair
// t sits at bit pos(t) (+16) of h: moved to bit 4 (t even) or 8 (t odd)
template <int NB>
__device__ __forceinline__ void extra_bits(uint32_t h, int pos0, int step, uint32_t (&hm)[4]) {
    constexpr uint32_t m = NB == 1 ? 0x00010001u : 0x00030003u;
#pragma unroll
    for (int t = 0; t < 4; t++) {
        const int to = (t & 1) ? 8 : 4;
        hm[t] = and_or(shift_by(h, to - (pos0 + step * t)), m << to, MAGIC);
    }
}
// q * f from such pairs (the factor form of dec_nib_f)
__device__ __forceinline__ half8 nibs_f(const NibPairs &p, half2v f) {
    const half2v nb = f * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
    const half2v f16th = f * (half2v){(_Float16)0.0625f, (_Float16)0.0625f};
    const half2v nb16 = f * (half2v){(_Float16)-64.0f, (_Float16)-64.0f};
    return pack_pairs(__builtin_elementwise_fma(p.lo0, f, nb), __builtin_elementwise_fma(p.hi0, f16th, nb16),
                      __builtin_elementwise_fma(p.lo1, f, nb), __builtin_elementwise_fma(p.hi1, f16th, nb16));
}

// q * f for an integer factor f: v*f - 1024 f, and (1024 + 16 q) * (f/16) - 64 f
// (every constant and the exact results are f16 integers or 2^-4 multiples)
__device__ __forceinline__ half8 dec_nib_f(uint32_t w, half2v f) {
    const NibPairs p = nib_pairs(w);
    const half2v nb = f * (half2v){(_Float16)-1024.0f, (_Float16)-1024.0f};
    const half2v f16th = f * (half2v){(_Float16)0.0625f, (_Float16)0.0625f};
    const half2v nb16 = f * (half2v){(_Float16)-64.0f, (_Float16)-64.0f};
    return pack_pairs(__builtin_elementwise_fma(p.lo0, f, nb), __builtin_elementwise_fma(p.hi0, f16th, nb16),
                      __builtin_elementwise_fma(p.lo1, f, nb), __builtin_elementwise_fma(p.hi1, f16th, nb16));
}

// ---------------------------------------------------------------------------
// Format traits. For every format:
//   SUB16        sub-blocks of 16 (one per half-step) instead of 32 (per kstep)
//   MINS         affine format: value = scale*q - min
//   B0, B1       plane widths (bytes per lane per chunk) of p0 / p1
//   HB, H2       header bytes / h2 bytes per column group and header unit
//   hb_src, h2_src   the (column group, chunk)'s header unit in global memory
//   Hdr          per-lane header registers of one chunk (block factors)
//   RawK         per-lane plane words of one kstep
//   load_hdr(W, Kc, G, c, lane, hdr)      the chunk's headers for column r
//   load_k(W, Kc, G, c, s, lane, raw)     kstep s's plane words
//   hdr_lds(hb, h2b, c, lane, hdr), k_lds(r0, r1, s, lane, raw)
//                                         the same from staged LDS regions
//   decode(raw, s, kh)                    half8 of the integer quants of
//                                         half-step 2s+kh
//   scale(hdr, s, hh, &sc, &mn)           factor (and min) of kstep s's
//                                         sub-block hh (0 unless SUB16)
// The factors are computed exactly as the reference decoders do, so that
// sc*q - mn (or sc*q) reproduces their f32 values bit for bit (the dequant
// kernel).
//
// Formats whose sub-block factors are small integers under one f32 (or f16)
// super-block factor — Q2_K, Q3_K, Q4_K, Q5_K — also carry, for the product
// kernels:
//   FHdr                  the chunk's integer sub-block factors as f16 pairs
//                         (sf), the super-block factor d, and for the affine
//                         ones dm = 32 * dmin and the integer mins as the B
//                         operand of one MFMA (mb: slot j = min of sub-block j,
//                         in both lane halves)
//   load_fhdr / fhdr_lds  as load_hdr / hdr_lds
//   decode_f(raw, s, kh, fh)  half8 of q * (integer factor) of half-step
//                         2s+kh: exact f16 integers (|q*f| < 2048)
// ---------------------------------------------------------------------------
template <int QT> struct Fmt;

// headers per chunk: [G][Kc][32 columns][b]; per super-block: [G][Kc/2][32][b]
__device__ __forceinline__ const uint8_t *chunk_hdr(const uint8_t *h, int Kc, int G, int c, int b) {
    return h + hdr(G, Kc, c, 0) * b;
}
__device__ __forceinline__ const uint8_t *sb_hdr(const uint8_t *h, int Kc, int G, int c, int b) {
    return h + hdr(G, Kc / 2, c / 2, 0) * b;
}

template <> struct Fmt<QT_INT8> {
    static constexpr bool SUB16 = false, MINS = false;
    static constexpr int B0 = 64, B1 = 0, HB = 0, H2 = 128;
    struct Hdr { float s; };
    struct RawK { uint32_t w[4]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &W, int, int G, int) {
        return (const uint8_t *)(W.h2 + 32 * G);
    }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int, int G, int, int lane, Hdr &H) {
        H.s = W.h2[32 * G + (lane & 31)];
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *, const uint8_t *h2b, int, int lane, Hdr &H) {
        H.s = ((const float *)h2b)[lane & 31];
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<64>(W.p0, Kc, G, c, s, lane, R.w);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *, int s, int lane, RawK &R) {
        lds_kpart<64>(r0, s, lane, R.w);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int, int kh) { return dec_bytes(R.w[2 * kh], R.w[2 * kh + 1]); }
    static __device__ __forceinline__ void scale(const Hdr &H, int, int, float &sc, float &mn) { sc = H.s; mn = 0.0f; }
};

template <> struct Fmt<QT_INT4> {
    static constexpr bool SUB16 = false, MINS = false;
    static constexpr int B0 = 32, B1 = 0, HB = 0, H2 = 512;
    struct Hdr { float d[4]; };
    struct RawK { uint32_t w[2]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &W, int Kc, int G, int c) {
        return (const uint8_t *)(W.h2 + hdr(G, Kc, c, 0) * 4);
    }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        const float4 v = *(const float4 *)(W.h2 + hdr(G, Kc, c, lane) * 4);
        H.d[0] = v.x; H.d[1] = v.y; H.d[2] = v.z; H.d[3] = v.w;
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *, const uint8_t *h2b, int, int lane, Hdr &H) {
        const float4 v = *(const float4 *)(h2b + (lane & 31) * 16);
        H.d[0] = v.x; H.d[1] = v.y; H.d[2] = v.z; H.d[3] = v.w;
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<32>(W.p0, Kc, G, c, s, lane, R.w);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *, int s, int lane, RawK &R) {
        lds_kpart<32>(r0, s, lane, R.w);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int, int kh) { return dec_nib(R.w[kh], (_Float16)1032.0f); }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int, float &sc, float &mn) { sc = H.d[s]; mn = 0.0f; }
};

// Q8_0 / Q4_0: header unit = the chunk's four f16 block factors per column
struct BlkHdr { uint32_t d[2]; };
__device__ __forceinline__ void blk_scale(const BlkHdr &H, int s, float &sc, float &mn) {
    sc = h2f((H.d[s >> 1] >> (16 * (s & 1))) & 0xffff);
    mn = 0.0f;
}

template <> struct Fmt<QT_Q8_0> {
    static constexpr bool SUB16 = false, MINS = false;
    static constexpr int B0 = 64, B1 = 0, HB = 256, H2 = 0;
    using Hdr = BlkHdr;
    struct RawK { uint32_t w[4]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &W, int Kc, int G, int c) { return chunk_hdr(W.h, Kc, G, c, 8); }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        const uint2 hd = *(const uint2 *)(W.h + hdr(G, Kc, c, lane) * 8);
        H.d[0] = hd.x; H.d[1] = hd.y;
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *hb, const uint8_t *, int, int lane, Hdr &H) {
        const uint2 hd = *(const uint2 *)(hb + (lane & 31) * 8);
        H.d[0] = hd.x; H.d[1] = hd.y;
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<64>(W.p0, Kc, G, c, s, lane, R.w);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *, int s, int lane, RawK &R) {
        lds_kpart<64>(r0, s, lane, R.w);
    }
    // the plane holds q + 128 (offset binary; see repack.cpp)
    static __device__ __forceinline__ half8 decode(const RawK &R, int, int kh) { return dec_bytes_ob(R.w[2 * kh], R.w[2 * kh + 1]); }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int, float &sc, float &mn) { blk_scale(H, s, sc, mn); }
};

template <> struct Fmt<QT_Q4_0> {
    static constexpr bool SUB16 = false, MINS = false;
    static constexpr int B0 = 32, B1 = 0, HB = 256, H2 = 0;
    using Hdr = BlkHdr;
    struct RawK { uint32_t w[2]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &W, int Kc, int G, int c) { return chunk_hdr(W.h, Kc, G, c, 8); }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        const uint2 hd = *(const uint2 *)(W.h + hdr(G, Kc, c, lane) * 8);
        H.d[0] = hd.x; H.d[1] = hd.y;
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *hb, const uint8_t *, int, int lane, Hdr &H) {
        const uint2 hd = *(const uint2 *)(hb + (lane & 31) * 8);
        H.d[0] = hd.x; H.d[1] = hd.y;
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<32>(W.p0, Kc, G, c, s, lane, R.w);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *, int s, int lane, RawK &R) {
        lds_kpart<32>(r0, s, lane, R.w);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int, int kh) { return dec_nib(R.w[kh], (_Float16)1032.0f); }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int, float &sc, float &mn) { blk_scale(H, s, sc, mn); }
};

// Q4_K / Q5_K super-block header: f16 d, f16 dmin, 12 bytes of packed 6-bit
// scales and mins (ingot dequant.c:59-68 unpacking).
__device__ __forceinline__ void k4_ints(const uint32_t (&hd)[4], int j, uint32_t &s, uint32_t &m) {
    auto byte = [&](int i) -> uint32_t { return (sel4(hd, 1 + (i >> 2)) >> (8 * (i & 3))) & 0xffu; };
    if (j < 4) {
        s = byte(j) & 63u;
        m = byte(j + 4) & 63u;
    } else {
        s = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
}
__device__ __forceinline__ void k4_scale_min(const uint32_t (&hd)[4], int j, float &sc, float &mn) {
    const float d = h2f(hd[0] & 0xffff), dmin = h2f(hd[0] >> 16);
    uint32_t s, m;
    k4_ints(hd, j, s, m);
    sc = d * (float)s;
    mn = dmin * (float)m;
}

// folded factors of NS sub-blocks per chunk (see the trait notes)
template <int NS> struct FoldHdr {
    half2v sf[NS];
    float d, dm;
    half8 mb;
};
__device__ __forceinline__ half2v h2pair(int v) {
    const _Float16 f = (_Float16)(float)v;
    return (half2v){f, f};
}
__device__ __forceinline__ void k4fhdr_from(const uint8_t *p, int c, FoldHdr<4> &H) {
    const uint4 v = *(const uint4 *)p;
    const uint32_t hd[4] = {v.x, v.y, v.z, v.w};
    H.d = h2f(hd[0] & 0xffff);
    H.dm = h2f(hd[0] >> 16) * 32.0f;
#pragma unroll
    for (int s = 0; s < 8; s++) H.mb[s] = (_Float16)0.0f;
#pragma unroll
    for (int s = 0; s < 4; s++) {
        uint32_t sc, mn;
        k4_ints(hd, 4 * (c & 1) + s, sc, mn);
        H.sf[s] = h2pair((int)sc);
        H.mb[s] = (_Float16)(float)mn;
    }
}

// the chunk's four sub-block factors and mins, decoded once per chunk
struct K4Hdr { float sc[4], mn[4]; };
__device__ __forceinline__ void k4hdr_from(const uint8_t *p, int c, K4Hdr &H) {
    const uint4 v = *(const uint4 *)p;
    const uint32_t hd[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int s = 0; s < 4; s++) k4_scale_min(hd, 4 * (c & 1) + s, H.sc[s], H.mn[s]);
}

template <> struct Fmt<QT_Q4_K> {
    static constexpr bool SUB16 = false, MINS = true;
    static constexpr int B0 = 32, B1 = 0, HB = 512, H2 = 0;
    using Hdr = K4Hdr;
    struct RawK { uint32_t w[2]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &W, int Kc, int G, int c) { return sb_hdr(W.h, Kc, G, c, 16); }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        k4hdr_from(W.h + hdr(G, Kc / 2, c / 2, lane) * 16, c, H);
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *hb, const uint8_t *, int c, int lane, Hdr &H) {
        k4hdr_from(hb + (lane & 31) * 16, c, H);
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<32>(W.p0, Kc, G, c, s, lane, R.w);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *, int s, int lane, RawK &R) {
        lds_kpart<32>(r0, s, lane, R.w);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int, int kh) { return dec_nib(R.w[kh], (_Float16)1024.0f); }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int, float &sc, float &mn) {
        sc = H.sc[s];
        mn = H.mn[s];
    }
    using FHdr = FoldHdr<4>;
    static __device__ __forceinline__ void load_fhdr(const DevW &W, int Kc, int G, int c, int lane, FHdr &H) {
        k4fhdr_from(W.h + hdr(G, Kc / 2, c / 2, lane) * 16, c, H);
    }
    static __device__ __forceinline__ void fhdr_lds(const uint8_t *hb, const uint8_t *, int c, int lane, FHdr &H) {
        k4fhdr_from(hb + (lane & 31) * 16, c, H);
    }
    static __device__ __forceinline__ half8 decode_f(const RawK &R, int s, int kh, const FHdr &H) {
        return dec_nib_f(R.w[kh], H.sf[s]);
    }
};

template <> struct Fmt<QT_Q5_K> {
    static constexpr bool SUB16 = false, MINS = true;
    static constexpr int B0 = 32, B1 = 8, HB = 512, H2 = 0;
    using Hdr = K4Hdr;
    struct RawK { uint32_t w[2]; uint32_t hb[1]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &W, int Kc, int G, int c) { return sb_hdr(W.h, Kc, G, c, 16); }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        k4hdr_from(W.h + hdr(G, Kc / 2, c / 2, lane) * 16, c, H);
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *hb, const uint8_t *, int c, int lane, Hdr &H) {
        k4hdr_from(hb + (lane & 31) * 16, c, H);
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<32>(W.p0, Kc, G, c, s, lane, R.w);
        load_kpart<8>(W.p1, Kc, G, c, s, lane, R.hb);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *r1, int s, int lane, RawK &R) {
        lds_kpart<32>(r0, s, lane, R.w);
        lds_kpart<8>(r1, s, lane, R.hb);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int s, int kh) {
        const int u = 2 * s + kh;
        const uint32_t w = R.w[kh], h = R.hb[0];
        uint32_t p[4];
#pragma unroll
        for (int t = 0; t < 4; t++) p[t] = nib_pair(w, t) | (bit_pair(h, u, t) << 4) | MAGIC;
        return pairs_to_half8(p[0], p[1], p[2], p[3], (_Float16)1024.0f);
    }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int, float &sc, float &mn) {
        sc = H.sc[s];
        mn = H.mn[s];
    }
    using FHdr = FoldHdr<4>;
    static __device__ __forceinline__ void load_fhdr(const DevW &W, int Kc, int G, int c, int lane, FHdr &H) {
        k4fhdr_from(W.h + hdr(G, Kc / 2, c / 2, lane) * 16, c, H);
    }
    static __device__ __forceinline__ void fhdr_lds(const uint8_t *hb, const uint8_t *, int c, int lane, FHdr &H) {
        k4fhdr_from(hb + (lane & 31) * 16, c, H);
    }
    static __device__ __forceinline__ half8 decode_f(const RawK &R, int s, int kh, const FHdr &H) {
        // the 5th bit of pair t of half-step u is bit 4 (u & 3) + t of hb
        uint32_t hm[4];
        extra_bits<1>(R.hb[0], 4 * ((2 * s + kh) & 3), 1, hm);
        return nibs_f(nib_pairs_hi(R.w[kh], hm), H.sf[s]);
    }
};

// Q6_K / Q3_K: header unit = 16 sub-block scale bytes (Q3_K: 12 packed + 4
// pad) per column and super-block; h2 = d (f32).
struct ScHdr { float sc[8]; };  // the chunk's eight 16-element sub-block factors

template <> struct Fmt<QT_Q6_K> {
    static constexpr bool SUB16 = true, MINS = false;
    static constexpr int B0 = 32, B1 = 16, HB = 512, H2 = 128;
    using Hdr = ScHdr;
    struct RawK { uint32_t w[2]; uint32_t hi[1]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &W, int Kc, int G, int c) { return sb_hdr(W.h, Kc, G, c, 16); }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &W, int Kc, int G, int c) {
        return (const uint8_t *)(W.h2 + hdr(G, Kc / 2, c / 2, 0));
    }
    static __device__ __forceinline__ void from(const uint8_t *p, float d, int c, Hdr &H) {
        const uint4 v = *(const uint4 *)p;
        const uint32_t sc[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int j = 8 * (c & 1) + q;
            H.sc[q] = d * (float)(int8_t)((sel4(sc, j >> 2) >> (8 * (j & 3))) & 0xffu);
        }
    }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        const size_t u = hdr(G, Kc / 2, c / 2, lane);
        from(W.h + u * 16, W.h2[u], c, H);
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *hb, const uint8_t *h2b, int c, int lane, Hdr &H) {
        from(hb + (lane & 31) * 16, ((const float *)h2b)[lane & 31], c, H);
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<32>(W.p0, Kc, G, c, s, lane, R.w);
        load_kpart<16>(W.p1, Kc, G, c, s, lane, R.hi);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *r1, int s, int lane, RawK &R) {
        lds_kpart<32>(r0, s, lane, R.w);
        lds_kpart<16>(r1, s, lane, R.hi);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int s, int kh) {
        const int u = 2 * s + kh;
        const uint32_t w = R.w[kh], h = R.hi[0];
        uint32_t p[4];
#pragma unroll
        for (int t = 0; t < 4; t++) p[t] = nib_pair(w, t) | (crumb_pair(h, u, t) << 4) | MAGIC;
        return pairs_to_half8(p[0], p[1], p[2], p[3], (_Float16)1056.0f);
    }
    // the same values: the crumbs (bits 8 (u & 1) + 2t of hi) joined in place,
    // q - 32 by a packed add (low nibbles) or (1024 + 16 q) / 16 - 96 (high)
    static __device__ __forceinline__ half8 decode_fast(const RawK &R, int s, int kh) {
        uint32_t hm[4];
        extra_bits<2>(R.hi[0], 8 * ((2 * s + kh) & 1), 2, hm);
        const NibPairs p = nib_pairs_hi(R.w[kh], hm);
        const half2v nb = {(_Float16)-1056.0f, (_Float16)-1056.0f};
        const half2v r16 = {(_Float16)0.0625f, (_Float16)0.0625f}, nb16 = {(_Float16)-96.0f, (_Float16)-96.0f};
        return pack_pairs(p.lo0 + nb, __builtin_elementwise_fma(p.hi0, r16, nb16), p.lo1 + nb,
                          __builtin_elementwise_fma(p.hi1, r16, nb16));
    }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int hh, float &sc, float &mn) {
        sc = H.sc[2 * s + hh];
        mn = 0.0f;
    }
};

template <> struct Fmt<QT_Q3_K> {
    static constexpr bool SUB16 = true, MINS = false;
    static constexpr int B0 = 16, B1 = 8, HB = 512, H2 = 128;
    using Hdr = ScHdr;
    struct RawK { uint32_t w[1]; uint32_t hb[1]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &W, int Kc, int G, int c) { return sb_hdr(W.h, Kc, G, c, 16); }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &W, int Kc, int G, int c) {
        return (const uint8_t *)(W.h2 + hdr(G, Kc / 2, c / 2, 0));
    }
    static __device__ __forceinline__ void from(const uint8_t *p, float d, int c, Hdr &H) {
        const uint4 v = *(const uint4 *)p;
        const uint32_t sc[4] = {v.x, v.y, v.z, v.w};
        auto byte = [&](int i) -> int { return (int)((sel4(sc, i >> 2) >> (8 * (i & 3))) & 0xffu); };
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int j = 8 * (c & 1) + q;
            const int lo = j < 8 ? (byte(j) & 15) : (byte(j - 8) >> 4);
            const int hi = (byte(8 + (j & 3)) >> (2 * (j >> 2))) & 3;
            H.sc[q] = d * (float)((lo | (hi << 4)) - 32);
        }
    }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        const size_t u = hdr(G, Kc / 2, c / 2, lane);
        from(W.h + u * 16, W.h2[u], c, H);
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *hb, const uint8_t *h2b, int c, int lane, Hdr &H) {
        from(hb + (lane & 31) * 16, ((const float *)h2b)[lane & 31], c, H);
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<16>(W.p0, Kc, G, c, s, lane, R.w);
        load_kpart<8>(W.p1, Kc, G, c, s, lane, R.hb);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *r1, int s, int lane, RawK &R) {
        lds_kpart<16>(r0, s, lane, R.w);
        lds_kpart<8>(r1, s, lane, R.hb);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int s, int kh) {
        const int u = 2 * s + kh;
        const uint32_t w = R.w[0], h = R.hb[0];
        uint32_t p[4];
#pragma unroll
        for (int t = 0; t < 4; t++) p[t] = crumb_pair(w, u, t) | (bit_pair(h, u, t) << 2) | MAGIC;
        return pairs_to_half8(p[0], p[1], p[2], p[3], (_Float16)1028.0f);
    }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int hh, float &sc, float &mn) {
        sc = H.sc[2 * s + hh];
        mn = 0.0f;
    }
    // folded: factor lo | hi << 4 minus 32 (|q*f| <= 128); no mins
    using FHdr = FoldHdr<8>;
    static __device__ __forceinline__ void ffrom(const uint8_t *p, float d, int c, FHdr &H) {
        const uint4 v = *(const uint4 *)p;
        const uint32_t sc[4] = {v.x, v.y, v.z, v.w};
        auto byte = [&](int i) -> int { return (int)((sel4(sc, i >> 2) >> (8 * (i & 3))) & 0xffu); };
        H.d = d;
        H.dm = 0.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int j = 8 * (c & 1) + q;
            const int lo = j < 8 ? (byte(j) & 15) : (byte(j - 8) >> 4);
            const int hi = (byte(8 + (j & 3)) >> (2 * (j >> 2))) & 3;
            H.sf[q] = h2pair((lo | (hi << 4)) - 32);
            H.mb[q] = (_Float16)0.0f;
        }
    }
    static __device__ __forceinline__ void load_fhdr(const DevW &W, int Kc, int G, int c, int lane, FHdr &H) {
        const size_t u = hdr(G, Kc / 2, c / 2, lane);
        ffrom(W.h + u * 16, W.h2[u], c, H);
    }
    static __device__ __forceinline__ void fhdr_lds(const uint8_t *hb, const uint8_t *h2b, int c, int lane, FHdr &H) {
        ffrom(hb + (lane & 31) * 16, ((const float *)h2b)[lane & 31], c, H);
    }
    static __device__ __forceinline__ half8 decode_f(const RawK &R, int s, int kh, const FHdr &H) {
        const half8 q = decode(R, s, kh);
        const half2v f = H.sf[2 * s + kh];
        half8 r;
#pragma unroll
        for (int t = 0; t < 4; t++) {
            const half2v v = (half2v){q[2 * t], q[2 * t + 1]} * f;
            r[2 * t] = v[0];
            r[2 * t + 1] = v[1];
        }
        return r;
    }
};

// Q2_K: header unit = 16 scale|min bytes per column, h2 = (d, dmin) (f32 pair).
struct Q2Hdr { float sc[8], mn[8]; };  // the chunk's eight sub-block factors and mins

template <> struct Fmt<QT_Q2_K> {
    static constexpr bool SUB16 = true, MINS = true;
    static constexpr int B0 = 16, B1 = 0, HB = 512, H2 = 256;
    using Hdr = Q2Hdr;
    struct RawK { uint32_t w[1]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &W, int Kc, int G, int c) { return sb_hdr(W.h, Kc, G, c, 16); }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &W, int Kc, int G, int c) {
        return (const uint8_t *)(W.h2 + 2 * hdr(G, Kc / 2, c / 2, 0));
    }
    static __device__ __forceinline__ void from(const uint8_t *p, float2 dd, int c, Hdr &H) {
        const uint4 v = *(const uint4 *)p;
        const uint32_t sc[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int j = 8 * (c & 1) + q;
            const uint32_t b = (sel4(sc, j >> 2) >> (8 * (j & 3))) & 0xffu;
            H.sc[q] = dd.x * (float)(b & 15u);
            H.mn[q] = dd.y * (float)(b >> 4);
        }
    }
    static __device__ __forceinline__ void load_hdr(const DevW &W, int Kc, int G, int c, int lane, Hdr &H) {
        const size_t u = hdr(G, Kc / 2, c / 2, lane);
        from(W.h + u * 16, *(const float2 *)(W.h2 + 2 * u), c, H);
    }
    static __device__ __forceinline__ void hdr_lds(const uint8_t *hb, const uint8_t *h2b, int c, int lane, Hdr &H) {
        from(hb + (lane & 31) * 16, *(const float2 *)(h2b + (lane & 31) * 8), c, H);
    }
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        load_kpart<16>(W.p0, Kc, G, c, s, lane, R.w);
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *, int s, int lane, RawK &R) {
        lds_kpart<16>(r0, s, lane, R.w);
    }
    static __device__ __forceinline__ half8 decode(const RawK &R, int s, int kh) {
        const int u = 2 * s + kh;
        const uint32_t w = R.w[0];
        return pairs_to_half8(crumb_pair(w, u, 0) | MAGIC, crumb_pair(w, u, 1) | MAGIC,
                              crumb_pair(w, u, 2) | MAGIC, crumb_pair(w, u, 3) | MAGIC,
                              (_Float16)1024.0f);
    }
    static __device__ __forceinline__ void scale(const Hdr &H, int s, int hh, float &sc, float &mn) {
        sc = H.sc[2 * s + hh];
        mn = H.mn[2 * s + hh];
    }
    using FHdr = FoldHdr<8>;
    static __device__ __forceinline__ void ffrom(const uint8_t *p, float2 dd, int c, FHdr &H) {
        const uint4 v = *(const uint4 *)p;
        const uint32_t sc[4] = {v.x, v.y, v.z, v.w};
        H.d = dd.x;
        H.dm = dd.y * 32.0f;
#pragma unroll
        for (int q = 0; q < 8; q++) {
            const int j = 8 * (c & 1) + q;
            const uint32_t b = (sel4(sc, j >> 2) >> (8 * (j & 3))) & 0xffu;
            H.sf[q] = h2pair((int)(b & 15u));
            H.mb[q] = (_Float16)(float)(b >> 4);
        }
    }
    static __device__ __forceinline__ void load_fhdr(const DevW &W, int Kc, int G, int c, int lane, FHdr &H) {
        const size_t u = hdr(G, Kc / 2, c / 2, lane);
        ffrom(W.h + u * 16, *(const float2 *)(W.h2 + 2 * u), c, H);
    }
    static __device__ __forceinline__ void fhdr_lds(const uint8_t *hb, const uint8_t *h2b, int c, int lane, FHdr &H) {
        ffrom(hb + (lane & 31) * 16, *(const float2 *)(h2b + (lane & 31) * 8), c, H);
    }
    static __device__ __forceinline__ half8 decode_f(const RawK &R, int s, int kh, const FHdr &H) {
        const int u = 2 * s + kh;
        const uint32_t w = R.w[0];
        return pairs_to_half8_f(crumb_pair(w, u, 0) | MAGIC, crumb_pair(w, u, 1) | MAGIC,
                                crumb_pair(w, u, 2) | MAGIC, crumb_pair(w, u, 3) | MAGIC, H.sf[u]);
    }
};

// F32: (wh, wl) f16 fragments of w * 2^shw_n; the plane's 16-byte part 2u is
// wh of half-step u and part 2u+1 its wl; h2 = shw_n per row.
template <> struct Fmt<QT_F32> {
    static constexpr bool SUB16 = false, MINS = false;
    static constexpr int B0 = 256, B1 = 0, HB = 0, H2 = 0;
    struct Hdr {};
    struct RawK { half8 h[2], l[2]; };
    static __device__ __forceinline__ const uint8_t *hb_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ const uint8_t *h2_src(const DevW &, int, int, int) { return nullptr; }
    static __device__ __forceinline__ void load_hdr(const DevW &, int, int, int, int, Hdr &) {}
    static __device__ __forceinline__ void hdr_lds(const uint8_t *, const uint8_t *, int, int, Hdr &) {}
    static __device__ __forceinline__ void load_k(const DevW &W, int Kc, int G, int c, int s, int lane, RawK &R) {
        const size_t base = ((size_t)G * Kc + c) * 16 + 4 * s;
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            R.h[kh] = *(const half8 *)(W.p0 + ((base + 2 * kh) * 64 + lane) * 16);
            R.l[kh] = *(const half8 *)(W.p0 + ((base + 2 * kh + 1) * 64 + lane) * 16);
        }
    }
    static __device__ __forceinline__ void k_lds(const uint8_t *r0, const uint8_t *, int s, int lane, RawK &R) {
        // staged half = parts 8h .. 8h+7; kstep s is local kstep s & 1
#pragma unroll
        for (int kh = 0; kh < 2; kh++) {
            R.h[kh] = *(const half8 *)(r0 + ((4 * (s & 1) + 2 * kh) * 64 + lane) * 16);
            R.l[kh] = *(const half8 *)(r0 + ((4 * (s & 1) + 2 * kh + 1) * 64 + lane) * 16);
        }
    }
};
