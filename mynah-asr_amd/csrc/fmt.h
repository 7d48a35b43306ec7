// fmt.h — device-side view of the resident weight layouts (gfx950).
//
// Every weight format is repacked at upload into an "MFMA-native" layout: the
// quant bits each lane of a wave feeds into v_mfma_f32_16x16x32_f16 sit at
// consecutive addresses, so one wave-wide load of 4/8/16 bytes per lane moves a
// contiguous 256 B/512 B/1 KiB block. Nothing is widened: the planes hold the
// same bits as the ggml blocks (or the qmat INT8/INT4 arrays), only reordered.
//
// Geometry shared by every kernel:
//   row group  G  = 16 weight rows (the B/N side of one MFMA)
//   kstep         = 32 elements of K (one MFMA); chunk = 4 ksteps = 128 of K
//   lane l (0..63): column r = l & 15, k-group g = l >> 4; in kstep s it carries
//                   elements 8g .. 8g+7 of that kstep for weight row 16G + r.
// MFMA operand convention (16x16x32 f16): A = activations (row = l&15, k =
// 8g+j), B = weights (column = l&15, k = 8g+j); D lane l holds rows 4g+i,
// column l&15.
//
// Planes (bytes per lane per chunk = b):  b <= 16: [G][chunk][64][b]
//                                         b  > 16: [G][chunk][b/16][64][16]
// Lane bit layouts inside a plane, chosen so that a pair of elements (2t, 2t+1)
// lands in the two 16-bit halves of a dword with one shift and one mask:
//   bytes  (8 b/elt) : kstep s = dwords 2s, 2s+1; dword 2s holds elements
//                      {0,4,1,5}, dword 2s+1 elements {2,6,3,7} in bytes 0..3
//                      (the order in which a nibble dword expands to bytes,
//                      w & 0x0F0F0F0F and (w >> 4) & 0x0F0F0F0F, so that one
//                      int8 activation layout serves byte and nibble weights)
//   nibble (4 b/elt) : kstep s = dword s; element 2t+u at bit 16u + 4t
//   crumb  (2 b/elt) : ksteps 2v, 2v+1 = dword v; element 2t+u of kstep 2v+w
//                      at bit 16u + 8w + 2t
//   bit    (1 b/elt) : one dword per chunk; element 2t+u of kstep s at bit
//                      16u + 4s + t
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float f4 __attribute__((ext_vector_type(4)));

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

__device__ __forceinline__ uint32_t ldg32(const uint8_t *p) { return *(const uint32_t *)p; }

// Load b bytes per lane of plane p for (row group G, chunk c) into w[b/4].
template <int B>
__device__ __forceinline__ void load_plane(const uint8_t *p, int Kc, int G, int c, int lane,
                                           uint32_t (&w)[(B + 3) / 4]) {
    const size_t tile = (size_t)G * Kc + c;
    if constexpr (B <= 16) {
        const uint8_t *q = p + (tile * 64 + lane) * B;
        if constexpr (B == 16) {
            const uint4 v = *(const uint4 *)q;
            w[0] = v.x; w[1] = v.y; w[2] = v.z; w[3] = v.w;
        } else if constexpr (B == 8) {
            const uint2 v = *(const uint2 *)q;
            w[0] = v.x; w[1] = v.y;
        } else {
            w[0] = ldg32(q);
        }
    } else {
#pragma unroll
        for (int part = 0; part < B / 16; part++) {
            const uint4 v = *(const uint4 *)(p + ((tile * (B / 16) + part) * 64 + lane) * 16);
            w[4 * part + 0] = v.x; w[4 * part + 1] = v.y;
            w[4 * part + 2] = v.z; w[4 * part + 3] = v.w;
        }
    }
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

#define MAGIC 0x64006400u
__device__ __forceinline__ uint32_t nib_pair(uint32_t w, int t) { return (w >> (4 * t)) & 0x000F000Fu; }
__device__ __forceinline__ uint32_t crumb_pair(uint32_t w, int s, int t) {
    return (w >> (8 * (s & 1) + 2 * t)) & 0x00030003u;
}
__device__ __forceinline__ uint32_t bit_pair(uint32_t w, int s, int t) {
    return (w >> (4 * s + t)) & 0x00010001u;
}

// int8 bytes -> half8 of their signed values (pairs (0,1) (2,3) (4,5) (6,7))
__device__ __forceinline__ half8 dec_bytes(uint32_t w0, uint32_t w1) {
    const uint32_t a = (w0 & 0x00FF00FFu) ^ 0x64806480u, b = (w1 & 0x00FF00FFu) ^ 0x64806480u;
    const uint32_t c = ((w0 >> 8) & 0x00FF00FFu) ^ 0x64806480u, d = ((w1 >> 8) & 0x00FF00FFu) ^ 0x64806480u;
    return pairs_to_half8(a, b, c, d, (_Float16)1152.0f);
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// ---------------------------------------------------------------------------
// Format traits. For every format:
//   B0, B1       bytes per lane per chunk in plane 0 / plane 1
//   SUB16        sub-blocks of 16 (two scales per kstep) instead of 32
//   MINS         affine format: value = scale*q - min
//   Raw          per-lane registers for one chunk
//   load(...)    fetch the chunk's planes and headers for column r
//   decode(raw,s)            half8 of the integer quant values of kstep s
//   scale(raw,s,h, &sc,&mn)  factor (and min) of kstep s's sub-block h (h = 0
//                            for SUB16 == false; 0/1 for the two 16-halves)
// The factors are computed exactly as the reference decoders do, so that
// sc*q - mn (or sc*q) reproduces their f32 values bit for bit.
// ---------------------------------------------------------------------------
template <int QT> struct Fmt;

template <> struct Fmt<QT_Q8_0> {
    static constexpr int B0 = 32, B1 = 0;
    static constexpr bool SUB16 = false, MINS = false;
    struct Raw { uint32_t w[8]; uint32_t d[2]; };  // d: the chunk's four f16 block factors
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<32>(W.p0, Kc, G, c, lane, R.w);
        const uint2 hd = *(const uint2 *)(W.h + (((size_t)G * Kc + c) * 16 + (lane & 15)) * 8);
        R.d[0] = hd.x; R.d[1] = hd.y;
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) { return dec_bytes(R.w[2 * s], R.w[2 * s + 1]); }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int, float &sc, float &mn) {
        sc = h2f((R.d[s >> 1] >> (16 * (s & 1))) & 0xffff);
        mn = 0.0f;
    }
};

template <> struct Fmt<QT_Q4_0> {
    static constexpr int B0 = 16, B1 = 0;
    static constexpr bool SUB16 = false, MINS = false;
    struct Raw { uint32_t w[4]; uint32_t d[2]; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<16>(W.p0, Kc, G, c, lane, R.w);
        const uint2 hd = *(const uint2 *)(W.h + (((size_t)G * Kc + c) * 16 + (lane & 15)) * 8);
        R.d[0] = hd.x; R.d[1] = hd.y;
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) {
        const uint32_t w = R.w[s];
        return pairs_to_half8(nib_pair(w, 0) | MAGIC, nib_pair(w, 1) | MAGIC, nib_pair(w, 2) | MAGIC,
                              nib_pair(w, 3) | MAGIC, (_Float16)1032.0f);
    }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int, float &sc, float &mn) {
        sc = h2f((R.d[s >> 1] >> (16 * (s & 1))) & 0xffff);
        mn = 0.0f;
    }
};

template <> struct Fmt<QT_INT8> {
    static constexpr int B0 = 32, B1 = 0;
    static constexpr bool SUB16 = false, MINS = false;
    struct Raw { uint32_t w[8]; float s; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<32>(W.p0, Kc, G, c, lane, R.w);
        R.s = W.h2[16 * G + (lane & 15)];
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) { return dec_bytes(R.w[2 * s], R.w[2 * s + 1]); }
    static __device__ __forceinline__ void scale(const Raw &R, int, int, float &sc, float &mn) { sc = R.s; mn = 0.0f; }
};

template <> struct Fmt<QT_INT4> {
    static constexpr int B0 = 16, B1 = 0;
    static constexpr bool SUB16 = false, MINS = false;
    struct Raw { uint32_t w[4]; float d[4]; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<16>(W.p0, Kc, G, c, lane, R.w);
        const float4 v = *(const float4 *)(W.h2 + (((size_t)G * Kc + c) * 16 + (lane & 15)) * 4);
        R.d[0] = v.x; R.d[1] = v.y; R.d[2] = v.z; R.d[3] = v.w;
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) {
        const uint32_t w = R.w[s];
        return pairs_to_half8(nib_pair(w, 0) | MAGIC, nib_pair(w, 1) | MAGIC, nib_pair(w, 2) | MAGIC,
                              nib_pair(w, 3) | MAGIC, (_Float16)1032.0f);
    }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int, float &sc, float &mn) { sc = R.d[s]; mn = 0.0f; }
};

// Q4_K / Q5_K super-block header: f16 d, f16 dmin, 12 bytes of packed 6-bit
// scales and mins (ingot dequant.c:59-68 unpacking).
__device__ __forceinline__ void k4_scale_min(const uint32_t (&hd)[4], int j, float &sc, float &mn) {
    const float d = h2f(hd[0] & 0xffff), dmin = h2f(hd[0] >> 16);
    auto byte = [&](int i) -> uint32_t { return (hd[1 + i / 4] >> (8 * (i % 4))) & 0xffu; };
    uint32_t s, m;
    if (j < 4) {
        s = byte(j) & 63u;
        m = byte(j + 4) & 63u;
    } else {
        s = (byte(j + 4) & 15u) | ((byte(j - 4) >> 6) << 4);
        m = (byte(j + 4) >> 4) | ((byte(j) >> 6) << 4);
    }
    sc = d * (float)s;
    mn = dmin * (float)m;
}

template <> struct Fmt<QT_Q4_K> {
    static constexpr int B0 = 16, B1 = 0;
    static constexpr bool SUB16 = false, MINS = true;
    struct Raw { uint32_t w[4]; uint32_t hd[4]; int half_sb; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<16>(W.p0, Kc, G, c, lane, R.w);
        const uint4 v = *(const uint4 *)(W.h + (((size_t)G * (Kc / 2) + c / 2) * 16 + (lane & 15)) * 16);
        R.hd[0] = v.x; R.hd[1] = v.y; R.hd[2] = v.z; R.hd[3] = v.w;
        R.half_sb = 4 * (c & 1);
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) {
        const uint32_t w = R.w[s];
        return pairs_to_half8(nib_pair(w, 0) | MAGIC, nib_pair(w, 1) | MAGIC, nib_pair(w, 2) | MAGIC,
                              nib_pair(w, 3) | MAGIC, (_Float16)1024.0f);
    }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int, float &sc, float &mn) {
        k4_scale_min(R.hd, R.half_sb + s, sc, mn);
    }
};

template <> struct Fmt<QT_Q5_K> {
    static constexpr int B0 = 16, B1 = 4;
    static constexpr bool SUB16 = false, MINS = true;
    struct Raw { uint32_t w[4]; uint32_t hb[1]; uint32_t hd[4]; int half_sb; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<16>(W.p0, Kc, G, c, lane, R.w);
        load_plane<4>(W.p1, Kc, G, c, lane, R.hb);
        const uint4 v = *(const uint4 *)(W.h + (((size_t)G * (Kc / 2) + c / 2) * 16 + (lane & 15)) * 16);
        R.hd[0] = v.x; R.hd[1] = v.y; R.hd[2] = v.z; R.hd[3] = v.w;
        R.half_sb = 4 * (c & 1);
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) {
        const uint32_t w = R.w[s], h = R.hb[0];
        uint32_t p[4];
#pragma unroll
        for (int t = 0; t < 4; t++) p[t] = nib_pair(w, t) | (bit_pair(h, s, t) << 4) | MAGIC;
        return pairs_to_half8(p[0], p[1], p[2], p[3], (_Float16)1024.0f);
    }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int, float &sc, float &mn) {
        k4_scale_min(R.hd, R.half_sb + s, sc, mn);
    }
};

// Q6_K: header plane = 16 int8 sub-block scales per super-block, h2 = d (f32).
template <> struct Fmt<QT_Q6_K> {
    static constexpr int B0 = 16, B1 = 8;
    static constexpr bool SUB16 = true, MINS = false;
    struct Raw { uint32_t w[4]; uint32_t hi[2]; uint32_t sc[4]; float d; int half_sb; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<16>(W.p0, Kc, G, c, lane, R.w);
        load_plane<8>(W.p1, Kc, G, c, lane, R.hi);
        const size_t u = ((size_t)G * (Kc / 2) + c / 2) * 16 + (lane & 15);
        const uint4 v = *(const uint4 *)(W.h + u * 16);
        R.sc[0] = v.x; R.sc[1] = v.y; R.sc[2] = v.z; R.sc[3] = v.w;
        R.d = W.h2[u];
        R.half_sb = 8 * (c & 1);
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) {
        const uint32_t w = R.w[s], h = R.hi[s >> 1];
        uint32_t p[4];
#pragma unroll
        for (int t = 0; t < 4; t++) p[t] = nib_pair(w, t) | (crumb_pair(h, s, t) << 4) | MAGIC;
        return pairs_to_half8(p[0], p[1], p[2], p[3], (_Float16)1056.0f);
    }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int hh, float &sc, float &mn) {
        const int j = R.half_sb + 2 * s + hh;
        const int8_t v = (int8_t)((R.sc[j >> 2] >> (8 * (j & 3))) & 0xffu);
        sc = R.d * (float)v;
        mn = 0.0f;
    }
};

// Q3_K: header plane = the 12 packed scale bytes (+4 pad), h2 = d (f32).
template <> struct Fmt<QT_Q3_K> {
    static constexpr int B0 = 8, B1 = 4;
    static constexpr bool SUB16 = true, MINS = false;
    struct Raw { uint32_t w[2]; uint32_t hb[1]; uint32_t sc[4]; float d; int half_sb; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<8>(W.p0, Kc, G, c, lane, R.w);
        load_plane<4>(W.p1, Kc, G, c, lane, R.hb);
        const size_t u = ((size_t)G * (Kc / 2) + c / 2) * 16 + (lane & 15);
        const uint4 v = *(const uint4 *)(W.h + u * 16);
        R.sc[0] = v.x; R.sc[1] = v.y; R.sc[2] = v.z; R.sc[3] = v.w;
        R.d = W.h2[u];
        R.half_sb = 8 * (c & 1);
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) {
        const uint32_t w = R.w[s >> 1], h = R.hb[0];
        uint32_t p[4];
#pragma unroll
        for (int t = 0; t < 4; t++) p[t] = crumb_pair(w, s, t) | (bit_pair(h, s, t) << 2) | MAGIC;
        return pairs_to_half8(p[0], p[1], p[2], p[3], (_Float16)1028.0f);
    }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int hh, float &sc, float &mn) {
        const int j = R.half_sb + 2 * s + hh;
        auto byte = [&](int i) -> int { return (int)((R.sc[i >> 2] >> (8 * (i & 3))) & 0xffu); };
        const int lo = j < 8 ? (byte(j) & 15) : (byte(j - 8) >> 4);
        const int hi = (byte(8 + (j & 3)) >> (2 * (j >> 2))) & 3;
        sc = R.d * (float)((lo | (hi << 4)) - 32);
        mn = 0.0f;
    }
};

// Q2_K: header plane = 16 scale|min bytes, h2 = (d, dmin) (f32 pair).
template <> struct Fmt<QT_Q2_K> {
    static constexpr int B0 = 8, B1 = 0;
    static constexpr bool SUB16 = true, MINS = true;
    struct Raw { uint32_t w[2]; uint32_t sc[4]; float d, dmin; int half_sb; };
    static __device__ __forceinline__ void load(const DevW &W, int Kc, int G, int c, int lane, Raw &R) {
        load_plane<8>(W.p0, Kc, G, c, lane, R.w);
        const size_t u = ((size_t)G * (Kc / 2) + c / 2) * 16 + (lane & 15);
        const uint4 v = *(const uint4 *)(W.h + u * 16);
        R.sc[0] = v.x; R.sc[1] = v.y; R.sc[2] = v.z; R.sc[3] = v.w;
        const float2 dd = *(const float2 *)(W.h2 + 2 * u);
        R.d = dd.x; R.dmin = dd.y;
        R.half_sb = 8 * (c & 1);
    }
    static __device__ __forceinline__ half8 decode(const Raw &R, int s) {
        const uint32_t w = R.w[s >> 1];
        return pairs_to_half8(crumb_pair(w, s, 0) | MAGIC, crumb_pair(w, s, 1) | MAGIC,
                              crumb_pair(w, s, 2) | MAGIC, crumb_pair(w, s, 3) | MAGIC,
                              (_Float16)1024.0f);
    }
    static __device__ __forceinline__ void scale(const Raw &R, int s, int hh, float &sc, float &mn) {
        const int j = R.half_sb + 2 * s + hh;
        const uint32_t b = (R.sc[j >> 2] >> (8 * (j & 3))) & 0xffu;
        sc = R.d * (float)(b & 15u);
        mn = R.dmin * (float)(b >> 4);
    }
};
