// repack.cpp — host-side conversion of a weight, as the caller holds it, into
// the resident device layout described in fmt.h. Bits are moved, never
// re-rounded: the quants and the f16/f32 block factors stay what the caller
// handed in (f16 super-block factors of the K-quants are widened to f32, which
// is exact). F32 weights are the one exception: they are stored as a pair of
// f16 terms (wh, wl) of w * 2^shw_n, which the EXACT product needs.
#include "repack.h"

#include <math.h>
#include <string.h>

namespace {

inline float f16_bits_to_f32(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
inline uint16_t ld16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

struct Src {
    const mynah_asr_hip_wdesc *w;
    int be, bb;  // block elements / bytes (1/elem-bytes for the qmat formats)
};

// Integer code of element (n, kk) of the weight (0 outside the logical shape),
// in the format's own range: Q8_0/INT8 as a byte, Q4_0/INT4 nibble, Q4_K nibble,
// Q5_K 5 bits, Q6_K 6 bits, Q3_K 3 bits (q2 | hbit<<2), Q2_K 2 bits. Follows
// the element walks of ingot dequant.c:73-445 and qmat.c:152-169.
uint32_t code_of(const Src &S, int n, int kk) {
    const mynah_asr_hip_wdesc *w = S.w;
    if (n >= w->n || kk >= w->k) return 0;
    const uint8_t *d = (const uint8_t *)w->data;
    if (w->qtype == MYNAH_ASR_HIP_INT8) return (uint8_t)d[(size_t)n * w->k + kk];
    if (w->qtype == MYNAH_ASR_HIP_INT4) {
        const uint8_t b = d[(size_t)n * (w->k / 2) + kk / 2];
        return (kk & 1) ? (b >> 4) : (b & 15);
    }
    const size_t nblk = (size_t)w->k / S.be;
    const uint8_t *blk = d + ((size_t)n * nblk + kk / S.be) * S.bb;
    const int e = kk % S.be;
    const int h = e / 128, r = e % 128, f = r / 32, l = r % 32;
    switch (w->qtype) {
    case MYNAH_ASR_HIP_Q8_0: return blk[2 + e];
    case MYNAH_ASR_HIP_Q4_0: return e < 16 ? (blk[2 + e] & 15) : (blk[2 + e - 16] >> 4);
    case MYNAH_ASR_HIP_Q4_K: return (blk[16 + 32 * (e / 64) + e % 32] >> (4 * ((e / 32) & 1))) & 15;
    case MYNAH_ASR_HIP_Q5_K: {
        const uint32_t lo = (blk[48 + 32 * (e / 64) + e % 32] >> (4 * ((e / 32) & 1))) & 15;
        const uint32_t hb = (blk[16 + e % 32] >> (e / 32)) & 1;
        return lo | (hb << 4);
    }
    case MYNAH_ASR_HIP_Q6_K: {
        const uint32_t lo = (blk[64 * h + 32 * (f & 1) + l] >> (4 * (f / 2))) & 15;
        const uint32_t hi = (blk[128 + 32 * h + l] >> (2 * f)) & 3;
        return lo | (hi << 4);
    }
    case MYNAH_ASR_HIP_Q3_K: {
        const uint32_t q2 = (blk[32 + 32 * h + l] >> (2 * f)) & 3;
        const uint32_t hb = (blk[l] >> (4 * h + f)) & 1;
        return q2 | (hb << 2);
    }
    case MYNAH_ASR_HIP_Q2_K: return (blk[16 + 32 * h + l] >> (2 * f)) & 3;
    }
    return 0;
}

// Store b bytes (as b/4 dwords) of lane `lane` for tile (G, c) of a plane.
void put_lane(uint8_t *plane, int b, int Kc, int G, int c, int lane, const uint32_t *dw) {
    const size_t tile = (size_t)G * Kc + c;
    if (b <= 16) {
        memcpy(plane + (tile * 64 + lane) * b, dw, b);
    } else {
        for (int part = 0; part < b / 16; part++)
            memcpy(plane + ((tile * (b / 16) + part) * 64 + lane) * 16, dw + 4 * part, 16);
    }
}

size_t align256(size_t v) { return (v + 255) & ~(size_t)255; }

}  // namespace

int mh_format_info(int qtype, int *be, int *bb) {
    int e = 0, b = 0;
    switch (qtype) {
    case MYNAH_ASR_HIP_F32: e = 1; b = 4; break;
    case MYNAH_ASR_HIP_INT8: e = 1; b = 1; break;
    case MYNAH_ASR_HIP_INT4: e = 32; b = 16; break;
    case MYNAH_ASR_HIP_Q4_0: e = 32; b = 18; break;
    case MYNAH_ASR_HIP_Q8_0: e = 32; b = 34; break;
    case MYNAH_ASR_HIP_Q2_K: e = 256; b = 84; break;
    case MYNAH_ASR_HIP_Q3_K: e = 256; b = 110; break;
    case MYNAH_ASR_HIP_Q4_K: e = 256; b = 144; break;
    case MYNAH_ASR_HIP_Q5_K: e = 256; b = 176; break;
    case MYNAH_ASR_HIP_Q6_K: e = 256; b = 210; break;
    default: return -1;
    }
    if (be) *be = e;
    if (bb) *bb = b;
    return 0;
}

int mh_repack(const mynah_asr_hip_wdesc *w, HostLayout *L) {
    int be, bb;
    if (!w || !w->data || w->n <= 0 || w->k <= 0 || mh_format_info(w->qtype, &be, &bb) != 0) return -1;
    if (w->k % be != 0) return -1;
    if ((w->qtype == MYNAH_ASR_HIP_INT8 || w->qtype == MYNAH_ASR_HIP_INT4) && !w->scales) return -1;
    const int qt = w->qtype;
    const int n = w->n, k = w->k;
    const int Np = (n + 127) / 128 * 128;
    const int Kp = (k + 255) / 256 * 256;
    const int Kc = Kp / 128, NG = Np / 32;
    L->Np = Np;
    L->Kp = Kp;
    int b0 = 0, b1 = 0;
    size_t hbytes = 0, h2floats = 0;
    const size_t slots = (size_t)NG * Kc * 32, sb_slots = (size_t)NG * (Kc / 2) * 32;
    switch (qt) {
    case MYNAH_ASR_HIP_F32: b0 = 256; h2floats = Np; break;
    case MYNAH_ASR_HIP_INT8: b0 = 64; h2floats = Np; break;
    case MYNAH_ASR_HIP_INT4: b0 = 32; h2floats = slots * 4; break;
    case MYNAH_ASR_HIP_Q8_0: b0 = 64; hbytes = slots * 8; break;
    case MYNAH_ASR_HIP_Q4_0: b0 = 32; hbytes = slots * 8; break;
    case MYNAH_ASR_HIP_Q4_K: b0 = 32; hbytes = sb_slots * 16; break;
    case MYNAH_ASR_HIP_Q5_K: b0 = 32; b1 = 8; hbytes = sb_slots * 16; break;
    case MYNAH_ASR_HIP_Q6_K: b0 = 32; b1 = 16; hbytes = sb_slots * 16; h2floats = sb_slots; break;
    case MYNAH_ASR_HIP_Q3_K: b0 = 16; b1 = 8; hbytes = sb_slots * 16; h2floats = sb_slots; break;
    case MYNAH_ASR_HIP_Q2_K: b0 = 16; hbytes = sb_slots * 16; h2floats = sb_slots * 2; break;
    }
    L->p0.assign((size_t)NG * Kc * 64 * b0, 0);
    L->p1.assign((size_t)NG * Kc * 64 * b1, 0);
    L->h.assign(hbytes, 0);
    L->h2.assign(h2floats, 0.0f);

    if (qt == MYNAH_ASR_HIP_F32) {
        // per-row shift: max|w_n| * 2^sh in [2^14, 2^15); terms wh = f16(w'), wl = f16(w' - wh)
        const float *W = (const float *)w->data;
        std::vector<int> sh(Np, 0);
        for (int r = 0; r < n; r++) {
            float amax = 0.0f;
            for (int j = 0; j < k; j++) amax = fmaxf(amax, fabsf(W[(size_t)r * k + j]));
            int e = 0;
            if (amax > 0.0f) (void)frexpf(amax, &e);
            sh[r] = amax > 0.0f ? 15 - e : 0;
            L->h2[r] = (float)sh[r];
        }
        // 16-byte part 2u = wh of half-step u, part 2u+1 = wl
        for (int G = 0; G < NG; G++)
            for (int c = 0; c < Kc; c++)
                for (int lane = 0; lane < 64; lane++) {
                    const int row = 32 * G + (lane & 31), h = lane >> 5;
                    uint32_t dw[64];
                    for (int u = 0; u < 8; u++) {
                        _Float16 hi[8], lo[8];
                        for (int j = 0; j < 8; j++) {
                            const int kk = 128 * c + 16 * u + 8 * h + j;
                            const float v = (row < n && kk < k) ? ldexpf(W[(size_t)row * k + kk], sh[row]) : 0.0f;
                            hi[j] = (_Float16)v;
                            lo[j] = (_Float16)(v - (float)hi[j]);
                        }
                        memcpy(dw + 8 * u, hi, 16);
                        memcpy(dw + 8 * u + 4, lo, 16);
                    }
                    put_lane(L->p0.data(), 256, Kc, G, c, lane, dw);
                }
        return 0;
    }

    const Src S{w, be, bb};
    const bool bytes8 = qt == MYNAH_ASR_HIP_Q8_0 || qt == MYNAH_ASR_HIP_INT8;
    const bool nib = qt == MYNAH_ASR_HIP_Q4_0 || qt == MYNAH_ASR_HIP_INT4 || qt == MYNAH_ASR_HIP_Q4_K ||
                     qt == MYNAH_ASR_HIP_Q5_K || qt == MYNAH_ASR_HIP_Q6_K;
    for (int G = 0; G < NG; G++)
        for (int c = 0; c < Kc; c++)
            for (int lane = 0; lane < 64; lane++) {
                const int row = 32 * G + (lane & 31), h = lane >> 5;
                uint32_t w0[16] = {0}, w1[4] = {0};
                for (int u = 0; u < 8; u++)
                    for (int j = 0; j < 8; j++) {
                        const uint32_t code = code_of(S, row, 128 * c + 16 * u + 8 * h + j);
                        const int t = j >> 1, v = j & 1;
                        if (bytes8) {
                            // dword 2u: elements {0,4,1,5}; dword 2u+1: {2,6,3,7}
                            static const int kWord[8] = {0, 0, 1, 1, 0, 0, 1, 1};
                            static const int kByte[8] = {0, 2, 0, 2, 1, 3, 1, 3};
                            // Q8_0 bytes offset-binary (q + 128): the decoder then
                            // builds each f16 pair with one byte permute
                            const uint32_t byte = qt == MYNAH_ASR_HIP_Q8_0 ? (code ^ 0x80u) & 0xffu : code & 0xffu;
                            w0[2 * u + kWord[j]] |= byte << (8 * kByte[j]);
                        } else if (nib) {
                            w0[u] |= (code & 15u) << (16 * v + 4 * t);
                            if (qt == MYNAH_ASR_HIP_Q5_K)
                                w1[u >> 2] |= ((code >> 4) & 1u) << (16 * v + 4 * (u & 3) + t);
                            else if (qt == MYNAH_ASR_HIP_Q6_K)
                                w1[u >> 1] |= ((code >> 4) & 3u) << (16 * v + 8 * (u & 1) + 2 * t);
                        } else {  // Q3_K, Q2_K: low two bits as crumbs
                            w0[u >> 1] |= (code & 3u) << (16 * v + 8 * (u & 1) + 2 * t);
                            if (qt == MYNAH_ASR_HIP_Q3_K)
                                w1[u >> 2] |= ((code >> 2) & 1u) << (16 * v + 4 * (u & 3) + t);
                        }
                    }
                put_lane(L->p0.data(), b0, Kc, G, c, lane, w0);
                if (b1) put_lane(L->p1.data(), b1, Kc, G, c, lane, w1);
            }

    // headers: one slot per (column group, chunk or super-block, column)
    const uint8_t *d = (const uint8_t *)w->data;
    const size_t nblk = (size_t)k / be;
    for (int G = 0; G < NG; G++)
        for (int r = 0; r < 32; r++) {
            const int row = 32 * G + r;
            if (row >= n) continue;
            if (qt == MYNAH_ASR_HIP_INT8) {
                L->h2[row] = w->scales[row];
                continue;
            }
            if (qt == MYNAH_ASR_HIP_INT4) {
                for (int b = 0; b < k / 32; b++)
                    L->h2[(((size_t)G * Kc + b / 4) * 32 + r) * 4 + b % 4] = w->scales[(size_t)row * (k / 32) + b];
                continue;
            }
            for (size_t b = 0; b < nblk; b++) {
                const uint8_t *blk = d + ((size_t)row * nblk + b) * bb;
                if (qt == MYNAH_ASR_HIP_Q8_0 || qt == MYNAH_ASR_HIP_Q4_0) {
                    memcpy(&L->h[(((size_t)G * Kc + b / 4) * 32 + r) * 8 + 2 * (b % 4)], blk, 2);
                    continue;
                }
                const size_t u = ((size_t)G * (Kc / 2) + b) * 32 + r;
                uint8_t *hh = &L->h[u * 16];
                switch (qt) {
                case MYNAH_ASR_HIP_Q4_K:
                case MYNAH_ASR_HIP_Q5_K: memcpy(hh, blk, 16); break;
                case MYNAH_ASR_HIP_Q6_K:
                    memcpy(hh, blk + 192, 16);
                    L->h2[u] = f16_bits_to_f32(ld16(blk + 208));
                    break;
                case MYNAH_ASR_HIP_Q3_K:
                    memcpy(hh, blk + 96, 12);
                    L->h2[u] = f16_bits_to_f32(ld16(blk + 108));
                    break;
                case MYNAH_ASR_HIP_Q2_K:
                    memcpy(hh, blk, 16);
                    L->h2[2 * u] = f16_bits_to_f32(ld16(blk + 80));
                    L->h2[2 * u + 1] = f16_bits_to_f32(ld16(blk + 82));
                    break;
                }
            }
        }
    return 0;
}

size_t mh_layout_bytes(const HostLayout &L, size_t off[4]) {
    size_t o = 0;
    off[0] = o; o = align256(o + L.p0.size());
    off[1] = o; o = align256(o + L.p1.size());
    off[2] = o; o = align256(o + L.h.size());
    off[3] = o; o = align256(o + L.h2.size() * sizeof(float));
    return o;
}
