// decoder.hip — the non-GEMV kernels of the AED (Canary) decoder step
// (the reference's src/decoder_aed.c:139-232), device-resident:
//
//   k_embed_ln   x = LN(emb[token] + pos[p])                  decoder_aed.c:183-186
//   k_att_part   one query against a split of KC keys, per head: running max,
//                sum of exponentials and the weighted sum of V rows; with
//                `append`, the split holding key p first stores this step's
//                k and v rows into the self-attention cache  decoder_aed.c:124-137, 195-198
//   k_att_combine the splits of each head merged (the decoder step merges them
//                instead in the prologue of the GEMV that reads the result)
//   k_argmax     first maximum of the logits, the next token; advances p and
//                forms the next position's x as k_embed_ln would (so only
//                the first position launches k_embed_ln)   decoder_aed.c:217-222
//   k_bias_rows  y[t] += b                                    decoder_aed.c:132-136
//
// The step's position p and its token live in device memory (`st`: st[0] = p,
// st[1] = the last argmax), so one captured launch sequence serves every
// step: position p reads prompt[p] while p < n_prompt, else the argmax of the
// step before (decoder_aed.c:213-222 chooses the same tokens).
#include <hip/hip_runtime.h>
#include <math.h>
#include <stdint.h>

#include "launch.h"

namespace {

constexpr int LN_T = 256;   // threads of the one-workgroup row kernels
constexpr int LN_V = 16;    // values per thread: d <= 4096
constexpr int KC = MH_ATT_KC;   // keys per attention split

// Sum over the NT threads of the workgroup in double (the reference's ln
// accumulates in double).
template <int NT>
__device__ double block_sum(double v, double *red) {
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < NT / 64; i++) s += red[i];
    return s;
}

// y = LN(v) over d values held V per thread (i = tid + NT * u):
// (float)((x - mean) * inv) * w + b with inv = (float)(1 / sqrt(var + 1e-5))
template <int NT, int V>
__device__ void ln_store(float (&v)[V], int d, const float *w, const float *b, float *y) {
    __shared__ double red[NT / 64];
    const int tid = threadIdx.x;
    float lw[V], lb[V];   // loaded before the sums, so their latency overlaps them
#pragma unroll
    for (int u = 0; u < V; u++) {
        const int i = tid + NT * u;
        lw[u] = i < d ? w[i] : 0.0f;
        lb[u] = i < d ? b[i] : 0.0f;
    }
    double s = 0.0;
#pragma unroll
    for (int u = 0; u < V; u++)
        if (tid + NT * u < d) s += (double)v[u];
    const double mu = block_sum<NT>(s, red) / d;
    double q = 0.0;
#pragma unroll
    for (int u = 0; u < V; u++)
        if (tid + NT * u < d) {
            const double c = (double)v[u] - mu;
            q += c * c;
        }
    const double var = block_sum<NT>(q, red) / d;
    const float inv = (float)(1.0 / sqrt(var + 1e-5));
#pragma unroll
    for (int u = 0; u < V; u++) {
        const int i = tid + NT * u;
        if (i < d) {
            const float t = (float)(((double)v[u] - mu) * (double)inv);
            y[i] = t * lw[u] + lb[u];
        }
    }
}

__global__ __launch_bounds__(LN_T) void k_embed_ln(const float *__restrict__ emb, const float *__restrict__ pos,
                                                   const int *__restrict__ prompt, int n_prompt,
                                                   const int *__restrict__ st, const float *__restrict__ w,
                                                   const float *__restrict__ b, float *__restrict__ x, int d) {
    const int p = st[0];
    const int tok = p < n_prompt ? prompt[p] : st[1];
    const float *e = emb + (size_t)tok * d, *pe = pos + (size_t)p * d;
    float v[LN_V];
#pragma unroll
    for (int u = 0; u < LN_V; u++) {
        const int i = threadIdx.x + LN_T * u;
        v[u] = i < d ? e[i] + pe[i] : 0.0f;
    }
    ln_store<LN_T, LN_V>(v, d, w, b, x);
}

// Workgroup (head h, split s) over keys [s*KC, min((s+1)*KC, n)), n = n_fixed,
// or p + 1 for self attention (n_fixed = 0). Four waves, wave w the keys
// 16w .. 16w+15 of the split: for the scores 4 lanes per key (DK/4 features
// each, q read by every lane from global); for the values lane = features
// DK/64 per lane over the wave's 16 keys. Two workgroup barriers: the waves'
// score maxima, then their partial outputs and sums, which wave 0 adds in
// wave order. Writes o[h][s][dk] (unnormalised) and ml[h][s] = (max, sum).
template <int DK>
__global__ __launch_bounds__(256) void k_att_part(const float *__restrict__ q, float *K, float *V,
                                                  const float *__restrict__ kn, const float *__restrict__ vn,
                                                  const int *__restrict__ st, int n_fixed, int d, float scale,
                                                  float *__restrict__ o_part, float *__restrict__ ml_part,
                                                  int nsplit) {
    static_assert(KC == 64, "four waves of 16 keys");
    constexpr int FPL = DK / 64;   // value features per lane
    __shared__ float wm[4], wl[4];
    __shared__ float wo[4][DK];
    const int h = blockIdx.x, s = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int ho = h * DK;
    const int p = n_fixed > 0 ? -1 : st[0];   // (cross attention does not wait for st)
    const int n = n_fixed > 0 ? n_fixed : p + 1;
    const int j0 = s * KC, j1 = min(j0 + KC, n);
    float *op = o_part + ((size_t)h * nsplit + s) * DK;
    float *mlp = ml_part + ((size_t)h * nsplit + s) * 2;
    if (j0 >= j1) {   // nothing in this split (uniform per workgroup)
        if (tid < DK) op[tid] = 0.0f;
        if (tid == 0) mlp[0] = -INFINITY, mlp[1] = 0.0f;
        return;
    }
    const bool append = n_fixed == 0 && p >= j0 && p < j1;
    if (append && tid < DK) {   // this step's k, v rows join the cache (read below from kn, vn)
        K[(size_t)p * d + ho + tid] = kn[ho + tid];
        V[(size_t)p * d + ho + tid] = vn[ho + tid];
    }
    const int cnt = j1 - j0;
    // the V values of this lane's features for the wave's 16 keys, loaded now
    // so that their latency overlaps the scores
    float vv[16][FPL];
#pragma unroll
    for (int t = 0; t < 16; t++) {
        const int jj = 16 * w + t, j = j0 + jj;
        const float *vr = (append && j == p) ? vn + ho : V + (size_t)j * d + ho;
#pragma unroll
        for (int i = 0; i < FPL; i++) vv[t][i] = jj < cnt ? vr[lane + 64 * i] : 0.0f;
    }
    // scores: key 16w + (lane >> 2), features (lane & 3) * DK/4 ..
    const int kq = lane >> 2, part = lane & 3, jj = 16 * w + kq, j = j0 + jj;
    const bool live = jj < cnt;
    float acc = 0.0f;
    if (live) {
        const float *kr = (append && j == p) ? kn + ho : K + (size_t)j * d + ho;
#pragma unroll
        for (int i = 0; i < DK / 16; i++) {
            const float4 kv = *(const float4 *)(kr + part * (DK / 4) + 4 * i);
            const float4 qv = *(const float4 *)(q + ho + part * (DK / 4) + 4 * i);
            acc = fmaf(qv.x, kv.x, acc);
            acc = fmaf(qv.y, kv.y, acc);
            acc = fmaf(qv.z, kv.z, acc);
            acc = fmaf(qv.w, kv.w, acc);
        }
    }
    acc += __shfl_xor(acc, 1, 64);
    acc += __shfl_xor(acc, 2, 64);
    const float sc = live ? scale * acc : -INFINITY;
    // the split's maximum: the wave's (every lane of a key holds its score), then the workgroup's
    float m = sc;
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) m = fmaxf(m, __shfl_xor(m, o, 64));
    if (lane == 0) wm[w] = m;
    __syncthreads();
    m = fmaxf(fmaxf(wm[0], wm[1]), fmaxf(wm[2], wm[3]));
    const float e = live ? expf(sc - m) : 0.0f;
    float l = part == 0 ? e : 0.0f;   // one lane per key
#pragma unroll
    for (int o = 4; o < 64; o <<= 1) l += __shfl_xor(l, o, 64);
    // values: this lane's features over the wave's keys, in key order
    float o[FPL];
#pragma unroll
    for (int i = 0; i < FPL; i++) o[i] = 0.0f;
#pragma unroll
    for (int t = 0; t < 16; t++) {
        const float pt = __shfl(e, 4 * t, 64);   // (zero past cnt)
#pragma unroll
        for (int i = 0; i < FPL; i++) o[i] = fmaf(pt, vv[t][i], o[i]);
    }
#pragma unroll
    for (int i = 0; i < FPL; i++) wo[w][lane + 64 * i] = o[i];
    if (lane == 0) wl[w] = l;
    __syncthreads();
    if (w == 0) {
#pragma unroll
        for (int i = 0; i < FPL; i++) {
            const int f = lane + 64 * i;
            op[f] = ((wo[0][f] + wo[1][f]) + wo[2][f]) + wo[3][f];
        }
        if (lane == 0) mlp[0] = m, mlp[1] = ((wl[0] + wl[1]) + wl[2]) + wl[3];
    }
}

// out[h] = sum_s o_s e^(m_s - M) / sum_s l_s e^(m_s - M) over the used splits
template <int DK>
__global__ __launch_bounds__(DK) void k_att_combine(const float *__restrict__ o_part,
                                                    const float *__restrict__ ml_part, const int *__restrict__ st,
                                                    int n_fixed, float *__restrict__ out, int nsplit) {
    const int h = blockIdx.x, f = threadIdx.x;
    const int n = n_fixed > 0 ? n_fixed : st[0] + 1;
    const int ns = min((n + KC - 1) / KC, nsplit);
    const float *ml = ml_part + (size_t)h * nsplit * 2;
    float M = -INFINITY;
    for (int s = 0; s < ns; s++) M = fmaxf(M, ml[2 * s]);
    float L = 0.0f, o = 0.0f;
    for (int s = 0; s < ns; s++) {
        const float c = expf(ml[2 * s] - M);
        L += ml[2 * s + 1] * c;
        o += o_part[((size_t)h * nsplit + s) * DK + f] * c;
    }
    out[h * DK + f] = o / L;
}

// First maximum of logits[0..vocab) (the reference's strict > scan) -> st[1];
// optionally the logits to logits_out[p]; then p + 1 -> st[0].
__global__ __launch_bounds__(1024) void k_argmax(const float *__restrict__ logits, int vocab, int *st,
                                                 float *__restrict__ logits_out, MhEmbNext en) {
    __shared__ float bv[16];
    __shared__ int bi[16];
    __shared__ int nxt;
    constexpr int AV = 16;   // logits per thread per batch: all of them go out at once
    const int tid = threadIdx.x, p = st[0];
    // the next position's rows that do not depend on this argmax go out first
    const int q = p + 1;
    const bool next = en.emb && q < en.max_pos;   // (uniform)
    float pv[4], ev[4];   // d <= 4096
    const bool in_prompt = next && q < en.n_prompt;
    if (next) {
        const float *pe = en.pos + (size_t)q * en.d;
        const float *e = in_prompt ? en.emb + (size_t)en.prompt[q] * en.d : nullptr;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = tid + 1024 * u;
            pv[u] = i < en.d ? pe[i] : 0.0f;
            ev[u] = in_prompt && i < en.d ? e[i] : 0.0f;
        }
    }
    float best = -INFINITY;
    int idx = 0x7fffffff;
    for (int i0 = 0; i0 < vocab; i0 += 1024 * AV) {
        float v[AV];
#pragma unroll
        for (int u = 0; u < AV; u++) {
            const int i = i0 + tid + 1024 * u;
            v[u] = i < vocab ? logits[i] : 0.0f;
        }
#pragma unroll
        for (int u = 0; u < AV; u++) {
            const int i = i0 + tid + 1024 * u;
            if (i < vocab) {
                if (v[u] > best) best = v[u], idx = i;   // i grows: a tie keeps the earlier index
                if (logits_out) logits_out[(size_t)p * vocab + i] = v[u];
            }
        }
    }
    for (int o = 32; o > 0; o >>= 1) {
        const float ov = __shfl_xor(best, o, 64);
        const int oi = __shfl_xor(idx, o, 64);
        if (ov > best || (ov == best && oi < idx)) best = ov, idx = oi;
    }
    if ((tid & 63) == 0) bv[tid >> 6] = best, bi[tid >> 6] = idx;
    __syncthreads();
    if (tid == 0) {
        for (int w = 1; w < 16; w++)
            if (bv[w] > best || (bv[w] == best && bi[w] < idx)) best = bv[w], idx = bi[w];
        st[1] = idx == 0x7fffffff ? 0 : idx;
        st[0] = p + 1;
        nxt = st[1];
    }
    // the next position's input row, as k_embed_ln would form it
    if (!next) return;
    __syncthreads();
    if (!in_prompt) {
        const float *e = en.emb + (size_t)nxt * en.d;
#pragma unroll
        for (int u = 0; u < 4; u++) {
            const int i = tid + 1024 * u;
            ev[u] = i < en.d ? e[i] : 0.0f;
        }
    }
    float v[4];
#pragma unroll
    for (int u = 0; u < 4; u++) v[u] = ev[u] + pv[u];
    ln_store<1024, 4>(v, en.d, en.w, en.b, en.x);
}

__global__ void k_bias_rows(float *__restrict__ y, const float *__restrict__ b, size_t rows, int d) {
    const size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < rows * (size_t)d) y[i] = y[i] + b[i % d];
}

__global__ void k_set_state(int *st, int p, int cur) {
    st[0] = p;
    st[1] = cur;
}

}  // namespace

int mh_att_splits(int n) { return mh_att_splits_dev(n); }

hipError_t mh_launch_embed_ln(const float *emb, const float *pos, const int *prompt, int n_prompt, const int *st,
                              const float *w, const float *b, float *x, int d, hipStream_t s) {
    if (d > LN_T * LN_V) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_embed_ln, dim3(1), dim3(LN_T), 0, s, emb, pos, prompt, n_prompt, st, w, b, x, d);
    return hipGetLastError();
}

hipError_t mh_launch_attend1(const float *q, float *K, float *V, const float *kn, const float *vn, const int *st,
                             int n_fixed, int d, int H, float *o_part, float *ml_part, int nsplit, float *out,
                             hipStream_t s) {
    const int dk = d / H;
    const float scale = 1.0f / sqrtf((float)dk);
    if (dk == 128) {
        hipLaunchKernelGGL(k_att_part<128>, dim3(H, nsplit), dim3(256), 0, s, q, K, V, kn, vn, st, n_fixed, d, scale,
                           o_part, ml_part, nsplit);
        if (out)
            hipLaunchKernelGGL(k_att_combine<128>, dim3(H), dim3(128), 0, s, o_part, ml_part, st, n_fixed, out, nsplit);
    } else if (dk == 64) {
        hipLaunchKernelGGL(k_att_part<64>, dim3(H, nsplit), dim3(256), 0, s, q, K, V, kn, vn, st, n_fixed, d, scale,
                           o_part, ml_part, nsplit);
        if (out)
            hipLaunchKernelGGL(k_att_combine<64>, dim3(H), dim3(64), 0, s, o_part, ml_part, st, n_fixed, out, nsplit);
    } else {
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t mh_launch_argmax(const float *logits, int vocab, int *st, float *logits_out, const MhEmbNext *en,
                            hipStream_t s) {
    if (en && en->emb && en->d > 4096) return hipErrorInvalidValue;
    hipLaunchKernelGGL(k_argmax, dim3(1), dim3(1024), 0, s, logits, vocab, st, logits_out, en ? *en : MhEmbNext{});
    return hipGetLastError();
}

hipError_t mh_launch_bias_rows(float *y, const float *b, size_t rows, int d, hipStream_t s) {
    const size_t n = rows * (size_t)d;
    if (n == 0) return hipSuccess;
    hipLaunchKernelGGL(k_bias_rows, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, y, b, rows, d);
    return hipGetLastError();
}

hipError_t mh_launch_set_state(int *st, int p, int cur, hipStream_t s) {
    hipLaunchKernelGGL(k_set_state, dim3(1), dim3(1), 0, s, st, p, cur);
    return hipGetLastError();
}
