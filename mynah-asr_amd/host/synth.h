/* synth.h — weight preparation and seeded synthetic inputs.
 *
 * Quantizers into the ggml block formats (load/export time, CPU): Q8_0, Q4_0,
 * Q4_K and Q6_K follow the reference's own quantizers bit for bit
 * (third_party/ingot/src/quantize.c:49-71, 129-168; kernels.c:175-318).
 * Q2_K, Q3_K and Q5_K have no quantizer in the reference (docs/gguf.md:87-94);
 * the ones here are this library's own simple range fits, used to make
 * benchmark and test weights.
 *
 * mynah_synth_randn: the generator that defines "N(0, sigma), seed s" for
 * every benchmark and test input: SplitMix64 -> Box-Muller in double -> f32. */
#ifndef MYNAH_SYNTH_H
#define MYNAH_SYNTH_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[i] = (float)(sigma * z_i), z = standard normal stream of seed `seed`. */
void mynah_synth_randn(uint64_t seed, double sigma, float *out, size_t n);

/* f32 [count] -> ggml blocks; qtype uses the MYNAH_ASR_HIP_* ids.
 * Returns the bytes written, 0 for an unsupported format / count. */
size_t mynah_synth_quantize(int qtype, const float *x, size_t count, void *out);

/* bytes of `count` elements in a block format (0 if unsupported) */
size_t mynah_synth_nbytes(int qtype, size_t count);

#ifdef __cplusplus
}
#endif
#endif
