/* cpb_synth.h -- deterministic synthetic weights and activations.
 *
 * Generates the bench workloads' tensors from (seed, stream) so that the
 * host here, the GPU box and every test produce identical bytes.  Counter
 * based (splitmix64 finaliser of key + index), so any slice can be generated
 * independently and in parallel.  Host-only; no GPU calls.
 *
 * No counterpart in the reference: its benches read a real GGUF blob
 * (bench_real.rs) or simulate int4 bytes (bench_moe.rs); there is no network
 * here for model files, so workloads are synthesised with the documented
 * distributions instead.
 */
#ifndef CPB_SYNTH_H
#define CPB_SYNTH_H
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* 64-bit word `i` of stream (seed, stream). */
uint64_t cpb_synth_u64(uint64_t seed, uint64_t stream, uint64_t i);

/* MXFP4 GGUF blocks: nblocks x 17 bytes; e8m0 byte = e_lo + U{0..e_span-1},
 * nibbles uniform over all 16 codes.  (bench config 0: e_lo=121, e_span=4
 * i.e. exponent uniform in [-6,-3].) */
void cpb_synth_mxfp4(uint8_t* out, size_t nblocks, int e_lo, int e_span, uint64_t seed, uint64_t stream);

/* fp32 N(mean, sigma^2) by Box-Muller in double precision. */
void cpb_synth_normal(float* out, size_t n, float mean, float sigma, uint64_t seed, uint64_t stream);

/* Q4_K superblocks (144 B): d, dmin = fp16 |N(0, dsig^2)|, scales and qs uniform. */
void cpb_synth_q4k(uint8_t* out, size_t nsuper, float dsig, uint64_t seed, uint64_t stream);
/* Q6_K superblocks (210 B): ql, qh, int8 scales uniform, d = fp16 |N(0, dsig^2)|. */
void cpb_synth_q6k(uint8_t* out, size_t nsuper, float dsig, uint64_t seed, uint64_t stream);

/* Zipf(s) router bias: a seeded permutation assigns rank r in 1..ne to each
 * expert; bias = ln(r^-s / sum_r' r'^-s). */
void cpb_synth_zipf_bias(float* out, int ne, float s, uint64_t seed, uint64_t stream);

/* fp32 -> IEEE half (round to nearest even), used for Q4_K/Q6_K d fields. */
uint16_t cpb_f32_to_half(float f);

#ifdef __cplusplus
}
#endif
#endif
