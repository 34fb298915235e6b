/*
 * msplat_synth.h -- seeded random streams for synthetic scenes (host only).
 *
 * The reference initialises splats from loaded point clouds or uniform
 * random points (input_data.hpp initializeRandomPoints, model.cpp:43-121,
 * using std::mt19937); the benchmark workloads here are synthetic, so the
 * engine ships a portable counter-based generator instead: element i of a
 * stream with seed s is SplitMix64 applied to s + (i+1) * 0x9E3779B97F4A7C15
 * (Steele, Lea & Flood 2014), so a stream gives the same values on every
 * host and can be consumed from any offset.
 */
#ifndef MSPLAT_SYNTH_H
#define MSPLAT_SYNTH_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* out[k] = lo + (hi - lo) * U(offset + k), U in [0, 1) with 53-bit
 * resolution, computed in double and rounded to float. */
void msplat_synth_uniform(uint64_t seed, uint64_t offset, int64_t n, double lo,
                          double hi, float *out);

/* Box-Muller normals: pair j uses u1 = 1 - U(offset + 2j), u2 =
 * U(offset + 2j + 1) and yields r*cos(2 pi u2), r*sin(2 pi u2) with
 * r = sqrt(-2 ln u1); out[k] = mean + std * z_k.  Consumes 2*ceil(n/2)
 * stream elements. */
void msplat_synth_normal(uint64_t seed, uint64_t offset, int64_t n, double mean,
                         double std, float *out);

#ifdef __cplusplus
}
#endif

#endif
