/* Synthetic inputs and GGUF-block quantizers for the MoE-layer configurations.
 *
 * No counterpart in the reference: Ingot only reads GGUF files (src/gguf.rs)
 * and never quantizes. The benchmark configurations fix
 * distributions (weights N(0, 0.02) before quantization, x ~ N(0, 1), Zipf
 * router bias, U(-0.1, 0.1) correction bias), so this library draws them from
 * seeded SplitMix64 streams (Box-Muller in double, rounded to float) and
 * encodes them into the same block layouts the loader accepts
 * (src/gguf.rs:470-491). Both the GPU path and the CPU path consume these
 * exact bytes. Host-only code, no GPU needed.
 *
 * Streams: every generated row r of a tensor uses its own SplitMix64 state
 * ingot_synth_stream(key, r, 0, 0), so rows are independent and generation is
 * parallel and reproducible on any thread count.
 */
#pragma once
#include <stdint.h>
#ifdef __cplusplus
extern "C" {
#endif

/* A 64-bit stream key from up to four components (config, layer, tensor, expert...). */
uint64_t ingot_synth_stream(uint64_t a, uint64_t b, uint64_t c, uint64_t d);

/* out[r][j] = mean + sigma * N(0,1) for rows x cols, row r from stream (key, r). */
void ingot_synth_normal(uint64_t key, uint64_t rows, uint64_t cols, float mean, float sigma,
                        float* out, int threads);
/* out[r][j] ~ U(lo, hi). */
void ingot_synth_uniform(uint64_t key, uint64_t rows, uint64_t cols, float lo, float hi,
                         float* out, int threads);

/* Round every value to bfloat16 (round to nearest even) and back to float. */
void ingot_round_bf16(float* x, uint64_t n);

/* IEEE binary16 conversions (round to nearest even). */
uint16_t ingot_f32_to_f16(float f);
float ingot_f16_to_f32(uint16_t h);

/* Row stride in bytes of a `cols`-wide row of GGML type `kind`; 0 if the kind
 * has no quantizer here or cols is not a multiple of its block. */
uint64_t ingot_quant_row_bytes(uint32_t kind, uint64_t cols);

/* Quantize rows x cols floats into GGUF blocks of type kind
 * (0 F32, 2 Q4_0, 8 Q8_0, 12 Q4_K, 17 IQ2_XS, 18 IQ3_XXS, 20 IQ4_NL).
 * dst holds rows * ingot_quant_row_bytes(kind, cols) bytes. Returns 0 on success. */
int ingot_quantize(uint32_t kind, const float* src, uint64_t rows, uint64_t cols, uint8_t* dst,
                   int threads);

/* Generate N(0, sigma) weights for `count` matrices of rows x cols (row r of
 * matrix e from stream (key, e * rows + r)) and quantize them into dst, never
 * holding more than a few rows of floats per thread. Returns 0 on success. */
int ingot_synth_quantized(uint32_t kind, uint64_t key, uint64_t count, uint64_t rows,
                          uint64_t cols, float sigma, uint8_t* dst, int threads);

#ifdef __cplusplus
}
#endif
