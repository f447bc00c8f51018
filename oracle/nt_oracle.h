/*
 * nt_oracle.h — scalar CPU restatement of mavenkim2/neural_textures' train/decode path.
 *
 * TEST INFRASTRUCTURE ONLY. This code is the parity checker for the HIP library and the
 * CPU baseline timed by bench.py; the product never links, loads or calls it. Only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg use it.
 *
 * It works on host memory laid out exactly as the device buffers described in
 * include/nt/nt.h (the same structs, holding host pointers). Every function cites the
 * reference file:line it restates. Floating-point policy (shared with the HIP kernels so
 * that both produce identical bits where the arithmetic is deterministic):
 *   - compiled with -ffp-contract=off; an explicit fmaf() stands wherever nvcc's default
 *     contraction would fuse a product into an add in the reference source;
 *   - fp16 conversions round to nearest even and keep subnormals;
 *   - MLP dot products accumulate in double here (the GPU accumulates in fp32 MFMA);
 *     results are compared with a tolerance, as the reference itself is order-
 *     nondeterministic (float atomics).
 *
 * Parity unpinned: the reference's MLP runs inside tiny-cuda-nn (mlp.h:7), which is not
 * in the reference tree (absent submodule, unknown commit). Its internal numerics
 * (accumulator precision, fp16 per-warp weight-gradient partials mlp.h:170-172,
 * activate_bwd at exactly 0) are not reproduced. ntref_mlp_forward_one beyond the 2-layer
 * known answers of tests/forward_pass_test.cu, and ntref_mlp_backward_one, are pinned by
 * mathematics only (float64 GEMM, finite differences), not by reference outputs.
 * Reference-texture sampling uses the exact 16-tap Catmull-Rom; the reference's 9 hardware
 * bilinear fetches with 8-bit fractional weights (filter/catmull_rom.h:76-86) are not
 * emulated.
 */
#ifndef NT_ORACLE_H
#define NT_ORACLE_H

#include <stdint.h>
#include "../include/nt/nt.h"

#ifdef __cplusplus
extern "C" {
#endif

/* ---- scalar helpers ---------------------------------------------------------------- */
uint16_t ntref_f32_to_f16(float f);
float ntref_f16_to_f32(uint16_t h);
uint16_t ntref_f16_add(uint16_t a, uint16_t b);
uint32_t ntref_xorshift32(uint32_t *state);
float ntref_uniform(uint32_t *state);
uint32_t ntref_sample_seed(uint32_t sample_index, int step);

/* MurmurHash3's 32-bit finalizer (texel placement of NT_SAMPLES_RANDOM). */
uint32_t ntref_fmix32(uint32_t h);
/* Sample position of sample i (train.cu:827-844; NT_SAMPLES_RANDOM as nt.h defines it):
 * writes (u, v, p->sample_mip) (z = 0 in the reference). */
void ntref_sample_uvz(const nt_params *p, uint32_t sample_index, float uvz[3]);

/* Latent sampling: bilinear/trilinear with fp16 accumulation (train.cu:263-314). */
void ntref_sample_latents_bilinear(const nt_latents *lat, const float uvz[3], uint16_t *out);
/* 16-tap Catmull-Rom on mip 0 of every grid, fp32 accumulation, fp16 result. */
void ntref_sample_latents_catmull_rom(const nt_latents *lat, const float uvz[3], uint16_t *out);
/* Differentiable BC6 block latents (train.cu:316-371). */
void ntref_sample_latents_bc6(const nt_latents *lat, const float uvz[3], uint16_t *out);

/* Latent gradient scatter of one sample: grads += corner weight * dinput
 * (train.cu:460-509), and its BC6 counterpart (train.cu:373-458). */
void ntref_scatter_unconstrained(const nt_latents *lat, const float uvz[3], const uint16_t *dinput);
void ntref_scatter_bc6(const nt_latents *lat, const float uvz[3], const uint16_t *dinput);

/* Catmull-Rom weights for fractional offset f (filter/catmull_rom.h:56-59). */
void ntref_catmull_rom_weights(float f, float w[4]);
/* Reference-texture sample with Catmull-Rom at mip coordinate z (train.cu:78-103). */
void ntref_sample_texture(const nt_texture *t, float u, float v, float z, float out[4]);
/* Target packing (train.cu:105-157). Returns the number of packed channels. */
int ntref_expected_values(const nt_params *p, const float uvz[3], float expected[16],
                          float weights[16]);

/* BC6 emulation (train.cu:159-202). */
float ntref_bc6_unquantize(float e, int bits);
float ntref_bc6_decompress(float e0, float e1, int bits, float x);
extern const int ntref_bc6_partition_sets[32];
extern const int ntref_bc6_partition_bits[10];

/* BC6 block initialisation from unconstrained latents (nt_bc6_init; no reference
 * counterpart). ntref_bc6_value_to_y inverts the BC6 decode's y -> value map;
 * ntref_bc6_fit_subset fits one partition subset (pixel mask) of a block [16][C] with a
 * line in y space and returns its decoded squared error; ntref_bc6_init_block picks the
 * partition of least total error and writes a block record; ntref_bc6_init does every
 * block of every mip of every grid (block_params from values). */
float ntref_bc6_value_to_y(float v);
float ntref_bc6_fit_subset(const float *v, const float *y, int C, int pixels, int bits, float *e0,
                           float *e1, float *x);
void ntref_bc6_init_block(const float *v, int C, int valid, float *rec);
int ntref_bc6_init(const nt_latents *lat);

/*
 * MLP forward for one sample (mlp.h:18-99). in: sizes[0] fp16. acts (optional): the
 * fp16 input of every layer, layer l at acts + l*64 (64 = max padded width), zero-padded.
 * out: padded output (AlignUp(sizes[L],16)) fp16.
 */
void ntref_mlp_forward_one(const nt_mlp *mlp, const uint16_t *in, uint16_t *acts,
                           uint16_t *out);
/*
 * MLP backward for one sample (mlp.h:222-362) given the saved layer inputs and the output
 * gradient dy (padded, fp16). Adds weight/bias gradients into the double accumulators
 * dw[l] (padIn*padOut) and db[l] (padOut); writes the fp16 input gradient (sizes[0]).
 */
void ntref_mlp_backward_one(const nt_mlp *mlp, const uint16_t *acts, const uint16_t *dy,
                            double **dw, double **db, uint16_t *dinput);

/* ---- whole passes (mirroring the C ABI) --------------------------------------------- */
int ntref_train_step(const nt_params *p, int type, int num_threads);
/* 1: ntref_train_step rounds each 32-sample weight-gradient partial to fp16 before summing
 * (the reference's __half2 warp partials, mlp.h:166-173); 0 (default): double sums. */
void ntref_set_dw_partial_fp16(int on);
/* 1: the MLP's forward and dY W^T sums accumulate in fp32 (index order); 0 (default): in
 * float64. Tests use the difference between the two as each element's sensitivity to the
 * order of fp32 sums. */
void ntref_set_mlp_accum_f32(int on);
int ntref_optimize_network(const nt_params *p);
int ntref_optimize_latents(const nt_params *p, int type);
int ntref_inference(const nt_params *p);
int ntref_mlp_forward(const nt_mlp *mlp, const uint16_t *inputs, uint16_t *outputs, int count);
int ntref_forward(const nt_latents *lat, const nt_mlp *mlp, int filter, const float *uvz,
                  int count, uint16_t *features, uint16_t *outputs);
/* Per-sample loss gradients and targets of a train step, for debugging and tests:
 * dy: [num_samples][16] fp16, target: [num_samples][16] fp32 (either may be NULL). */
int ntref_train_intermediates(const nt_params *p, int type, uint16_t *features, uint16_t *dy,
                              float *target);

/* Block codec (no reference counterpart). */
uint16_t ntref_codec_key(uint16_t h);
uint16_t ntref_codec_unkey(uint16_t k);
uint16_t ntref_codec_interp(uint16_t k0, uint16_t k1, int index);
int ntref_codec_encode(const float *values, int width, int height, int channels,
                       uint8_t *blocks);
int ntref_codec_decode(const uint8_t *blocks, int width, int height, int channels,
                       float *values);
/* Decode a full image from codec latents (mirrors nt_decode). */
int ntref_decode(const nt_decode_params *p, int num_threads);
/* The pixels [x0, x0 + w) x [y0, y0 + h) of that image (their jitter and mip as in the full
 * image), written row-major to p->output as a w x h image. */
int ntref_decode_rect(const nt_decode_params *p, int x0, int y0, int w, int h, int num_threads);
/* Thread count of the oracle's OpenMP loops that take none (the codec). */
void ntref_set_threads(int n);

#ifdef __cplusplus
}
#endif

#endif
