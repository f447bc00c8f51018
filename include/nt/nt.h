/*
 * nt.h — C ABI of the MI355X (gfx950) neural-texture train/decode hot path.
 *
 * This header is the drop-in boundary. It replaces the reference's four C++ launchers
 * (mavenkim2/neural_textures train.h:158-161):
 *
 *   void InvokeOptimizeNetwork(KernelParams);                    -> nt_optimize_network
 *   void InvokeOptimizeFeatures(KernelParams, TrainingKernelType); -> nt_optimize_latents
 *   void InvokeTraining(KernelParams, TrainingKernelType);       -> nt_train_step
 *   void InvokeInference(KernelParams);                          -> nt_inference
 *
 * and adds the codec and decode entry points that the reference does not have
 * (nt_codec_encode / nt_codec_decode / nt_decode), plus the tiny-MLP forward used by the
 * reference's only unit test (tests/forward_pass_test.cu:15-32) and the Catmull-Rom latent
 * forward pass (nt_forward).
 *
 * Contract (same as the reference unless stated):
 *  - Every buffer is caller-owned device memory (hipMalloc or torch); the library never
 *    allocates. Scratch space for the train step is passed in nt_params.workspace; its size
 *    comes from nt_train_workspace_bytes().
 *  - nt_train_step ACCUMULATES into the network and latent gradient buffers, which must
 *    start at zero; nt_optimize_network / nt_optimize_latents consume the gradients and
 *    re-zero them (train.cu:586, 621, 638).
 *  - All work is enqueued on the given stream (a hipStream_t passed as void*, NULL = the
 *    null stream) and is asynchronous; nothing synchronises.
 *  - Errors are reported as nt_status codes, never as exceptions; nt_last_error() returns a
 *    human-readable message for the last failing call on the calling thread. Argument
 *    checking happens before anything is enqueued: a failing call enqueues nothing.
 *  - Calls that share buffers must not overlap (the reference is not re-entrant either).
 *
 * Floating-point numbers use the reference's formats: fp32 latents, gradients and Adam
 * moments; fp16 (IEEE binary16, passed as uint16_t bit patterns) network weights, biases
 * and sampled features.
 */
#ifndef NT_NT_H
#define NT_NT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define NT_ABI_VERSION 2

#define NT_MAX_GRIDS 4     /* NT_NUM_FEATURES (train.h:18) is the reference's fixed count */
#define NT_MAX_MIPS 16
#define NT_MAX_LAYERS 6    /* weight layers; the reference has NT_NUM_NETWORK_LAYERS = 3 */
#define NT_MAX_TEXTURES 16 /* NT_MAX_REFERENCE_TEXTURES (train.h:19) */
#define NT_MAX_OUTPUTS 16  /* NT_OUTPUT_SIZE (train.h:11) */
#define NT_DEFAULT_REGION 512 /* kTrainingRegionSize (train.cu:827) */

typedef enum nt_status {
    NT_OK = 0,
    NT_ERR_INVALID_ARGUMENT = 1, /* bad shape, count or enum value */
    NT_ERR_NULL_POINTER = 2,     /* a required buffer pointer is NULL */
    NT_ERR_MISALIGNED = 3,       /* a buffer is not aligned as documented */
    NT_ERR_UNSUPPORTED = 4,      /* valid, but no kernel is built for this shape */
    NT_ERR_WORKSPACE = 5,        /* workspace missing or smaller than required */
    NT_ERR_HIP = 6,              /* the HIP runtime reported an error (launch) */
    NT_ERR_FORMAT = 7            /* a model image fails its checks (nt_model_load) */
} nt_status;

/* Mirrors TrainingKernelType (train.h:22-27). */
typedef enum nt_kernel_type {
    NT_UNCONSTRAINED = 0, /* float latents (train.cu:263-314, 460-509, 764-803) */
    NT_BLOCK_FEATURES = 1, /* differentiable BC6 block latents (train.cu:316-458, 728-762) */
    NT_FINALIZE = 2        /* BC6 latents, no latent gradient (train.cu:906-913) */
} nt_kernel_type;

/* Latent filter used when sampling the latent grids. */
typedef enum nt_filter {
    NT_FILTER_BILINEAR = 0,   /* trilinear over mips, fp16 accumulation (train.cu:263-314) */
    NT_FILTER_CATMULL_ROM = 1 /* 16-tap Catmull-Rom on mip 0 (forward only, nt_forward) */
} nt_filter;

/*
 * Where the samples of a train step sit. NT_SAMPLES_REGION is the reference's
 * (train.cu:827-844): sample i at texel (texel_offset_x + i % region_width,
 * texel_offset_y + i / region_width), jittered by U[-0.5, 0.5) per axis. NT_SAMPLES_RANDOM
 * (no reference counterpart): sample i at a uniformly random texel of the whole image,
 * x = min(floor(U(h1) * image_width), image_width - 1), y likewise from U(h2), then the
 * same jitter; h1 = fmix32(seed), h2 = fmix32(h1) with fmix32 the MurmurHash3 finalizer and
 * seed the sample's RNG seed (train.cu:833), U(h) = (h & 0xFFFFFF) * 2^-24. (The
 * reference's xorshift draws of consecutive seeds are too correlated to place texels.)
 * Region fields are unused.
 */
typedef enum nt_sample_mode {
    NT_SAMPLES_REGION = 0,
    NT_SAMPLES_RANDOM = 1
} nt_sample_mode;

/*
 * What nt_optimize_latents visits. NT_LATENT_DENSE is the reference's (train.cu:764-803,
 * 641-679): every texel (or block record) of every mip, lazy per value. NT_LATENT_TOUCHED
 * (no reference counterpart, same results): the last 256 bytes of params->workspace hold an
 * update log. A train step of the 16-channel kernel records there the texel rectangle of
 * each grid that its samples' bilinear footprints can reach, and a BC6-phase step
 * (NT_BLOCK_FEATURES) of the reference network with region sampling the rectangle of mip-0
 * block records under them; when exactly one such step was logged since the last optimizer
 * call and the optimizer's kernel type matches (texels for NT_UNCONSTRAINED, blocks
 * otherwise), nt_optimize_latents updates only those rectangles (lazy per value as before),
 * and everything otherwise (several steps accumulated, another kernel, a fresh workspace).
 * Values outside the rectangles hold zero gradients, which the lazy rule skips, so the
 * update is the same; this holds when every gradient since the last optimizer call came
 * from nt_train_step calls with this workspace (a caller that writes latent gradients itself
 * uses NT_LATENT_DENSE). A fresh workspace needs no initialisation. NT_LATENT_TOUCHED needs
 * params->workspace in nt_optimize_latents too. nt_train_step_static keeps no log and
 * refuses NT_LATENT_TOUCHED.
 */
typedef enum nt_latent_update {
    NT_LATENT_DENSE = 0,
    NT_LATENT_TOUCHED = 1
} nt_latent_update;

/* Mirrors AdamConstants (train.h:29-35). */
typedef struct nt_adam {
    float beta1;
    float beta2;
    float learning_rate;
    float epsilon;
} nt_adam;

/*
 * One latent grid (a reference `Feature`, train.h:51-67) with its mip chain.
 *
 * Unconstrained storage: all mips are flattened into one buffer per quantity. Mip m is
 * max(width>>m,1) x max(height>>m,1) texels starting at texel mip_offset[m]; texel t of the
 * buffer holds `channels` consecutive floats at [t*channels, (t+1)*channels). With
 * channels = 3 this is exactly the reference's float3 row-major layout (train.cu:306).
 *
 * Block (BC6) storage, used by NT_BLOCK_FEATURES / NT_FINALIZE: mip m has
 * max(w_m>>2,1) x max(h_m>>2,1) blocks starting at block block_offset[m]. A block record of
 * block_params is (4*channels + 16) floats followed by two int32 (partition, mode): for
 * channels = 3 it is the reference's 120-byte BC6Parameters (train.h:37-43). Gradient and
 * moment records are (4*channels + 16) floats (BC6ParameterGradients, train.h:45-49).
 */
typedef struct nt_grid {
    int width;
    int height;
    int num_mips;
    int reserved0;
    int64_t mip_offset[NT_MAX_MIPS];
    float *values;
    float *grads;
    float *moment1;
    float *moment2;
    int64_t block_offset[NT_MAX_MIPS];
    float *block_params;
    float *block_grads;
    float *block_moment1;
    float *block_moment2;
} nt_grid;

typedef struct nt_latents {
    int num_grids; /* 1..NT_MAX_GRIDS */
    int channels;  /* per grid: 3, 4, 8 or 16 */
    nt_grid grids[NT_MAX_GRIDS];
} nt_latents;

/*
 * The tiny MLP (mlp.h). Layer l maps sizes[l] inputs to sizes[l+1] outputs; ReLU follows
 * every layer but the last. Weights are fp16, column-major and padded to multiples of 16
 * in both dimensions: W_l[col * AlignUp(sizes[l],16) + row], row = input, col = output
 * (main.cpp:195, train.h:96-118); padding entries must be zero. Biases are sizes[l+1]
 * fp16 values. Gradients and Adam moments are fp32 with the same layouts.
 * used_outputs (<= sizes[num_layers]) is the reference's usedOutputChannels: the last
 * layer's Adam update touches only its first used_outputs columns (train.cu:704-706).
 */
typedef struct nt_mlp {
    int num_layers; /* 2..NT_MAX_LAYERS */
    int sizes[NT_MAX_LAYERS + 1];
    int used_outputs;
    uint16_t *weights[NT_MAX_LAYERS];
    float *weight_grads[NT_MAX_LAYERS];
    float *weight_moment1[NT_MAX_LAYERS];
    float *weight_moment2[NT_MAX_LAYERS];
    uint16_t *biases[NT_MAX_LAYERS];
    float *bias_grads[NT_MAX_LAYERS];
    float *bias_moment1[NT_MAX_LAYERS];
    float *bias_moment2[NT_MAX_LAYERS];
} nt_mlp;

/*
 * A reference texture (train.h:69-77), in plain device memory instead of a CUDA texture
 * object. texels holds the mip chain flattened like nt_grid: texel t of mip m is at
 * [(mip_offset[m] + t) * pitch, ... + num_channels). pitch is 4 for 2..4 channels
 * (the reference uploads 3-channel EXRs as float4, main.cpp:215-222) and 1 or 4 for one
 * channel; addressing wraps (main.cpp:613-621).
 */
typedef struct nt_texture {
    const float *texels;
    int width;
    int height;
    int num_channels;
    int num_mips;
    int pitch;
    float loss_weight;
    int64_t mip_offset[NT_MAX_MIPS];
} nt_texture;

/*
 * Everything one launch needs, mirroring KernelParams (train.h:120-157), passed by pointer.
 */
typedef struct nt_params {
    nt_latents latents;
    nt_mlp mlp;
    nt_adam network_adam;
    nt_adam feature_adam;
    nt_texture textures[NT_MAX_TEXTURES];
    int num_textures;

    int image_width; /* sampling domain in texels (the reference textures' size) */
    int image_height;
    int texel_offset_x; /* training region origin (main.cpp:1043-1044) */
    int texel_offset_y;
    int region_width;   /* samples per region row; 0 means NT_DEFAULT_REGION */
    int num_samples;    /* batch size; sample i sits at (i % region_width, i / region_width) */
    int step;           /* Adam step; bias correction uses max(step, 1) (train.cu:528) */
    int sample_mode;    /* NT_SAMPLES_REGION (the reference) or NT_SAMPLES_RANDOM */
    float sample_mip;   /* mip coordinate z of every train sample: the reference uses 0
                           (train.cu:844); z > 0 samples the latents trilinearly across
                           mips floor(z), floor(z)+1 (train.cu:263-314) and the targets
                           with trilinear Catmull-Rom across their mips (train.cu:78-103) */
    int latent_update;  /* nt_latent_update: NT_LATENT_DENSE (the reference) or
                           NT_LATENT_TOUCHED */

    float *inference_output;   /* nt_inference: [pixel][sizes[num_layers]] fp32 */
    float *inference_mse_accum; /* nt_inference: SSE accumulator (one float) */

    void *workspace; /* nt_train_step scratch, see nt_train_workspace_bytes; with
                        NT_LATENT_TOUCHED its last 256 bytes hold the update log */
    size_t workspace_bytes;
} nt_params;

/* ---- layout helpers (host-only, no GPU needed) ------------------------------------- */

int nt_abi_version(void);
const char *nt_status_string(int status);
/* Message for the last failing call on this thread ("" if none). */
const char *nt_last_error(void);

/* Fills mip_offset[0..num_mips) for a flattened mip chain and returns the total texel
 * count (or -1 on a bad argument). Mip m has max(w>>m,1) x max(h>>m,1) texels. */
int64_t nt_mip_chain_layout(int width, int height, int num_mips, int64_t *mip_offset);
/* The same for 4x4 block storage (blocks per dimension = max(size>>2, 1), train.cu:220). */
int64_t nt_block_chain_layout(int width, int height, int num_mips, int64_t *block_offset);
/* Bytes of scratch nt_train_step needs for these parameters (0 on error); also enough for
 * nt_inference's fixed-order SSE. A NT_SAMPLES_RANDOM step of 262,144 samples or more also
 * holds its sample sort (keys, sample indices and per-tile counts, ~12 bytes a sample). */
size_t nt_train_workspace_bytes(const nt_params *params, nt_kernel_type type);

/* Profiling hook (no reference counterpart): the next nt_train_step, nt_optimize_latents,
 * nt_inference, nt_forward, nt_mlp_forward, nt_decode, nt_codec_encode or nt_codec_decode
 * on this thread records `start` right before and `stop` right after its main kernel, on
 * that call's stream. Both are hipEvent_t passed as void*; NULL clears. One-shot. */
int nt_profile_next_launch(void *start_event, void *stop_event);

/* Test hooks (no reference counterpart; for this library's own tests, not for production
 * runs). Process-wide, taking effect at the next nt_train_step:
 *   max_train_workgroups > 0 caps the 16-channel train kernel's workgroups (0: one per
 *   compute unit), so that small regions give each workgroup several tiles;
 *   flags bit 0 (NT_HOOK_DROP_MARGINS) removes the margin of that kernel's chunk cell box,
 *   which drives its latent scatter's out-of-box path (per-sample global atomics);
 *   flags bit 1 (NT_HOOK_SORT_RANDOM) makes NT_SAMPLES_RANDOM steps sort their samples by
 *   bin at any sample count (they do from 262,144 samples), so that small tests reach
 *   the sorted order.
 * nt_set_test_hooks(0, 0) restores the defaults. */
#define NT_HOOK_DROP_MARGINS 1
#define NT_HOOK_SORT_RANDOM 2
int nt_set_test_hooks(int max_train_workgroups, int flags);
/* Test hook (no reference counterpart): the order in which nt_train_step with these
 * parameters (NT_UNCONSTRAINED) would read its NT_SAMPLES_RANDOM samples, written to
 * order[0 .. num_samples) on the device: the sample indices sorted stably by the
 * 64 x 64-texel bin (row-major over the image) of their texels. Uses params->workspace
 * (nt_train_workspace_bytes). NT_ERR_UNSUPPORTED when the step trains in slot order
 * (fewer than 262,144 samples without NT_HOOK_SORT_RANDOM, or another kernel). */
int nt_random_sample_order(const nt_params *params, uint32_t *order, void *stream);

/* ---- the hot path ----------------------------------------------------------------- */

/*
 * One fused training pass over params->num_samples samples (InvokeTraining,
 * train.cu:1028-1048 -> TrainLoopPass :818-915): jittered sample position, latent sample,
 * Catmull-Rom target, MLP forward, L2 loss gradient, MLP backward, latent gradient scatter.
 * Accumulates into mlp.*_grads and the latent gradients.
 */
int nt_train_step(const nt_params *params, nt_kernel_type type, void *stream);

/*
 * nt_train_step without a workspace: the same kernels, with their scratch (the per-workgroup
 * MLP-gradient partials, the prepared weight image of the general kernel, and the texels the
 * BC6 block phase expands) in a static device array of nt_train_static_scratch_bytes() =
 * 32 MiB. The array is part of the library's code object: it is reserved on every GPU on
 * which the process loads the library (any nt_* kernel launch there), whether or not this
 * entry point is ever called, and held until the process ends. params->workspace is ignored. No reference
 * counterpart: this entry point is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc); it calls
 * no allocating routine. A step whose scratch exceeds the array fails with
 * NT_ERR_WORKSPACE before anything is enqueued (the 16-channel kernel needs at most one
 * gradient row per compute unit: 13.8 MB at the 4-grid network). Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (two streams, two threads) race
 * and must be serialised by the caller. Nothing in the array needs to start at zero.
 */
int nt_train_step_static(const nt_params *params, nt_kernel_type type, void *stream);
size_t nt_train_static_scratch_bytes(void);

/* Lazy Adam on the MLP (InvokeOptimizeNetwork, train.cu:985-988 -> :681-726). */
int nt_optimize_network(const nt_params *params, void *stream);

/* Lazy Adam on every texel (or block) of every grid and mip
 * (InvokeOptimizeFeatures, train.cu:990-1026 -> :728-816). */
int nt_optimize_latents(const nt_params *params, nt_kernel_type type, void *stream);

/* One iteration of the reference's training loop body (main.cpp:1071-1076, the calls
 * InvokeTraining, InvokeOptimizeNetwork, InvokeOptimizeFeatures): the same as nt_train_step,
 * nt_optimize_network and nt_optimize_latents called in that order, bit for bit. With
 * every kernel type the MLP-gradient reduction and both optimizers (latent texels or block
 * records) share one launch after the train step (two launches fewer per iteration). Every
 * argument of all three is checked before anything is enqueued. */
int nt_train_iteration(const nt_params *params, nt_kernel_type type, void *stream);

/* Full-image inference at texel centres, mip 0 (InvokeInference, train.cu:1050-1062 ->
 * :917-961): writes inference_output and adds the squared error to inference_mse_accum.
 * With params->workspace of at least nt_inference_workspace_bytes (every train workspace
 * of the same params is), the squared errors are summed in a fixed order, so the SSE is
 * the same bits on every run; without one, partial sums are added atomically in arrival
 * order, as the reference does (train.cu:960). */
int nt_inference(const nt_params *params, void *stream);
/* Workspace bytes for the fixed-order SSE of nt_inference (0 on a bad argument). */
size_t nt_inference_workspace_bytes(const nt_params *params);

/*
 * Tiny-MLP forward on given fp16 inputs (the ForwardPass* functions of mlp.h:18-99, as
 * exercised by tests/forward_pass_test.cu). inputs: [count][sizes[0]] fp16;
 * outputs: [count][sizes[num_layers]] fp16.
 */
int nt_mlp_forward(const nt_mlp *mlp, const uint16_t *inputs, uint16_t *outputs, int count,
                   void *stream);

/*
 * Latent sample + MLP forward at caller-given coordinates. uvz: [count][3] fp32 (u, v, mip).
 * filter selects bilinear/trilinear (train.cu:263-314) or 16-tap Catmull-Rom on mip 0.
 * features (optional, may be NULL): [count][G*C] fp16 sampled features;
 * outputs: [count][sizes[num_layers]] fp16.
 */
int nt_forward(const nt_latents *latents, const nt_mlp *mlp, nt_filter filter,
               const float *uvz, int count, uint16_t *features, uint16_t *outputs,
               void *stream);

/* ---- the block codec -------------------------------------------------------------- */

/*
 * Initialises every grid's BC6 block records (block_params, all mips) from its
 * unconstrained latents (values), for the switch from NT_UNCONSTRAINED to
 * NT_BLOCK_FEATURES training. No reference counterpart: the reference zero-fills its block
 * records (main.cpp:689-694) and its schedule (main.cpp:1052-1060) would start the block
 * phase from those. Per 4x4 block: values, clamped to the decode's range [0, 65504]
 * (unsigned half: negative latents become 0), are mapped to the BC6 decode's linear domain
 * (train.cu:159-181), each of the 32 two-subset partitions is fitted with one line per
 * subset, and the partition whose record decodes with the least squared error is written
 * (mode 0, pixel indices in [0, 1]). Channels 3, 4, 8 or 16; grid sizes multiples of 4
 * (or at most 4). Block gradients and moments are not touched.
 */
int nt_bc6_init(const nt_latents *latents, void *stream);

/*
 * BC6H-style block codec for latent grids (no reference counterpart: the reference has no
 * encoder). Each 4x4 texel block stores, per channel, two fp16 endpoints and sixteen 4-bit
 * indices; a texel decodes to the fp16 whose order key is the BC6H 4-bit interpolation of
 * the endpoint keys. Block record (channels multiple of 4): endpoints [channels][2] uint16,
 * then for each of the 16 block pixels a channels*4-bit index word -> 12*channels bytes.
 * Blocks per dimension = ceil(size / 4); texels outside the image are ignored.
 */
size_t nt_codec_block_bytes(int channels);
size_t nt_codec_mip_chain_layout(int width, int height, int num_mips, int channels,
                                 int64_t *byte_offset);
/* values: [height*width][channels] fp32 (one mip); blocks: ceil(h/4)*ceil(w/4) records. */
int nt_codec_encode(const float *values, int width, int height, int channels, void *blocks,
                    void *stream);
int nt_codec_decode(const void *blocks, int width, int height, int channels, float *values,
                    void *stream);

/* A grid quantized with the codec: mip m's blocks start at byte byte_offset[m]. */
typedef struct nt_codec_grid {
    int width;
    int height;
    int num_mips;
    int reserved0;
    int64_t byte_offset[NT_MAX_MIPS];
    const void *blocks;
} nt_codec_grid;

typedef struct nt_decode_params {
    int num_grids;
    int channels; /* 16 (multiple of 4) */
    nt_codec_grid grids[NT_MAX_GRIDS];
    nt_mlp mlp;       /* weights and biases only */
    int out_width;    /* output image size in pixels */
    int out_height;
    uint32_t seed;    /* per-pixel jitter / mip RNG seed */
    float jitter;     /* jitter amplitude in output pixels (1 -> U[-0.5, 0.5)) */
    float mip_min;    /* mip coordinate z ~ U[mip_min, mip_max) */
    float mip_max;
    uint16_t *output; /* [pixel][mlp.used_outputs] fp16 */
    /* Optional scratch (NULL: none). With nt_decode_workspace_bytes() bytes the decode runs
     * in two passes: every block is first expanded once into fp16 texels, then the pixels
     * sample those. Same results, fewer operations per pixel. 16-byte aligned. */
    void *workspace;
    size_t workspace_bytes;
} nt_decode_params;

/* Workspace bytes for the two-pass decode (0 on a bad argument). */
size_t nt_decode_workspace_bytes(const nt_decode_params *params);

/*
 * Decode a full image from codec-quantized latents: per pixel, jittered UV and random mip,
 * trilinear sample of every grid, MLP forward, fp16 output.
 */
int nt_decode(const nt_decode_params *params, void *stream);

/* ---- model container ----------------------------------------------------------------
 *
 * A versioned, checksummed file image of a neural texture (no reference counterpart: the
 * reference writes only PNG renders, main.cpp:855-904). It always holds the fp16 network;
 * with NT_MODEL_CODEC the codec-quantized latent mip chains (what nt_decode reads), and
 * with NT_MODEL_STATE the training state (fp32 unconstrained latents, their Adam moments,
 * the network's Adam moments and the step) so a training run resumes from it, and with
 * NT_MODEL_BLOCKS the BC6 block records and their moments (a run in its block phase).
 * Host memory only; moving buffers to and from the device is the caller's.
 *
 * Image (little-endian): a 64-byte header {"NTMODEL\0", version, header bytes, section
 * count, contents, image bytes, crc32 of the description and the section table}, the
 * description (32 int32: the fields of nt_model_info in order, zero padded), a table of
 * 32-byte section entries {type, index, offset, bytes, crc32}, then the sections, each at
 * a 256-byte aligned offset. A reader accepts images of its version only and checks every
 * size and checksum.
 */
#define NT_MODEL_VERSION 1
#define NT_MODEL_CODEC 1u /* codec mip chains */
#define NT_MODEL_STATE 2u /* training state */
#define NT_MODEL_BLOCKS 4u /* BC6 block records and their Adam moments (with NT_MODEL_STATE) */

typedef struct nt_model_info {
    uint32_t contents; /* NT_MODEL_CODEC | NT_MODEL_STATE (at least one) | NT_MODEL_BLOCKS */
    int num_grids;     /* 1..NT_MAX_GRIDS */
    int channels;      /* per grid: 1..16; 4, 8, 12 or 16 with NT_MODEL_CODEC */
    int width[NT_MAX_GRIDS];
    int height[NT_MAX_GRIDS];
    int num_mips[NT_MAX_GRIDS]; /* 1..NT_MAX_MIPS */
    int num_layers;             /* network as nt_mlp: 1..NT_MAX_LAYERS */
    int sizes[NT_MAX_LAYERS + 1]; /* 1..1024 */
    int used_outputs;             /* 1..sizes[num_layers] */
    int step;                     /* Adam step of the training state (0 without it) */
} nt_model_info;

/*
 * Host buffers of one model, in the layouts of nt_mlp and nt_grid:
 *   codec[g]       grid g's codec mip chain, nt_codec_mip_chain_layout bytes (CODEC)
 *   weights[l]     fp16 bits, AlignUp(sizes[l],16) x AlignUp(sizes[l+1],16)
 *   biases[l]      fp16 bits, sizes[l+1]
 *   latents[g], latent_moment1[g], latent_moment2[g]   fp32 [texel][channels] over grid
 *                  g's mips back to back (mip m after the texels of mips < m) (STATE)
 *   weight_moment1/2[l], bias_moment1/2[l]   fp32, as weights / biases (STATE)
 *   block_params[g]  grid g's block records over its mips, (4 channels + 18) x 4 bytes
 *                    each (nt_grid's block layout); block_moment1/2[g] the
 *                    (4 channels + 16)-float moment records (BLOCKS)
 * nt_model_load points these into the image (zero copy) and sets absent ones to NULL.
 */
typedef struct nt_model_data {
    const void *codec[NT_MAX_GRIDS];
    const uint16_t *weights[NT_MAX_LAYERS];
    const uint16_t *biases[NT_MAX_LAYERS];
    const float *latents[NT_MAX_GRIDS];
    const float *latent_moment1[NT_MAX_GRIDS];
    const float *latent_moment2[NT_MAX_GRIDS];
    const float *weight_moment1[NT_MAX_LAYERS];
    const float *weight_moment2[NT_MAX_LAYERS];
    const float *bias_moment1[NT_MAX_LAYERS];
    const float *bias_moment2[NT_MAX_LAYERS];
    const float *block_params[NT_MAX_GRIDS];
    const float *block_moment1[NT_MAX_GRIDS];
    const float *block_moment2[NT_MAX_GRIDS];
} nt_model_data;

/* Bytes of the image of a model (0 on a bad description, reason in nt_last_error). */
size_t nt_model_bytes(const nt_model_info *info);
/* Writes the image into out (16-byte aligned, out_bytes >= nt_model_bytes). */
int nt_model_save(const nt_model_info *info, const nt_model_data *data, void *out,
                  size_t out_bytes);
/* Checks an image (magic, version, description, table, checksums; in 16-byte aligned) and
 * fills info and data, whose pointers point into in. NT_ERR_FORMAT if the checks fail. */
int nt_model_load(const void *in, size_t in_bytes, nt_model_info *info, nt_model_data *data);

#ifdef __cplusplus
}
#endif

#endif /* NT_NT_H */
