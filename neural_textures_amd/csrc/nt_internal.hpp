// nt_internal.hpp — launch descriptors passed by value to the gfx950 kernels, and the
// internal launcher entry points the C ABI (nt_api.cpp) dispatches to. Descriptors carry
// only what a kernel reads, so kernel arguments stay small.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/nt/nt.h"
#include "nt_mlp.hpp"

namespace ntk {

// Samples per workgroup chunk in the train kernel: a 16 x 8 block of region positions,
// four waves of 32 samples (one 32-sample MFMA tile per wave).
constexpr int kChunkW = 16;
constexpr int kChunkH = 8;
constexpr int kChunk = kChunkW * kChunkH;
constexpr int kTrainThreads = 256;
constexpr int kRowStride = kChunk + 8; // fp16 row stride of the LDS transposes
// fp16 row stride of the 16-channel kernel's sample rows: 34 dwords, so that the 8-byte
// stores of 16 consecutive rows (what gfx950's LDS serves per cycle) hit distinct banks.
constexpr int kFeatStride = 68;
// ... and of its dX0 rows (k0 inputs): k0 + 4 halves (an odd number of 8-byte chunks) puts
// the 8-byte stores of 16 consecutive rows in distinct LDS banks.
__host__ __device__ constexpr int dx_stride(int k0) { return k0 + 4; }
// Catmull-Rom target tile of one chunk: texels [cx0-3, cx0+20) x [cy0-3, cy0+12) of every
// reference texture, float4 each (covers all 16 taps of every jittered sample of the chunk).
constexpr int kTileX0 = 3;
constexpr int kTileW = kChunkW + 7;
constexpr int kTileH = kChunkH + 7;
// The 16-channel train kernel's tile: texels [cx0-2, cx0+18) x [cy0-2, cy0+10) of every
// texture, exactly the Catmull-Rom taps of a chunk's jittered positions (a position in
// texel x has taps x-2 .. x+2), in rows of 32 float4 slots: rows 256-byte multiples apart,
// so the 16-byte tap reads of a 16-lane group never share LDS banks across rows.
constexpr int kT16TileX0 = 2;
constexpr int kT16TileW = kChunkW + 4;
constexpr int kT16TileH = kChunkH + 4;
constexpr int kT16TileStride = 32;
constexpr int kT16TileSlots = kT16TileH * kT16TileStride;

// One latent grid at the mip levels a kernel samples.
struct GridDesc {
    const float *values;
    float *grads;
    const float *block_params;
    float *block_grads;
    int w, h, num_mips;
    int fp_w, fp_h, fp_off; // train kernel: LDS footprint box and offset (floats)
    int vb_off;             // train kernel: first texel of this grid in the LDS value box
    int cb_w, cb_h, w_row0; // train kernel: chunk cell box and its first row in the scatter matrices
    int64_t mip_off[NT_MAX_MIPS];   // texels
    int64_t block_off[NT_MAX_MIPS]; // blocks
    // Train samples at mip coordinate z > 0 (TrainDesc::trilinear): values/grads and w, h
    // above are mip m0's, these mip m1's; mip weights mw0, mw1 (train.cu:266-281).
    const float *values1;
    float *grads1;
    int w1, h1, two_mips;
    float mw0, mw1;
};

struct TexDesc {
    const float *texels; // mip 0 (with TrainDesc::trilinear: mip m0 of the target's pair)
    int w, h, pitch, nch;
    // TrainDesc::trilinear: mip m1 and the blend weight frac (0: m0 only; train.cu:78-103)
    const float *texels1;
    int w1, h1;
    float frac;
};

// Everything the fused train kernel reads.
struct TrainDesc {
    MlpDesc mlp;
    GridDesc grid[NT_MAX_GRIDS];
    TexDesc tex[NT_MAX_TEXTURES];
    int8_t out_tex[NT_MAX_OUTPUTS]; // texture feeding each output channel, -1 = none
    int8_t out_ch[NT_MAX_OUTPUTS];
    float out_w[NT_MAX_OUTPUTS]; // per-channel loss weight (train.cu:105-157)
    int G, C, ntex;
    int image_w, image_h, off_x, off_y, region_w, num_samples;
    uint32_t step;
    int tiles_x, chunks_per_wg;
    int fp_floats;  // LDS footprint floats (0: scatter straight to global)
    int fp_stride;  // floats per texel in the footprint box (odd: spreads texels over banks)
    int vbox_floats; // LDS copy of the latent values under the footprint box (C = 16; 0: gather from HBM)
    int vbox_off;    // its byte offset in LDS
    int tile_ok;    // the chunk's target taps are staged in LDS (textures match the image size)
    int random_texels; // NT_SAMPLES_RANDOM: sample positions anywhere in the image
    int trilinear;     // nt_params.sample_mip > 0: latents and targets sampled across two mips
    int scatter_mfma; // latent scatter as an MFMA reduction over the chunk (else LDS atomics)
    int w_rows;     // rows of each bilinear-weight matrix (all grids, 16-row tiles)
    int union_off;  // byte offset of the LDS region shared by tile / transposes (/ scatter)
    int scatter_split; // the scatter matrices have their own LDS region (at scatter_off)
    int scatter_off;
    const uint4 *wfrags; // weight fragments in LDS order, prepared by prep_weights
    const float *wbias;
    float *partial; // [gridDim.x][grad_total] per-workgroup MLP gradient partials
};

// The unconstrained train kernel of nt_train16.hip (16-channel grids, or the reference
// network's four 3-channel grids).
struct Grid16 {
    const float *values; // mip 0, [texel][C]
    float *grads;
    int w, h;
    int cb_w, cb_h, ncell;  // chunk cell box (cb_w x cb_h cells); 0: per-sample scatter
    // Per-sample scatter into an LDS box over the workgroup tile's footprint (box_w x box_h
    // texels of C floats at float offset box_off of the box region; box_w 0: none, straight
    // to global atomics), added to the gradients once per tile.
    int box_off, box_w, box_h;
    // A boxed grid of 1/k of the image's size (k = 1, 2): float offset (in the box region,
    // past the boxes) of its per-sample records, [group][sample][4] = {fx, fy, gradient
    // channels 0, 1 as fp16, channel 2 as fp16 | x0 << 16 | y0 << 24 relative to the box};
    // each box texel then sums its corners from the records by gather, with no atomics.
    // slot_off -1 (k 0): the box takes per-sample LDS atomics.
    int slot_off, gk;
    int wcol0;              // first column of this grid's cells in the scatter weight rows
    int gcell0;             // first cell of this grid's chunk cell box in the gather boxes
    float inv_cb_w;
    float rx, ry; // grid texels per image texel
};

// NT_SAMPLES_RANDOM: the sample indices sorted by the 64 x 64-texel bin of their texels
// (nt_sort.hip). Keys and sample indices in two buffers each (the counting sort's two passes)
// and the per-tile digit counts, all in the train workspace.
constexpr int kRandomSortMinSamples = 1 << 18; // fewer samples train in slot order
constexpr int kRandomSortTile = 4096;          // samples per workgroup in the counting passes
constexpr int kRandomSortMaxTiles = 256;       // more samples make the tiles longer
struct RandomOrderDesc {
    int n;
    uint32_t step;
    int image_w, image_h, bins_x, key_bits, bin_shift;
    int high_bits; // random_order_high_bits: key_bits (one pass), else 8 (the first pass's digit)
    int tile;      // samples per tile: kRandomSortTile, or more for over 256 tiles
    int tiles;     // ceil(n / tile), at most kRandomSortMaxTiles
    uint16_t *keys, *keys_alt;
    uint32_t *vals, *vals_alt;
    uint32_t *counts; // tiles x max(4, 1 << high_bits), then the segment starts
    uint32_t *seg;    // (1 << high_bits) + 1 segment starts (set by launch_random_order)
};
// The tiles of the counting passes for n samples.
void random_order_tiles(int n, int *tile, int *tiles);
// The first pass's digit bits: key_bits when one pass sorts the keys, else 8.
int random_order_high_bits(int key_bits, int tiles);
// Bytes of the per-tile digit counts for n samples and keys of key_bits bits.
size_t random_order_count_bytes(int n, int key_bits);
// Bins, then the stable sort; *order is the sorted sample indices (d.vals).
hipError_t launch_random_order(const RandomOrderDesc &d, hipStream_t s, const uint32_t **order);

struct Train16Desc {
    Grid16 grid[NT_MAX_GRIDS];
    const float *tex[4]; // reference textures (pitch 4, image size), output rows 4t .. 4t+3
    int tex_nch[4];
    float tex_w[4];      // loss weight of texture t's rows
    int ntex;
    int four_channels;   // some texture has four channels
    // Three textures, region positions, one group: lane group g takes texture g whole and
    // channels 2g, 2g + 1 of texture 2 (output rows 8 + 4g + r), so that both groups read
    // six channels' taps instead of one group eight and the other four.
    int split3;
    int image_w, image_h, off_x, off_y, region_w, num_samples;
    uint32_t step;
    // 1/image_w, 1/image_h, 1/num_samples where that is a power of two (a product with the
    // reciprocal then equals the quotient exactly), else 0 (divide).
    float inv_w, inv_h, inv_samples;
    int tiles_x, ntiles, nwg, xcd_per; // xcd_per > 0: workgroups of one XCD take consecutive tiles
    int group_off, group_bytes, tile_bytes; // per 4-wave group: target tile, then the union
    int wcols;                              // halves per scatter-weight row (one row per sample)
    int wclear;                             // 16-byte chunks of a row the reduction reads
    int box_lds_off, box_floats;            // LDS region of the per-sample scatter boxes (bytes, floats)
    int gather_grids;                       // grids with slot_off >= 0
    // One group with every grid in the reduction: the latent texels of each chunk's cell
    // boxes (at most 64 cells) are copied into LDS one chunk ahead (two buffers of
    // gbox_bytes from byte offset gbox_off; gbox_items float4, four per cell, grid by grid
    // from cell gcell0), and the gather reads its corners there. gbox_off 0: the gather
    // reads global memory.
    int gbox_off, gbox_bytes, gbox_items;
    // NT_SAMPLES_RANDOM: positions at uniformly random texels of the image; no target tile
    // (taps read from global memory) and per-sample gradient atomics instead of the
    // chunk-box reduction; tiles of 512 consecutive samples.
    int random_texels;
    const uint32_t *order; // random texels: the sample of each slot (NULL: slot i is sample i)
    uint64_t perm;                          // nibble r: output index of output row r
    MlpDesc mlp;                            // fp16 weights and biases, read in the prologue
    float *partial; // [nwg][grad_total]
    // NT_LATENT_TOUCHED: the update log (NULL: none) and, per grid, the mip-0 texel
    // rectangle {x0, x1, y0, y1} (inclusive, before wrapping) that holds every bilinear
    // corner of the region's positions.
    struct UpdateLog *log;
    int32_t rect[NT_MAX_GRIDS][4];
};

// NT_LATENT_TOUCHED: the update log, the last kUpdateLogBytes of the train workspace. A
// train step that knows its footprint rectangles counts itself in and, if it is the first
// since the optimizer last ran, records them; other train steps only count. The optimizer
// updates the recorded rectangles when exactly one step is logged, every texel otherwise,
// and records the count it consumed, which the next train step sees and starts over from.
// A log without the magic (a fresh workspace) is initialised by the train step and makes
// the optimizer fall back to every texel.
struct UpdateLog {
    uint64_t magic;
    uint32_t count;    // train steps logged (saturating)
    uint32_t consumed; // count the last optimizer call consumed
    uint32_t kind;     // what the rectangles count: kUpdateLogTexels or kUpdateLogBlocks
    uint32_t pad;
    int32_t rect[NT_MAX_GRIDS][4];
};
constexpr uint32_t kUpdateLogTexels = 0; // mip-0 texels of unconstrained latents
constexpr uint32_t kUpdateLogBlocks = 1; // mip-0 blocks of BC6 block records (the BC6 phase's fold)
constexpr uint64_t kUpdateLogMagic = 0x4554414450555445ull;
constexpr size_t kUpdateLogBytes = 256;
constexpr uint32_t kUpdateLogDense = 0x7fffffffu; // a step without rectangles: update every texel

// Weight-fragment preparation (once per train step) for the train kernel.
struct PrepDesc {
    MlpDesc mlp;
    uint4 *frags;
    float *bias;
};

// Gradient reduction descriptor: partial[rows][P] -> mlp gradients.
// The MLP-gradient partial rows are summed as kReduceRanges contiguous ranges of
// ceil(rows / kReduceRanges) rows, each in row order, then the range sums in range order.
// reduce_rows and the fused optimizer both follow this split, so they give the same bits.
constexpr int kReduceRanges = 16;

struct ReduceDesc {
    const float *partial;
    int rows, P;
    int num_layers;
    int off[NT_MAX_LAYERS], kin[NT_MAX_LAYERS], kout[NT_MAX_LAYERS], nbias[NT_MAX_LAYERS];
    float *wgrad[NT_MAX_LAYERS];
    float *bgrad[NT_MAX_LAYERS];
};

enum FwdMode {
    kFwdMlp = 0,
    kFwdBilinear = 1,
    kFwdCatmullRom = 2,
    kFwdInference = 3,
    kFwdDecode = 4,   // samples codec blocks directly
    kFwdDecode16 = 5  // samples the fp16 texels of the first decode pass
};

struct CodecGrid {
    const uint8_t *blocks;
    int w, h, num_mips;
    int64_t byte_off[NT_MAX_MIPS];
};

// First pass of the two-pass decode: codec blocks of every (grid, mip) level -> fp16 texels.
constexpr int kMaxExpandLevels = NT_MAX_GRIDS * NT_MAX_MIPS;
struct CodecExpandDesc {
    int levels;
    int w[kMaxExpandLevels];
    const uint8_t *blocks[kMaxExpandLevels];
    uint16_t *out[kMaxExpandLevels];
    int64_t start[kMaxExpandLevels + 1]; // prefix of work items (texels x 2)
};

// BC6 block initialisation (nt_bc6_init): every (grid, mip) level, blocks numbered over
// all levels (start = prefix of block counts).
struct Bc6InitDesc {
    int C, levels;
    const float *values[kMaxExpandLevels]; // the level's first texel
    float *blocks[kMaxExpandLevels];       // the level's first block record
    int w[kMaxExpandLevels], h[kMaxExpandLevels], nbu[kMaxExpandLevels];
    int64_t start[kMaxExpandLevels + 1];
};

// BC6 block phase (NT_BLOCK_FEATURES, NT_FINALIZE): per (grid, mip) level a step samples,
// the block records under a rectangle of blocks that holds every footprint of the step are
// expanded to fp32 texels in the workspace ([y * w + x][C], the unconstrained layout; their
// gradients cleared); an unconstrained train step (the fused kernel or the general one)
// trains on those texels; the fold then turns each block's texel gradients into its
// record's endpoint and pixel-index gradients (train.cu:373-458), which are linear in the
// texel gradient.
struct Bc6PhaseLevel {
    const float *params; // the level's block records, 4C + 18 floats each
    float *grads;        // its block-gradient records, 4C + 16 floats each
    float *values;       // expanded texels (workspace), w * h * C floats
    float *tgrads;       // their gradients (workspace)
    int w, h, nbu, nbv;  // texels; blocks per row and column
    int bx0, by0, nbx, nby; // block rectangle: origin (may lie outside the level: wraps), size
    int64_t first_block;    // first block of this level in the launch's numbering
};
struct Bc6PhaseDesc {
    Bc6PhaseLevel level[2 * NT_MAX_GRIDS];
    int nlevels, C;
    int64_t total_blocks;
    // NT_LATENT_TOUCHED with one level per grid (mip 0): the update log, in which the fold
    // records each grid's block rectangle {bx0, bx1, by0, by1} (inclusive, before wrapping);
    // NULL: none.
    struct UpdateLog *log;
    int32_t rect[NT_MAX_GRIDS][4];
};

// Second pass of the two-pass decode, LDS-staged: a workgroup decodes blocks of
// kBoxBlockW x kBoxBlockH output pixels; for every (grid, mip) the pixels of a block can
// sample it first copies a box of expanded fp16 texels into LDS, then every pixel reads
// its corners from there.
constexpr int kBoxBlockW = 64;
constexpr int kBoxBlockH = 16;
constexpr int kBoxMaxBytes = 32 * 1024;
struct BoxGrid {
    const uint16_t *texels; // expanded fp16 mip chain, [texel][16]
    int w, h, num_mips, mip_lo, mip_hi;
    int box_w[NT_MAX_MIPS], box_h[NT_MAX_MIPS], box_off[NT_MAX_MIPS]; // LDS boxes, texels
    int64_t mip_off[NT_MAX_MIPS];
};
struct DecodeBoxDesc {
    MlpDesc mlp;
    BoxGrid grid[NT_MAX_GRIDS];
    int G;
    int image_w, image_h, blocks_x, blocks_y;
    float inv_w, inv_h; // 1/image_w, 1/image_h when powers of two (exact), else 0 (divide)
    int box_texels;  // all boxes, 32 bytes each
    int lds_box_off; // byte offset of the boxes in dynamic LDS
    uint16_t *out16;
    int out_stride;
    uint32_t seed;
    float jitter, mip_min, mip_max;
};

// Forward-only passes: 256-thread workgroups (four waves) striding over 32-sample tiles,
// at most kFwdMaxBlocks of them.
constexpr int kFwdThreads = 256;
constexpr int kFwdWaves = kFwdThreads / 64;
constexpr int kFwdMaxBlocks = 2048;
inline int forward_blocks(int count)
{
    const int tiles = (count + 31) / 32, blocks = (tiles + kFwdWaves - 1) / kFwdWaves;
    return blocks < 1 ? 1 : (blocks > kFwdMaxBlocks ? kFwdMaxBlocks : blocks);
}

// Forward-only passes: nt_mlp_forward, nt_forward, nt_inference, nt_decode.
struct FwdDesc {
    MlpDesc mlp;
    GridDesc grid[NT_MAX_GRIDS];
    CodecGrid cgrid[NT_MAX_GRIDS];
    TexDesc tex[NT_MAX_TEXTURES];
    int8_t out_tex[NT_MAX_OUTPUTS];
    int8_t out_ch[NT_MAX_OUTPUTS];
    int G, C, ntex;
    int count; // samples (pixels)
    int image_w, image_h;
    float inv_w, inv_h; // 1/image_w, 1/image_h when powers of two (exact), else 0 (divide)
    const uint16_t *half_values[NT_MAX_GRIDS]; // kFwdDecode16: expanded fp16 texel chains
    const uint16_t *inputs; // kFwdMlp
    const float *uvz;       // kFwdBilinear / kFwdCatmullRom
    uint16_t *features;     // optional fp16 features
    uint16_t *out16;        // fp16 outputs
    float *out32;           // kFwdInference
    float *sse;             // kFwdInference
    float *sse_partial;     // kFwdInference: per-wave sums [blocks * kFwdWaves] (NULL: atomics)
    int out_stride;         // outputs per sample
    uint32_t seed;
    float jitter, mip_min, mip_max;
};

struct AdamDesc {
    float beta1, beta2, lr, eps, bc1, bc2;
};

// Lazy Adam over the network (train.cu:681-726).
struct NetAdamDesc {
    AdamDesc a;
    int num_layers;
    int rows[NT_MAX_LAYERS], cols[NT_MAX_LAYERS], pin[NT_MAX_LAYERS], nbias[NT_MAX_LAYERS];
    int wstart[NT_MAX_LAYERS + 1]; // prefix over layers of rows*cols + nbias, each padded to 256
    uint16_t *w[NT_MAX_LAYERS];
    float *g[NT_MAX_LAYERS], *m1[NT_MAX_LAYERS], *m2[NT_MAX_LAYERS];
    uint16_t *b[NT_MAX_LAYERS];
    float *bg[NT_MAX_LAYERS], *bm1[NT_MAX_LAYERS], *bm2[NT_MAX_LAYERS];
};

// Lazy Adam over flat fp32 segments (latent texels or BC6 block records). Segments start at
// multiples of kAdamSpan work items.
constexpr int kAdamSpan = 1024;
struct LatentAdamDesc {
    AdamDesc a;
    int nseg;
    int64_t start[NT_MAX_GRIDS + 1]; // prefix of work items, each segment padded to kAdamSpan
    float *w[NT_MAX_GRIDS], *g[NT_MAX_GRIDS], *m1[NT_MAX_GRIDS], *m2[NT_MAX_GRIDS];
    int64_t n[NT_MAX_GRIDS]; // floats (unconstrained) or blocks (block records)
    int rec;                 // block record floats (4C+16); 0 = unconstrained
    // NT_LATENT_TOUCHED: the update log, and each grid's mip-0 size (its chain starts at
    // mip 0) in texels, or in blocks for block records.
    UpdateLog *log;
    int C;
    int gw[NT_MAX_GRIDS], gh[NT_MAX_GRIDS];
};


// Sets the message nt_last_error returns (cleared for NT_OK) and returns status.
int report(int status, const char *fmt, ...);

// ---- launchers (defined next to their kernels) -------------------------------------
enum ShapeId {
    kShapeRef = 0,   // 12(16) -> 32 -> 32 -> 16, C = 3 (the reference network)
    kShapeFpt = 1,   // 12(16) -> 16 -> 16 (forward_pass_test)
    kShapeC1 = 2,    // 8(16) -> 64 -> 64 -> 16, C = 8
    kShapeC2 = 3,    // 32 -> 64 -> 64 -> 16, C = 16
    kShapeC4 = 4,    // 64 -> 64 -> 64 -> 64 -> 16, C = 16
    kShapeCount = 5
};

hipError_t launch_train(int shape, int type, const TrainDesc &d, int num_wg, size_t lds,
                        hipStream_t s);
size_t train_lds_static(int shape);
size_t train_xt_bytes(int shape);
size_t train_weight_bytes(int shape);
size_t train_frag_bytes(int shape);
hipError_t launch_prep_weights(int shape, const PrepDesc &d, hipStream_t s);
// 16-channel kernel: groups of four waves per workgroup (1 or 2) for this shape, the
// static LDS bytes (weights), the transposes' bytes, and the launchers.
int train16_groups(int shape, bool random_texels);
// The random-texel kernels (nt_train16.hip compiled with NT_TRAIN16_RANDOM_UNIT).
hipError_t launch_train16_random(int shape, const Train16Desc &d, size_t lds, hipStream_t s);
size_t train16_head_bytes(int shape);
size_t train16_transpose_bytes(int shape);
int train16_slots(int shape); // dW slots per round of the end-of-kernel group handoff
size_t train16_raw_bytes(int shape); // fp16 weight matrices staged in the prologue
hipError_t launch_train16(int shape, const Train16Desc &d, size_t lds, hipStream_t s);
int train_grad_total(int shape);
hipError_t launch_reduce(const ReduceDesc &d, hipStream_t s);
hipError_t launch_forward(int shape, int mode, const FwdDesc &d, hipStream_t s);
// Box origin (first texel) along one axis for the pixels [b0, ...) of a block: the
// footprint origin of their lowest possible sample position (jitter at its extreme).
__host__ __device__ inline int box_origin(int b0, int image, float jitter, int level)
{
    const float jmin = jitter >= 0.f ? -0.5f : 0.5f - 0x1p-24f;
    float pos = fmaf(jitter, jmin, (float)b0 + 0.5f);
    pos = pos < 0.5f ? 0.5f : (pos > (float)image - 0.5f ? (float)image - 0.5f : pos);
    return (int)floorf(fmaf(pos / (float)image, (float)level, -0.5f));
}
// The footprint origin of the highest possible sample position of pixel b1.
__host__ __device__ inline int box_last(int b1, int image, float jitter, int level)
{
    const float jmax = jitter >= 0.f ? 0.5f - 0x1p-24f : -0.5f;
    float pos = fmaf(jitter, jmax, (float)b1 + 0.5f);
    pos = pos < 0.5f ? 0.5f : (pos > (float)image - 0.5f ? (float)image - 0.5f : pos);
    return (int)floorf(fmaf(pos / (float)image, (float)level, -0.5f));
}
hipError_t launch_decode_box(int shape, const DecodeBoxDesc &d, hipStream_t s);
size_t decode_box_weight_bytes(int shape);
// *sse += the sum of partial[0..n) in a fixed order (one workgroup).
hipError_t launch_sse_reduce(const float *partial, int n, float *sse, hipStream_t s);
hipError_t launch_net_adam(const NetAdamDesc &d, hipStream_t s);
hipError_t launch_latent_adam(const LatentAdamDesc &d, hipStream_t s);

// nt_train_iteration's optimizer launch: the MLP-gradient reduction with the network update,
// and the latent update, in one grid (nred reduction workgroups first).
// The network update's fields that the combined launch needs (its gradients are the
// reduction's); the whole descriptor stays under 1 KiB of kernel arguments.
struct NetUpdateDesc {
    AdamDesc a;
    int rows[NT_MAX_LAYERS], cols[NT_MAX_LAYERS]; // active inputs x outputs per layer
    uint16_t *w[NT_MAX_LAYERS], *b[NT_MAX_LAYERS];
    float *m1[NT_MAX_LAYERS], *m2[NT_MAX_LAYERS], *bm1[NT_MAX_LAYERS], *bm2[NT_MAX_LAYERS];
};
struct OptimizeStepDesc {
    ReduceDesc red;
    NetUpdateDesc net;
    LatentAdamDesc lat;
    int nred;
    // Workgroups of the latent part: 0 sizes it for the dense scan; nt_train_iteration sizes
    // it for the rectangles its own train step logs (the loops are grid-stride, so a dense
    // fallback on that grid gives the same results).
    int lat_wg;
};
hipError_t launch_optimize_step(const OptimizeStepDesc &d, hipStream_t s);
// Logs a train step whose footprints are not recorded (the optimizer then updates every
// texel): one thread, no memset node when a caller captures the stream.
hipError_t launch_log_dense_step(UpdateLog *log, hipStream_t s);
hipError_t launch_codec_encode(const float *values, int w, int h, int C, uint8_t *blocks,
                               hipStream_t s);
hipError_t launch_codec_decode(const uint8_t *blocks, int w, int h, int C, float *values,
                               hipStream_t s);
hipError_t launch_codec_expand(const CodecExpandDesc &d, hipStream_t s);
hipError_t launch_bc6_init(const Bc6InitDesc &d, hipStream_t s);
// The expansion before and the fold after the fused kernel of the BC6 block phase.
hipError_t launch_bc6_expand(const Bc6PhaseDesc &d, hipStream_t s);
hipError_t launch_bc6_fold(const Bc6PhaseDesc &d, hipStream_t s);

} // namespace ntk
