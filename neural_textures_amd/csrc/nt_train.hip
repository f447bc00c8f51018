// nt_train.hip — the fused training pass on gfx950 (replaces TrainLoopPass,
// train.cu:818-915, with mlp.h:101-362 and util/atomic.h).
//
// One workgroup (4 waves) owns a 64 x 8 block of training-region positions and walks it
// in four 16 x 8 chunks of 128 samples. Per chunk each wave takes 32 samples (one MFMA
// tile): jittered position, latent gather into fp16 B fragments, Catmull-Rom targets for
// the lane's output rows, MLP forward (activations kept in VGPRs), fp16 loss gradient and
// the dX chain on MFMA. Layer by layer, the waves write their layer inputs and output
// gradients transposed into LDS, and after a barrier compute dW = X^T dY for the whole
// 128-sample chunk on MFMA, each wave owning a fixed subset of 32x32 dW tiles whose fp32
// accumulators stay in registers across chunks. Bias gradients are row sums of the same
// LDS tiles. Latent gradients of unconstrained latents are reduced per chunk on MFMA
// (cell weights x input gradients over the chunk's samples) into an LDS footprint box that
// covers every texel the block can touch, then flushed once with global float atomics.
// The MLP gradient of the workgroup goes to a per-workgroup partial that a deterministic
// two-stage reduction adds to the network gradients (no weight-gradient atomics). This
// kernel serves what nt_train16.hip does not: samples at a mip coordinate above 0, textures
// of other sizes or pitches, the reference network's random texels, config 1's 8-channel
// network; BC6 block latents reach it through the BC6 phase (nt_bc6.hip) as unconstrained
// steps on expanded texels.
#include "nt_train_parts.hpp"

#include <mutex>

namespace ntk {

// Per-sample bilinear footprints at mip 0 for every grid (train.cu:284-303 with z = 0).
// Sized for NT_MAX_GRIDS; with 16 channels the grid count is K0/16 and the unused entries
// fold away.
struct SampleFootprints {
    int x0[NT_MAX_GRIDS], y0[NT_MAX_GRIDS];
    float w[NT_MAX_GRIDS][4];
};

// A per-lane choice between two entries of a register array, kept a register select: the
// compiler would otherwise fold `g ? a[i] : a[j]` into a[g ? i : j], a dynamic index that
// moves the whole array to scratch memory.
template <class T>
__device__ __forceinline__ T pick(bool second, T a, T b)
{
    asm volatile("" : "+v"(a), "+v"(b));
    return second ? b : a;
}

template <int GM>
__device__ __forceinline__ void sample_footprints(const TrainDesc &d, float u, float v,
                                                  SampleFootprints &f)
{
#pragma unroll
    for (int gi = 0; gi < NT_MAX_GRIDS; ++gi) {
        if (gi < GM && gi < d.G) {
            const Footprint t = bilinear_footprint(u, v, d.grid[gi].w, d.grid[gi].h, 1.f - 0.f);
            f.x0[gi] = t.x0;
            f.y0[gi] = t.y0;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                f.w[gi][c] = t.w[c];
        } else {
            f.x0[gi] = f.y0[gi] = 0;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                f.w[gi][c] = 0.f;
        }
    }
}

// Select grid gi's footprint without dynamic register indexing.
template <int GM = NT_MAX_GRIDS>
__device__ __forceinline__ void pick_footprint(const SampleFootprints &f, int gi, int &x0,
                                               int &y0, float (&w)[4])
{
    x0 = f.x0[0];
    y0 = f.y0[0];
#pragma unroll
    for (int c = 0; c < 4; ++c)
        w[c] = f.w[0][c];
#pragma unroll
    for (int k = 1; k < GM; ++k) {
        x0 = pick(gi == k, x0, f.x0[k]);
        y0 = pick(gi == k, y0, f.y0[k]);
#pragma unroll
        for (int c = 0; c < 4; ++c)
            w[c] = pick(gi == k, w[c], f.w[k][c]);
    }
}

__device__ __forceinline__ const GridDesc &grid_ref(const TrainDesc &d, int gi)
{
    return d.grid[gi];
}

// Unconstrained latent gather into natural-layout B fragments: lane group g of a sample
// holds features 16q + 8g + e. Corner contributions are rounded to fp16 and summed in
// fp16, corner by corner (train.cu:293-310).
template <int C, int KQ>
__device__ __forceinline__ void gather_unconstrained(const TrainDesc &d, const SampleFootprints &f,
                                                     int g, h8 (&x)[KQ])
{
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
        h8 acc;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            acc[e] = (_Float16)0.f;
        if constexpr (C == 16 || C == 8) {
            const int gi = C == 16 ? q : 2 * q + g;
            const int cb = C == 16 ? 8 * g : 0;
            if (gi < d.G) {
                int x0, y0;
                float w[4];
                pick_footprint(f, gi, x0, y0, w);
                const float *vals = C == 16 ? d.grid[q].values
                                            : (g ? d.grid[(2 * q + 1) & 3].values : d.grid[2 * q].values);
                const int gw = C == 16 ? d.grid[q].w : (g ? d.grid[(2 * q + 1) & 3].w : d.grid[2 * q].w);
                const int gh = C == 16 ? d.grid[q].h : (g ? d.grid[(2 * q + 1) & 3].h : d.grid[2 * q].h);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int tx = wrap_near(x0 + (c & 1), gw);
                    const int ty = wrap_near(y0 + (c >> 1), gh);
                    const float4 *p = (const float4 *)(vals + ((int64_t)ty * gw + tx) * C + cb);
                    acc = accumulate_products(acc, w[c], load_global(p), load_global(p + 1));
                }
            }
        } else {
            // Element e is feature 16q + e in lane group 0 and 16q + 8 + e in group 1: both
            // candidates' grid and channel are compile-time, their descriptor fields uniform
            // (SGPRs), and each lane selects its own. All 32 corner loads are issued before
            // the first product.
            float val[8][4], wgt[8][4];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                constexpr int GN = NT_MAX_GRIDS;
                const int f0 = 16 * q + e, f1 = 16 * q + 8 + e;
                const int gi0 = f0 / C < GN ? f0 / C : 0, gi1 = f1 / C < GN ? f1 / C : 0;
                const bool has = g ? f1 < d.G * C : f0 < d.G * C;
                const int ch = g ? f1 % C : f0 % C;
                const float *vals = g ? sreg(d.grid[gi1].values) : sreg(d.grid[gi0].values);
                const int gw = g ? sreg(d.grid[gi1].w) : sreg(d.grid[gi0].w);
                const int gh = g ? sreg(d.grid[gi1].h) : sreg(d.grid[gi0].h);
                const int x0 = pick(g, f.x0[gi0], f.x0[gi1]), y0 = pick(g, f.y0[gi0], f.y0[gi1]);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    wgt[e][c] = pick(g, f.w[gi0][c], f.w[gi1][c]);
                    const int tx = wrap_near(x0 + (c & 1), gw);
                    const int ty = wrap_near(y0 + (c >> 1), gh);
                    val[e][c] = has ? load_global(vals + ((int64_t)ty * gw + tx) * C + ch) : 0.f;
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                _Float16 a = (_Float16)0.f;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    a = a + half_of_product(wgt[e][c], val[e][c]);
                acc[e] = a;
            }
        }
        x[q] = acc;
    }
}

// Copy the latent values under every grid's footprint box into LDS (16 channels: four
// float4 per texel, texel (lx, ly) of grid gi at vbox[(vb_off + ly * fp_w + lx) * 16]).
// Box texels map to the grid with wrap addressing, as the gathers do.
template <int GM>
__device__ __forceinline__ void load_value_box(const TrainDesc &d, float4 *vbox,
                                               const int (&flo_x)[NT_MAX_GRIDS],
                                               const int (&flo_y)[NT_MAX_GRIDS], int tid)
{
#pragma unroll
    for (int gi = 0; gi < GM; ++gi) {
        const GridDesc &gr = d.grid[gi];
        if (gi >= d.G)
            break;
        const int n4 = gr.fp_w * gr.fp_h * 4;
        float4 *dst = vbox + gr.vb_off * 4;
        for (int i = tid; i < n4; i += kTrainThreads) {
            const int texel = i >> 2, part = i & 3;
            const int lx = texel % gr.fp_w, ly = texel / gr.fp_w;
            const int gx = wrap_coord(flo_x[gi] + lx, gr.w), gy = wrap_coord(flo_y[gi] + ly, gr.h);
            dst[i] = load_global((const float4 *)(gr.values + ((int64_t)gy * gr.w + gx) * 16) + part);
        }
    }
}

// The 16-channel gather of gather_unconstrained reading the LDS value box (same products
// and fp16 accumulation order); corners outside the box (never expected: the box has a
// texel of slack on every side) read HBM.
template <int KQ>
__device__ __forceinline__ void gather_box16(const TrainDesc &d, const SampleFootprints &f,
                                             const int (&flo_x)[NT_MAX_GRIDS],
                                             const int (&flo_y)[NT_MAX_GRIDS], const float *vbox,
                                             int g, h8 (&x)[KQ])
{
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
        h8 acc;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            acc[e] = (_Float16)0.f;
        if (q < d.G) {
            const GridDesc &gr = d.grid[q];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int tx = f.x0[q] + (c & 1), ty = f.y0[q] + (c >> 1);
                const int lx = tx - flo_x[q], ly = ty - flo_y[q];
                float4 a, b;
                if (lx >= 0 && lx < gr.fp_w && ly >= 0 && ly < gr.fp_h) {
                    const float4 *p = (const float4 *)(vbox + (gr.vb_off + ly * gr.fp_w + lx) * 16 + 8 * g);
                    a = p[0];
                    b = p[1];
                } else {
                    const float4 *p = (const float4 *)(gr.values +
                                                       ((int64_t)wrap_near(ty, gr.h) * gr.w + wrap_near(tx, gr.w)) * 16 +
                                                       8 * g);
                    a = load_global(p);
                    b = load_global(p + 1);
                }
                acc = accumulate_products(acc, f.w[q][c], a, b);
            }
        }
        x[q] = acc;
    }
}

// 16-tap Catmull-Rom of one texture level (filter/catmull_rom.h:37-89 with exact taps),
// wrap addressing, fp32 fma in tap order, the first nch channels.
__device__ __forceinline__ void cr_texture(const float *texels, int w, int h, int pitch, int nch, float u,
                                           float v, float (&acc)[4])
{
    float wx[4], wy[4];
    const int x0 = cr_axis(u, w, wx);
    const int y0 = cr_axis(v, h, wy);
    for (int j = 0; j < 4; ++j) {
        const int y = wrap_coord(y0 + j, h);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int x = wrap_coord(x0 + i, w);
            const float wxy = wx[i] * wy[j];
            const int64_t base = ((int64_t)y * w + x) * pitch;
            if (pitch == 4) {
                const float4 p = *(const float4 *)(texels + base);
                acc[0] = fmaf(p.x, wxy, acc[0]);
                if (nch > 1)
                    acc[1] = fmaf(p.y, wxy, acc[1]);
                if (nch > 2)
                    acc[2] = fmaf(p.z, wxy, acc[2]);
                if (nch > 3)
                    acc[3] = fmaf(p.w, wxy, acc[3]);
            } else {
                acc[0] = fmaf(texels[base], wxy, acc[0]);
            }
        }
    }
}

// Trilinear latent gather for samples at mip coordinate z > 0 (train.cu:263-314): for every
// feature of the lane's natural-layout fragments (features 16q + 8g + e), the four corners
// of mip m0 and then of mip m1, each product rounded to fp16 and added in fp16.
template <int C, int KQ>
__device__ __forceinline__ void gather_trilinear(const TrainDesc &d, float u, float v, int g, h8 (&x)[KQ])
{
#pragma unroll
    for (int q = 0; q < KQ; ++q)
        for (int e = 0; e < 8; ++e) {
            const int feat = 16 * q + 8 * g + e;
            _Float16 a = (_Float16)0.f;
            if (feat < d.G * C) {
                const GridDesc &gr = d.grid[feat / C];
                const int ch = feat % C;
                for (int mi = 0; mi < 1 + gr.two_mips; ++mi) {
                    const int w = mi ? gr.w1 : gr.w, h = mi ? gr.h1 : gr.h;
                    const float *vals = mi ? gr.values1 : gr.values;
                    const Footprint f = bilinear_footprint(u, v, w, h, mi ? gr.mw1 : gr.mw0);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int tx = wrap_coord(f.x0 + (c & 1), w), ty = wrap_coord(f.y0 + (c >> 1), h);
                        a = a + half_of_product(f.w[c], vals[((int64_t)ty * w + tx) * C + ch]);
                    }
                }
            }
            x[q][e] = a;
        }
}

// The matching scatter (train.cu:460-509 with z > 0): global float atomics of
// weight * input gradient into both mips.
template <int C, int KQ>
__device__ __forceinline__ void scatter_trilinear(const TrainDesc &d, float u, float v, const h8 (&dx)[KQ], int g)
{
#pragma unroll
    for (int q = 0; q < KQ; ++q)
        for (int e = 0; e < 8; ++e) {
            const int feat = chained_feature(q, g, e);
            const float grad = (float)dx[q][e];
            if (feat >= d.G * C || grad == 0.f)
                continue;
            const GridDesc &gr = d.grid[feat / C];
            const int ch = feat % C;
            for (int mi = 0; mi < 1 + gr.two_mips; ++mi) {
                const int w = mi ? gr.w1 : gr.w, h = mi ? gr.h1 : gr.h;
                float *grads = mi ? gr.grads1 : gr.grads;
                const Footprint f = bilinear_footprint(u, v, w, h, mi ? gr.mw1 : gr.mw0);
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int tx = wrap_coord(f.x0 + (c & 1), w), ty = wrap_coord(f.y0 + (c >> 1), h);
                    global_add(grads + ((int64_t)ty * w + tx) * C + ch, f.w[c] * grad);
                }
            }
        }
}

// Texture, channel and loss weight of the lane's eight output rows o = chained_feature(0, g, e):
// uniform reads of both lane groups' rows, then a per-lane select (a lane-dependent index
// into the kernel arguments would be a per-lane memory load and a wait for every
// outstanding load).
__device__ __forceinline__ void lane_outputs(const TrainDesc &d, int g, int (&oti)[8], int (&och)[8],
                                             float (&wt)[8], float (&t)[8])
{
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int o0 = chained_feature(0, 0, e), o1 = chained_feature(0, 1, e);
        oti[e] = g ? sreg((int)d.out_tex[o1]) : sreg((int)d.out_tex[o0]);
        och[e] = g ? sreg((int)d.out_ch[o1]) : sreg((int)d.out_ch[o0]);
        wt[e] = g ? sreg(d.out_w[o1]) : sreg(d.out_w[o0]);
        t[e] = 0.f;
    }
}

// Catmull-Rom targets for the lane's eight output rows o = chained_feature(0, g, e)
// (train.cu:105-157; 16 taps, exact weights).
__device__ __forceinline__ void lane_targets(const TrainDesc &d, float u, float v, int g,
                                             float (&t)[8], float (&wt)[8])
{
    int oti[8], och[8];
    lane_outputs(d, g, oti, och, wt, t);
    for (int ti = 0; ti < d.ntex; ++ti) {
        bool need = false;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            need |= oti[e] == ti;
        if (!need)
            continue;
        const TexDesc tx = d.tex[ti];
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        cr_texture(tx.texels, tx.w, tx.h, tx.pitch, tx.nch, u, v, acc);
        if (d.trilinear && tx.frac > 0.f) {
            // SampleReferenceTextureTrilinear (train.cu:78-103): blend with mip m1
            float acc1[4] = {0.f, 0.f, 0.f, 0.f};
            cr_texture(tx.texels1, tx.w1, tx.h1, tx.pitch, tx.nch, u, v, acc1);
#pragma unroll
            for (int k = 0; k < 4; ++k)
                acc[k] = fmaf(acc1[k], tx.frac, acc[k] * (1.f - tx.frac));
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (oti[e] == ti) {
                const int c = och[e];
                t[e] = c == 0 ? acc[0] : c == 1 ? acc[1] : c == 2 ? acc[2] : acc[3];
            }
        }
    }
}

// Stage the chunk's Catmull-Rom footprint of every reference texture in LDS: texels
// [cx0 - kTileX0, cx0 - kTileX0 + kTileW) x [cy0 - kTileX0, ... + kTileH), float4 each,
// wrapped like the reference's texture objects (main.cpp:613-621).
// Every texture has the image size here (the tile is used only then), so one wrapped texel
// index serves all of them; the texture loop is uniform (descriptors in SGPRs) and issues
// the loads of four textures before the first LDS store.
__device__ __forceinline__ void load_target_tile(const TrainDesc &d, float4 *tile, int cx0, int cy0,
                                                 int tid)
{
    constexpr int per = kTileW * kTileH;
    constexpr int R = (per + kTrainThreads - 1) / kTrainThreads;
    int64_t texel[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
        const int i = min(tid + r * kTrainThreads, per - 1);
        int gx = cx0 - kTileX0 + i % kTileW, gy = cy0 - kTileX0 + i / kTileW;
        gx = (unsigned)gx < (unsigned)d.image_w ? gx : wrap_coord(gx, d.image_w);
        gy = (unsigned)gy < (unsigned)d.image_h ? gy : wrap_coord(gy, d.image_h);
        texel[r] = (int64_t)gy * d.image_w + gx;
    }
    for (int t0 = 0; t0 < d.ntex; t0 += 4) {
        float4 v[4][R];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const int t = t0 + k;
            const TexDesc &tex = d.tex[min(t, NT_MAX_TEXTURES - 1)];
            const float *texels = t < d.ntex ? tex.texels : nullptr;
            const int pitch = tex.pitch;
#pragma unroll
            for (int r = 0; r < R; ++r) {
                v[k][r] = make_float4(0.f, 0.f, 0.f, 0.f);
                if (texels) {
                    if (pitch == 4)
                        v[k][r] = load_global((const float4 *)(texels + texel[r] * 4));
                    else
                        v[k][r].x = load_global(texels + texel[r]);
                }
            }
        }
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int r = 0; r < R; ++r)
                if (t0 + k < d.ntex && tid + r * kTrainThreads < per)
                    tile[(t0 + k) * per + tid + r * kTrainThreads] = v[k][r];
    }
}

// Catmull-Rom targets for the lane's eight output rows from the staged tile: the same taps,
// weights and fp32 fma order as lane_targets (train.cu:105-157).
__device__ __forceinline__ void lane_targets_tile(const TrainDesc &d, const float4 *tile, int cx0,
                                                  int cy0, float u, float v, int g, float (&t)[8],
                                                  float (&wt)[8])
{
    int oti[8], och[8];
    lane_outputs(d, g, oti, och, wt, t);
    float wx[4], wy[4];
    const int x0 = cr_axis(u, d.image_w, wx) - (cx0 - kTileX0);
    const int y0 = cr_axis(v, d.image_h, wy) - (cy0 - kTileX0);
    const bool inside = x0 >= 0 && x0 + 3 < kTileW && y0 >= 0 && y0 + 3 < kTileH;
    for (int ti = 0; ti < d.ntex; ++ti) {
        bool need = false;
#pragma unroll
        for (int e = 0; e < 8; ++e)
            need |= oti[e] == ti;
        if (!need)
            continue;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        if (inside) {
            const float4 *base = tile + ti * (kTileW * kTileH) + y0 * kTileW + x0;
#pragma unroll
            for (int j = 0; j < 4; ++j)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 p = base[j * kTileW + i];
                    const float wxy = wx[i] * wy[j];
                    acc[0] = fmaf(p.x, wxy, acc[0]);
                    acc[1] = fmaf(p.y, wxy, acc[1]);
                    acc[2] = fmaf(p.z, wxy, acc[2]);
                    acc[3] = fmaf(p.w, wxy, acc[3]);
                }
        } else {
            const TexDesc tx = d.tex[ti];
            const int gx0 = x0 + (cx0 - kTileX0), gy0 = y0 + (cy0 - kTileX0);
            for (int j = 0; j < 4; ++j) {
                const int y = wrap_coord(gy0 + j, tx.h);
                for (int i = 0; i < 4; ++i) {
                    const int x = wrap_coord(gx0 + i, tx.w);
                    const float wxy = wx[i] * wy[j];
                    const int64_t b = ((int64_t)y * tx.w + x) * tx.pitch;
                    if (tx.pitch == 4) {
                        const float4 p = *(const float4 *)(tx.texels + b);
                        acc[0] = fmaf(p.x, wxy, acc[0]);
                        acc[1] = fmaf(p.y, wxy, acc[1]);
                        acc[2] = fmaf(p.z, wxy, acc[2]);
                        acc[3] = fmaf(p.w, wxy, acc[3]);
                    } else {
                        acc[0] = fmaf(tx.texels[b], wxy, acc[0]);
                    }
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            if (oti[e] == ti) {
                const int c = och[e];
                t[e] = c == 0 ? acc[0] : c == 1 ? acc[1] : c == 2 ? acc[2] : acc[3];
            }
        }
    }
}

// Latent gradient scatter of one sample (train.cu:460-509): LDS footprint box when the
// texel is inside it, global float atomics otherwise.
template <int C, int KQ>
__device__ __forceinline__ void scatter_unconstrained(const TrainDesc &d, const SampleFootprints &f,
                                                      const int (&flo_x)[NT_MAX_GRIDS],
                                                      const int (&flo_y)[NT_MAX_GRIDS], float *fp,
                                                      const h8 (&dx)[KQ], int g)
{
#pragma unroll
    for (int q = 0; q < KQ; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int feat = chained_feature(q, g, e);
            const float grad = (float)dx[q][e];
            if (feat >= d.G * C || grad == 0.f)
                continue;
            const int gi = feat / C, ch = feat % C;
            int x0, y0;
            float w[4];
            pick_footprint(f, gi, x0, y0, w);
            const GridDesc &gr = grid_ref(d, gi);
            int lox = flo_x[0], loy = flo_y[0];
#pragma unroll
            for (int k = 1; k < NT_MAX_GRIDS; ++k) {
                lox = pick(gi == k, lox, flo_x[k]);
                loy = pick(gi == k, loy, flo_y[k]);
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const float val = w[c] * grad;
                const int tx = x0 + (c & 1), ty = y0 + (c >> 1);
                const int lx = tx - lox, ly = ty - loy;
                if (d.fp_floats > 0 && lx >= 0 && lx < gr.fp_w && ly >= 0 && ly < gr.fp_h) {
                    lds_add(fp + gr.fp_off + (ly * gr.fp_w + lx) * d.fp_stride + ch, val);
                } else {
                    const int wx = wrap_near(tx, gr.w), wy = wrap_near(ty, gr.h);
                    global_add(gr.grads + ((int64_t)wy * gr.w + wx) * C + ch, val);
                }
            }
        }
}

// Latent gradient scatter without a footprint box, 16 channels (train.cu:460-509, the
// same adds): the wave stages its 32 samples' dX0 rows and bilinear corners (texel index,
// weight) in its own LDS slice, then walks the samples with lane = 16 * corner + channel,
// so one atomic instruction adds whole 64-byte texel records instead of 64 scattered
// floats. Called with all lanes of the wave; invalid samples have no corners.
template <int KQ, int GM>
struct Rows16 {
    static constexpr int K0 = KQ * 16;
    static constexpr int dx_bytes = 32 * K0 * 2;
    static constexpr int bytes = dx_bytes + 32 * GM * 4 * 8; // + texel index, weight per corner
};

template <int KQ, int GM>
__device__ __forceinline__ void scatter_rows16(const TrainDesc &d, const SampleFootprints &f, const h8 (&dx)[KQ],
                                               bool valid, int lane, unsigned char *slice)
{
    using R = Rows16<KQ, GM>;
    const int c = lane & 31, g = lane >> 5;
    _Float16 *dxr = (_Float16 *)slice;
    int *cidx = (int *)(slice + R::dx_bytes);
    float *cw = (float *)(cidx + 32 * GM * 4);
    // Chained fragment q of lane group g holds features 16q + 4g + (0..3) and 16q + 8 + 4g + (0..3).
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
        *(h4 *)(dxr + c * R::K0 + 16 * q + 4 * g) = __builtin_shufflevector(dx[q], dx[q], 0, 1, 2, 3);
        *(h4 *)(dxr + c * R::K0 + 16 * q + 8 + 4 * g) = __builtin_shufflevector(dx[q], dx[q], 4, 5, 6, 7);
    }
    // Lane group g records corners 2g and 2g + 1 of every grid.
#pragma unroll
    for (int gi = 0; gi < GM; ++gi) {
        const GridDesc &gr = d.grid[gi];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int k = 2 * g + kk;
            const int tx = f.x0[gi] + kk, ty = f.y0[gi] + g;
            const int slot = (c * GM + gi) * 4 + k;
            cidx[slot] = valid ? wrap_near(ty, gr.h) * gr.w + wrap_near(tx, gr.w) : -1;
            cw[slot] = g ? f.w[gi][2 + kk] : f.w[gi][kk];
        }
    }
    const int k = lane >> 4, ch = lane & 15;
#pragma unroll 4
    for (int s = 0; s < 32; ++s) {
#pragma unroll
        for (int gi = 0; gi < GM; ++gi) {
            const int slot = (s * GM + gi) * 4 + k;
            const int idx = cidx[slot];
            const float gv = (float)dxr[s * R::K0 + 16 * gi + ch];
            if (idx >= 0 && gv != 0.f)
                global_add(d.grid[gi].grads + (int64_t)idx * 16 + ch, cw[slot] * gv);
        }
    }
}

// Latent gradient scatter of one 128-sample chunk as an MFMA reduction over the samples
// (train.cu:460-509 without atomics): per grid, the chunk's cell-box gradient is
//   D[cell][ch] = sum_s W[cell][s] * dX0[s][ch]
// (C = 16 fills the 16 columns of a 16 x 16 D tile; C = 3 uses three of them: same-address
// LDS atomics, which the per-sample scatter of 3-channel latents would take, serialise),
// W holding each sample's four bilinear corner weights (fp32 split into fp16 hi + lo, so
// the products equal the reference's fp32 weight * fp16 gradient to ~2^-22). D is added
// into the workgroup footprint box by the one lane that owns each (cell, channel). Corners
// outside the chunk box (fp32 rounding at the box edge) go to the box with LDS atomics.
// LDS: dxt [K0][kRowStride] fp16 | W hi [w_rows][kRowStride] | W lo [w_rows][kRowStride].

// Chunk cell-box origin of every grid.
template <int GM>
__device__ __forceinline__ void chunk_box(const TrainDesc &d, int cx0, int cy0, int (&bx)[NT_MAX_GRIDS],
                                          int (&by)[NT_MAX_GRIDS])
{
#pragma unroll
    for (int gi = 0; gi < NT_MAX_GRIDS; ++gi) {
        const GridDesc &gr = d.grid[gi];
        bx[gi] = gi < GM ? (int)floorf((float)cx0 * (float)gr.w / (float)d.image_w - 0.5f) : 0;
        by[gi] = gi < GM ? (int)floorf((float)cy0 * (float)gr.h / (float)d.image_h - 0.5f) : 0;
    }
}

__device__ __forceinline__ void zero_scatter_weights(const TrainDesc &d, _Float16 *sct, int tid, int k0)
{
    uint4 *z = (uint4 *)(sct + k0 * kRowStride);
    const int n = 2 * d.w_rows * kRowStride / 8;
    for (int i = tid; i < n; i += kTrainThreads)
        z[i] = make_uint4(0u, 0u, 0u, 0u);
}

// Part 1 (before a barrier): this lane's input gradient into dxt and its two corner weights
// per grid into W (lane group g writes corners 2g, 2g+1); out-of-box corners by atomics.
template <class S, int C, int GM>
__device__ __forceinline__ void scatter_write(const TrainDesc &d, const SampleFootprints &f,
                                              const h8 (&dx)[S::K0 / 16], bool valid,
                                              const int (&cbx)[NT_MAX_GRIDS], const int (&cby)[NT_MAX_GRIDS],
                                              const int (&flo_x)[NT_MAX_GRIDS],
                                              const int (&flo_y)[NT_MAX_GRIDS], float *fp,
                                              _Float16 *sct, int col, int g)
{
    static_assert(C <= 16, "grid g's channels are rows [C g, C g + C) of the dX0 transpose");
    constexpr int KQ0 = S::K0 / 16;
    _Float16 *dxt = sct;
    _Float16 *whi = dxt + S::K0 * kRowStride;
    _Float16 *wlo = whi + d.w_rows * kRowStride;
    store_transposed<KQ0, true>(dxt, dx, col, g);
    if (!valid)
        return;
#pragma unroll
    for (int gi = 0; gi < GM; ++gi) {
        if (GM > 1 && gi >= d.G)
            continue;
        const GridDesc &gr = d.grid[gi];
#pragma unroll
        for (int corner = 0; corner < 4; ++corner) {
            const int tx = f.x0[gi] + (corner & 1), ty = f.y0[gi] + (corner >> 1);
            const int cx = tx - cbx[gi], cy = ty - cby[gi];
            const float w = f.w[gi][corner];
            if (cx >= 0 && cx < gr.cb_w && cy >= 0 && cy < gr.cb_h) {
                if ((corner >> 1) == g) {
                    const int row = gr.w_row0 + cy * gr.cb_w + cx;
                    const _Float16 hi = (_Float16)w;
                    whi[row * kRowStride + col] = hi;
                    wlo[row * kRowStride + col] = (_Float16)(w - (float)hi);
                }
            } else {
                const int lx = tx - flo_x[gi], ly = ty - flo_y[gi];
                const bool inbox = lx >= 0 && lx < gr.fp_w && ly >= 0 && ly < gr.fp_h;
                // This lane group's features of grid gi (for C = 16, all of fragment gi).
#pragma unroll
                for (int q = 0; q < KQ0; ++q)
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const int feat = chained_feature(q, g, e);
                        if (feat / C != gi)
                            continue;
                        const int ch = feat % C;
                        const float val = w * (float)dx[q][e];
                        if (inbox)
                            lds_add(fp + gr.fp_off + (ly * gr.fp_w + lx) * d.fp_stride + ch, val);
                        else
                            global_add(gr.grads + ((int64_t)wrap_near(ty, gr.h) * gr.w + wrap_near(tx, gr.w)) * C +
                                           ch,
                                       val);
                    }
            }
        }
    }
}

// Part 2 (after the barrier): one task per (grid, 16-row tile of its cells), dealt to the
// waves starting at wave `first`.
template <class S, int C, int GM>
__device__ __forceinline__ void scatter_reduce(const TrainDesc &d, const int (&cbx)[NT_MAX_GRIDS],
                                               const int (&cby)[NT_MAX_GRIDS],
                                               const int (&flo_x)[NT_MAX_GRIDS],
                                               const int (&flo_y)[NT_MAX_GRIDS], float *fp,
                                               const _Float16 *sct, int first, int wave, int lane)
{
    const _Float16 *dxt = sct;
    const _Float16 *whi = dxt + S::K0 * kRowStride;
    const _Float16 *wlo = whi + d.w_rows * kRowStride;
    int task = first;
#pragma unroll
    for (int gi = 0; gi < GM; ++gi) {
        if (GM > 1 && gi >= d.G)
            continue;
        const GridDesc &gr = d.grid[gi];
        const int ncell = gr.cb_w * gr.cb_h;
        const int ntile = (ncell + 15) >> 4;
        for (int t = 0; t < ntile; ++t, ++task) {
            if ((task & 3) != wave)
                continue;
            f4v acc = {0.f, 0.f, 0.f, 0.f};
            const int arow = (gr.w_row0 + 16 * t + (lane & 15)) * kRowStride + 8 * (lane >> 4);
            // Columns past C repeat channel C - 1 (their D entries are not used).
            const _Float16 *bp = dxt + (gi * C + min(lane & 15, C - 1)) * kRowStride + 8 * (lane >> 4);
#pragma unroll
            for (int k = 0; k < kChunk / 32; ++k) {
                const h8 bv = *(const h8 *)(bp + 32 * k);
                acc = mfma16(*(const h8 *)(whi + arow + 32 * k), bv, acc);
                acc = mfma16(*(const h8 *)(wlo + arow + 32 * k), bv, acc);
            }
            const int ch = lane & 15;
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int cell = 16 * t + 4 * (lane >> 4) + r;
                if (cell >= ncell || ch >= C || acc[r] == 0.f)
                    continue;
                const int tx = cbx[gi] + cell % gr.cb_w, ty = cby[gi] + cell / gr.cb_w;
                const int lx = tx - flo_x[gi], ly = ty - flo_y[gi];
                if (lx >= 0 && lx < gr.fp_w && ly >= 0 && ly < gr.fp_h)
                    fp[gr.fp_off + (ly * gr.fp_w + lx) * d.fp_stride + ch] += acc[r];
                else
                    global_add(gr.grads + ((int64_t)wrap_near(ty, gr.h) * gr.w + wrap_near(tx, gr.w)) * C + ch,
                               acc[r]);
            }
        }
    }
}

template <class S, int C>
__global__ __launch_bounds__(kTrainThreads) void train_kernel(TrainDesc d)
{
    using LY = TrainLayout<S>;
    constexpr int L = S::L, NH = S::NH, KQ0 = S::K0 / 16, HQ = S::H / 16, HA = S::t32(S::H);
    constexpr int GM = C == 16 ? S::K0 / 16 : NT_MAX_GRIDS; // grids, as far as known statically
    extern __shared__ __align__(16) unsigned char smem[];
    h8 *frags = (h8 *)smem;
    float *bias = (float *)(smem + LY::frag_bytes);
    float *fp = (float *)(smem + LY::head_bytes);
    unsigned char *un = smem + d.union_off;
    _Float16 *xt = (_Float16 *)un;
    _Float16 *dyt = xt + LY::xt_rows * kRowStride;
    float4 *tile = (float4 *)un; // aliases the transposes: dead before they are written
    // Scatter matrices: their own region when it fits (scatter_split), else the union.
    _Float16 *sct = (_Float16 *)(smem + (d.scatter_split ? d.scatter_off : d.union_off));

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 31, g = lane >> 5;
    {
        uint4 *dst = (uint4 *)frags;
        for (int i = tid; i < S::all_frags() * kWave; i += kTrainThreads)
            dst[i] = d.wfrags[i];
        for (int i = tid; i < S::bias_total(); i += kTrainThreads)
            bias[i] = d.wbias[i];
    }
    for (int i = tid; i < d.fp_floats; i += kTrainThreads)
        fp[i] = 0.f;
    float *vbox = (float *)(smem + d.vbox_off);

    const int tile_x = blockIdx.x % d.tiles_x, tile_y = blockIdx.x / d.tiles_x;
    const int tx0 = tile_x * kChunkW * d.chunks_per_wg, ty0 = tile_y * kChunkH;
    // Footprint box origin per grid: lowest texel any sample of this block can touch.
    int flo_x[NT_MAX_GRIDS], flo_y[NT_MAX_GRIDS];
#pragma unroll
    for (int gi = 0; gi < NT_MAX_GRIDS; ++gi) {
        const GridDesc &gr = d.grid[gi];
        flo_x[gi] = gi < GM ? (int)floorf((float)(d.off_x + tx0) * (float)gr.w / (float)d.image_w - 0.5f) - 1 : 0;
        flo_y[gi] = gi < GM ? (int)floorf((float)(d.off_y + ty0) * (float)gr.h / (float)d.image_h - 0.5f) - 1 : 0;
    }
    if constexpr (C == 16) {
        if (d.vbox_floats > 0)
            load_value_box<GM>(d, (float4 *)vbox, flo_x, flo_y, tid);
    }

    f16v dwacc[LY::slots];
#pragma unroll
    for (int j = 0; j < LY::slots; ++j)
#pragma unroll
        for (int e = 0; e < 16; ++e)
            dwacc[j][e] = 0.f;
    float dbacc[L];
#pragma unroll
    for (int l = 0; l < L; ++l)
        dbacc[l] = 0.f;

    const bool mfma_scatter = d.scatter_mfma;
    const int col = 32 * wave + c; // column of this lane's sample in the LDS transposes
    for (int chunk = 0; chunk < d.chunks_per_wg; ++chunk) {
        const int cx0 = d.off_x + tx0 + chunk * kChunkW, cy0 = d.off_y + ty0;
        if (mfma_scatter && d.scatter_split)
            zero_scatter_weights(d, sct, tid, S::K0); // last read before the previous chunk's final barrier
        if (d.tile_ok)
            load_target_tile(d, tile, cx0, cy0, tid);
        __syncthreads(); // weights staged / footprint box zeroed / tile loaded

        // ---- sample position (train.cu:827-844)
        const int sx = tx0 + chunk * kChunkW + (c & 15);
        const int sy = ty0 + 2 * wave + (c >> 4);
        const uint32_t sidx = (uint32_t)sy * (uint32_t)d.region_w + (uint32_t)sx;
        const bool valid = sx < d.region_w && sidx < (uint32_t)d.num_samples;
        uint32_t st = mix_seed(sidx, d.step);
        uint32_t tx = (uint32_t)(d.off_x + sx), ty = (uint32_t)(d.off_y + sy);
        if (d.random_texels) // a uniformly random texel of the image, then the jitter
            random_texel(st, d.image_w, d.image_h, tx, ty);
        const float jx = uniform01(st) - 0.5f;
        const float jy = uniform01(st) - 0.5f;
        const float px = clampf((float)tx + 0.5f + jx, 0.5f, (float)d.image_w - 0.5f);
        const float py = clampf((float)ty + 0.5f + jy, 0.5f, (float)d.image_h - 0.5f);
        const float u = px / (float)d.image_w;
        const float v = py / (float)d.image_h;

        h8 x0[KQ0];
        {
            SampleFootprints fps;
            sample_footprints<GM>(d, u, v, fps);
            if (valid) {
                if (d.trilinear)
                    gather_trilinear<C, KQ0>(d, u, v, g, x0);
                else if (C == 16 && d.vbox_floats > 0)
                    gather_box16<KQ0>(d, fps, flo_x, flo_y, vbox, g, x0);
                else
                    gather_unconstrained<C, KQ0>(d, fps, g, x0);
            } else {
#pragma unroll
                for (int q = 0; q < KQ0; ++q)
                    x0[q] = (h8)(_Float16)0.f;
            }
        }

        // ---- forward (mlp.h:65-99)
        h8 xh[NH][HQ];
        {
            f16v acc[HA];
            layer_forward<KQ0, HA>(frags + S::fwd_off(0) * kWave, bias + S::bias_off(0), x0, acc, lane);
            to_fragments<HQ, HA, true>(acc, xh[0]);
#pragma unroll
            for (int l = 1; l < NH; ++l) {
                layer_forward<HQ, HA>(frags + S::fwd_off(l) * kWave, bias + S::bias_off(l), xh[l - 1],
                                      acc, lane);
                to_fragments<HQ, HA, true>(acc, xh[l]);
            }
        }
        // ---- targets and loss gradient (train.cu:105-157, 876-888): dL/dy = fp16(2 w (y - t) / N)
        h8 dyo[1];
        {
            f16v out[1];
            layer_forward<HQ, 1>(frags + S::fwd_off(L - 1) * kWave, bias + S::bias_off(L - 1),
                                 xh[NH - 1], out, lane);
            float tgt[8], tw[8];
            if (d.tile_ok)
                lane_targets_tile(d, tile, cx0, cy0, u, v, g, tgt, tw);
            else
                lane_targets(d, u, v, g, tgt, tw);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float y = (float)(_Float16)out[0][e];
                const float err = y - tgt[e];
                const float gr = 2.f * tw[e] * err / (float)d.num_samples;
                dyo[0][e] = valid ? (_Float16)gr : (_Float16)0.f;
            }
        }
        if (d.tile_ok)
            __syncthreads(); // the transposes below overwrite the tile

        // ---- backward, last layer (mlp.h:302-362)
        h8 dyh[HQ];
        store_transposed<1, true>(dyt, dyo, col, g);
        store_transposed<HQ, true>(xt, xh[NH - 1], col, g);
        {
            f16v acc[HA];
            layer_backward_dx<1, HA>(frags + S::bwd_off(L - 1) * kWave, dyo, acc, lane);
            relu_backward<HQ, HA>(acc, xh[NH - 1], dyh);
        }
        __syncthreads();
        dw_phase<S, L - 1>(xt, dyt, dwacc, dbacc[L - 1], wave, lane, tid);
        __syncthreads();

        // ---- hidden layers L-2 .. 1
        backward_hidden<S, L - 2>(xt, dyt, frags, xh, dyh, dwacc, dbacc, col, wave, lane, tid);

        // ---- first layer: dW with the natural-layout inputs, dX = input gradient
        store_transposed<HQ, true>(dyt, dyh, col, g);
        store_transposed<KQ0, false>(xt, x0, col, g);
        h8 dx0[KQ0];
        {
            constexpr int MA = S::t32(S::K0);
            f16v acc[MA];
            layer_backward_dx<HQ, MA>(frags + S::bwd_off(0) * kWave, dyh, acc, lane);
#pragma unroll
            for (int q = 0; q < KQ0; ++q)
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    dx0[q][e] = (_Float16)acc[q >> 1][8 * (q & 1) + e];
        }
        // Footprints again (cheaper than keeping them live through the MLP).
        SampleFootprints fps;
        sample_footprints<GM>(d, rn32(u), rn32(v), fps);
        int cbx[NT_MAX_GRIDS], cby[NT_MAX_GRIDS];
        chunk_box<GM>(d, cx0, cy0, cbx, cby);
        if (mfma_scatter && d.scatter_split)
            scatter_write<S, C, GM>(d, fps, dx0, valid, cbx, cby, flo_x, flo_y, fp, sct, col, g);
        __syncthreads();
        dw_phase<S, 0>(xt, dyt, dwacc, dbacc[0], wave, lane, tid);
        if (mfma_scatter && d.scatter_split)
            scatter_reduce<S, C, GM>(d, cbx, cby, flo_x, flo_y, fp, sct, S::dw_total(), wave, lane);
        __syncthreads();

        // ---- latent gradient scatter when it cannot share the layer-0 phase
        {
            if (d.trilinear) {
                if (valid)
                    scatter_trilinear<C, KQ0>(d, rn32(u), rn32(v), dx0, g);
            } else if (mfma_scatter) {
                if (!d.scatter_split) {
                    zero_scatter_weights(d, sct, tid, S::K0);
                    __syncthreads();
                    scatter_write<S, C, GM>(d, fps, dx0, valid, cbx, cby, flo_x, flo_y, fp, sct, col, g);
                    __syncthreads();
                    scatter_reduce<S, C, GM>(d, cbx, cby, flo_x, flo_y, fp, sct, 0, wave, lane);
                    __syncthreads();
                }
            } else if constexpr (C == 16) {
                if (d.fp_floats == 0) {
                    static_assert(4 * Rows16<KQ0, GM>::bytes <= LY::transpose_bytes, "row slices fit the union");
                    scatter_rows16<KQ0, GM>(d, fps, dx0, valid, lane, un + wave * Rows16<KQ0, GM>::bytes);
                    if (d.tile_ok)
                        __syncthreads(); // the next chunk's target tile reuses the union
                } else if (valid) {
                    scatter_unconstrained<C, KQ0>(d, fps, flo_x, flo_y, fp, dx0, g);
                }
            } else if (valid) {
                scatter_unconstrained<C, KQ0>(d, fps, flo_x, flo_y, fp, dx0, g);
            }
        }
    }

    __syncthreads();
    // ---- flush the latent footprint box
    {
        // Grid by grid (uniform descriptors), each grid's box spread over the threads.
#pragma unroll
        for (int gi = 0; gi < GM; ++gi) {
            if (GM > 1 && gi >= d.G)
                continue;
            const GridDesc &gr = d.grid[gi];
            const int n = d.fp_floats > 0 ? gr.fp_w * gr.fp_h * d.fp_stride : 0;
            for (int i = tid; i < n; i += kTrainThreads) {
                const float val = fp[gr.fp_off + i];
                const int ch = i % d.fp_stride, cell = i / d.fp_stride;
                if (val == 0.f || ch >= C)
                    continue;
                const int lx = cell % gr.fp_w, ly = cell / gr.fp_w;
                const int wx = wrap_coord(flo_x[gi] + lx, gr.w), wy = wrap_coord(flo_y[gi] + ly, gr.h);
                global_add(gr.grads + ((int64_t)wy * gr.w + wx) * C + ch, val);
            }
        }
    }
    // ---- per-workgroup MLP gradient partial
    float *part = d.partial + (int64_t)blockIdx.x * S::grad_total();
#pragma unroll
    for (int j = 0; j < LY::slots; ++j) {
        const int t = 4 * j + wave;
        if (t < S::dw_total()) {
            int l = 0;
#pragma unroll
            for (int k = 0; k < L; ++k)
                if (t >= S::dw_start(k) && t < S::dw_start(k) + S::dw_tiles(k))
                    l = k;
            int kin = S::kin(0), kout = S::kout(0), start = S::dw_start(0), off = S::grad_off(0);
#pragma unroll
            for (int k = 1; k < L; ++k)
                if (l == k) {
                    kin = S::kin(k);
                    kout = S::kout(k);
                    start = S::dw_start(k);
                    off = S::grad_off(k);
                }
            const int kb = (kin + 31) / 32;
            const int a = (t - start) / kb, b = (t - start) % kb;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int n = 32 * a + 8 * (e >> 2) + 4 * g + (e & 3);
                const int k = 32 * b + c;
                if (n < kout && k < kin)
                    part[off + n * kin + k] = dwacc[j][e];
            }
        }
    }
#pragma unroll
    for (int l = 0; l < L; ++l)
        if (tid < 4 * S::kout(l) && (tid & 3) == 0)
            part[S::grad_off(l) + S::kout(l) * S::kin(l) + (tid >> 2)] = dbacc[l];
}

// Two-stage deterministic reduction of the per-workgroup partials into the network
// gradients (which the contract says are accumulated into, train.cu:1028-1048).
// partial[rows][P] -> the MLP gradients, in one pass and a fixed order: a workgroup owns 64
// parameters and splits the rows into 16 contiguous groups, one per wave; each lane sums its
// group's rows of one parameter in row order (all loads issued before the adds: every wave
// load is 256 contiguous bytes of one row), then wave 0 adds the 16 group sums in group
// order. The same bits on every run.
constexpr int kReduceCols = 64, kReduceGroups = kReduceRanges, kReduceUnroll = 16;
__global__ __launch_bounds__(kReduceCols *kReduceGroups) void reduce_rows(ReduceDesc d)
{
    __shared__ float part[kReduceGroups][kReduceCols];
    const int col = threadIdx.x % kReduceCols, grp = threadIdx.x / kReduceCols;
    const int p = blockIdx.x * kReduceCols + col;
    const int per = (d.rows + kReduceGroups - 1) / kReduceGroups;
    const int r0 = grp * per, r1 = min(r0 + per, d.rows);
    float sum = 0.f;
    if (p < d.P) {
        const float *c = d.partial + p;
        for (int r = r0; r < r1; r += kReduceUnroll) {
            float v[kReduceUnroll];
#pragma unroll
            for (int k = 0; k < kReduceUnroll; ++k)
                v[k] = r + k < r1 ? c[(int64_t)(r + k) * d.P] : 0.f;
#pragma unroll
            for (int k = 0; k < kReduceUnroll; ++k)
                sum += v[k];
        }
    }
    part[grp][col] = sum;
    __syncthreads();
    if (grp != 0 || p >= d.P)
        return;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kReduceGroups; ++k)
        s += part[k][col];
    int l = 0;
    for (int k = 1; k < d.num_layers; ++k)
        if (p >= d.off[k])
            l = k;
    const int local = p - d.off[l];
    const int nw = d.kin[l] * d.kout[l];
    if (local < nw)
        d.wgrad[l][local] += s;
    else if (local - nw < d.nbias[l])
        d.bgrad[l][local - nw] += s;
}

// Weight fragments and fp32 biases in the train kernel's LDS order, computed once per step
// so that every workgroup stages them with plain 16-byte copies.
template <class S>
__global__ __launch_bounds__(256) void prep_weights_kernel(PrepDesc d)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < S::all_frags() * kWave) {
        const h8 v = weight_fragment<S>(d.mlp, i);
        d.frags[i] = __builtin_bit_cast(uint4, v);
    }
    if (i < S::bias_total())
        d.bias[i] = bias_value<S>(d.mlp, i);
}

template <class S>
static hipError_t launch_prep(const PrepDesc &d, hipStream_t s)
{
    const int n = S::all_frags() * kWave > S::bias_total() ? S::all_frags() * kWave : S::bias_total();
    hipLaunchKernelGGL(prep_weights_kernel<S>, dim3((n + 255) / 256), dim3(256), 0, s, d);
    return hipGetLastError();
}

hipError_t launch_reduce(const ReduceDesc &d, hipStream_t s)
{
    hipLaunchKernelGGL(reduce_rows, dim3((d.P + kReduceCols - 1) / kReduceCols), dim3(kReduceCols * kReduceGroups), 0,
                       s, d);
    return hipGetLastError();
}

// The general kernel trains unconstrained latents; block records train through the BC6
// phase (expanded texels, then the fold), which calls it as an unconstrained step.
template <class S, int C>
static hipError_t launch_one(const TrainDesc &d, int num_wg, size_t lds, hipStream_t s)
{
    auto k = train_kernel<S, C>;
    // Raise the kernel's dynamic LDS limit to the whole 160 KB once (thread-safe).
    static std::once_flag once;
    static hipError_t configured = hipSuccess;
    std::call_once(once, [&] {
        configured = hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    if (lds > 65536 && configured != hipSuccess)
        return configured;
    hipLaunchKernelGGL(k, dim3(num_wg), dim3(kTrainThreads), lds, s, d);
    return hipGetLastError();
}

using ShapeRef = Shape<16, 32, 2>;
using ShapeC1 = Shape<16, 64, 2>; // BASELINE config 1's network: one grid of 8 channels, 8 -> 64 -> 64 -> 3
using ShapeC2 = Shape<32, 64, 2>;
using ShapeC4 = Shape<64, 64, 3>;

hipError_t launch_train(int shape, int type, const TrainDesc &d, int num_wg, size_t lds, hipStream_t s)
{
    if (type != NT_UNCONSTRAINED)
        return hipErrorInvalidValue;
    switch (shape) {
    case kShapeRef:
        return launch_one<ShapeRef, 3>(d, num_wg, lds, s);
    case kShapeC1:
        return launch_one<ShapeC1, 8>(d, num_wg, lds, s);
    case kShapeC2:
        return launch_one<ShapeC2, 16>(d, num_wg, lds, s);
    case kShapeC4:
        return launch_one<ShapeC4, 16>(d, num_wg, lds, s);
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_prep_weights(int shape, const PrepDesc &d, hipStream_t s)
{
    switch (shape) {
    case kShapeRef:
        return launch_prep<ShapeRef>(d, s);
    case kShapeC1:
        return launch_prep<ShapeC1>(d, s);
    case kShapeC2:
        return launch_prep<ShapeC2>(d, s);
    case kShapeC4:
        return launch_prep<ShapeC4>(d, s);
    default:
        return hipErrorInvalidValue;
    }
}

template <class S>
static size_t weight_bytes()
{
    return (size_t)S::all_frags() * kWave * 16 + (((size_t)S::bias_total() * 4 + 255) / 256) * 256;
}

size_t train_weight_bytes(int shape)
{
    switch (shape) {
    case kShapeRef:
        return weight_bytes<ShapeRef>();
    case kShapeC1:
        return weight_bytes<ShapeC1>();
    case kShapeC2:
        return weight_bytes<ShapeC2>();
    case kShapeC4:
        return weight_bytes<ShapeC4>();
    default:
        return 0;
    }
}

size_t train_frag_bytes(int shape)
{
    switch (shape) {
    case kShapeRef:
        return (size_t)ShapeRef::all_frags() * kWave * 16;
    case kShapeC1:
        return (size_t)ShapeC1::all_frags() * kWave * 16;
    case kShapeC2:
        return (size_t)ShapeC2::all_frags() * kWave * 16;
    case kShapeC4:
        return (size_t)ShapeC4::all_frags() * kWave * 16;
    default:
        return 0;
    }
}

size_t train_xt_bytes(int shape)
{
    switch (shape) {
    case kShapeRef:
        return TrainLayout<ShapeRef>::transpose_bytes;
    case kShapeC1:
        return TrainLayout<ShapeC1>::transpose_bytes;
    case kShapeC2:
        return TrainLayout<ShapeC2>::transpose_bytes;
    case kShapeC4:
        return TrainLayout<ShapeC4>::transpose_bytes;
    default:
        return 0;
    }
}

size_t train_lds_static(int shape)
{
    switch (shape) {
    case kShapeRef:
        return TrainLayout<ShapeRef>::head_bytes;
    case kShapeC1:
        return TrainLayout<ShapeC1>::head_bytes;
    case kShapeC2:
        return TrainLayout<ShapeC2>::head_bytes;
    case kShapeC4:
        return TrainLayout<ShapeC4>::head_bytes;
    default:
        return 0;
    }
}

int train_grad_total(int shape)
{
    switch (shape) {
    case kShapeRef:
        return ShapeRef::grad_total();
    case kShapeC1:
        return ShapeC1::grad_total();
    case kShapeC2:
        return ShapeC2::grad_total();
    case kShapeC4:
        return ShapeC4::grad_total();
    default:
        return 0;
    }
}

} // namespace ntk
