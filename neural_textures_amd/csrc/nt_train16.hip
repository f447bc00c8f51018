// nt_train16.hip — the fused training pass (TrainLoopPass, train.cu:818-915, with
// mlp.h:101-362 and util/atomic.h) specialised for unconstrained latents on gfx950: the
// 2- and 4-grid networks of 16-channel grids (32->64->64->16, 64->64->64->64->16) and the
// reference's own network of four 3-channel grids (12->32->32->16, train.h:9-20).
//
// A workgroup is NG groups of four waves (NG = 2 for the 2-grid network: two waves per
// SIMD, so one wave's LDS and memory latency hides behind the other's work). It owns a
// 64 x 8NG block of region positions; group gr walks rows [8gr, 8gr + 8) as four 16 x 8
// chunks of 128 samples, one 32-sample MFMA tile per wave. Per chunk:
//   - the group's Catmull-Rom target tile is copied into its LDS region by DMA
//     (global_load_lds) at the chunk start and published after the forward pass, so the
//     loads overlap sampling and MLP;
//   - lane group g (lane = 32g + c, sample c) gathers grids g and g + 2 only, so each
//     lane computes one bilinear footprint per fragment pair; the layer-0 weight
//     fragments carry the matching input-feature order;
//   - output rows are ordered 4t + channel for reference texture t, so lane group g
//     evaluates exactly textures g and g + 2 (16 exact Catmull-Rom taps from LDS); the
//     last layer's weight fragments carry the matching output permutation;
//   - dW = X^T dY per layer on MFMA over the group's 128 samples: sample rows in LDS read
//     back transposed (ds_read_b64_tr_b16), each wave owning fixed 32x32 dW tiles
//     accumulated in fp32 registers;
//   - the latent scatter is an MFMA reduction D[cell][ch] = sum_s W[cell][s] dX0[s][ch]
//     over the chunk's cell box (fp32 corner weights split into fp16 hi + lo). Each sample
//     has one scatter-weight row (hi and lo), cleared whole by its two lanes and filled with
//     the corners of the grids each gathers, and the rows are read transposed with
//     ds_read_b64_tr_b16. D goes to the latent gradients
//     with global float atomics, each instruction adding four whole 64-byte texel records
//     (an LDS footprint box with ds_add_f32 in between cost more: an LDS float atomic
//     occupies the LDS for 192 cycles per wave instruction on gfx950, and the chunks'
//     cell boxes overlap too little for the box to save global traffic). With 3-channel
//     grids three of the 16 D columns are a grid's channels (the 12-byte records of the
//     reference network).
//   - 3-channel grids whose cell box is too large for the reduction's LDS (grids as fine
//     as the image, or half as fine) sum into an LDS box over the workgroup tile's
//     footprint, added to the gradients once per tile: each sample writes a 16-byte record
//     (fractions, gradient, footprint origin), and each box texel gathers the corners that
//     land on it from the few positions that can reach it (3 x 3 or 4 x 4), with plain
//     LDS adds: no atomics.
// MLP gradients go to one partial row per group, summed by the deterministic two-stage
// reduction of nt_train.hip.
#include "nt_train_parts.hpp"

#include <mutex>

namespace ntk {


template <class S, int NG>
struct T16Layout {
    static constexpr int G = S::K0 / 16;
    static constexpr int frag_bytes = S::all_frags() * kWave * 16;
    static constexpr int bias_bytes = ((S::bias_total() * 4 + 15) / 16) * 16;
    static constexpr int head_bytes = frag_bytes + bias_bytes;
    // dW work items: a layer with at most two 32x32 tiles has each tile's 128-sample
    // reduction split into two halves (two items), so that all four waves of a group work
    // in every dW phase. Items are enumerated from the last layer down; wave w owns items
    // w, w + 4, ... (one accumulator slot each).
    static constexpr bool split(int l) { return S::dw_tiles(l) <= 2; }
    static constexpr int items(int l) { return S::dw_tiles(l) * (split(l) ? 2 : 1); }
    static constexpr int item_start(int l)
    {
        int o = 0;
        for (int j = S::L - 1; j > l; --j)
            o += items(j);
        return o;
    }
    // Index of layer l's first tile among the split tiles (the end-of-kernel merge buffer).
    static constexpr int split_start(int l)
    {
        int o = 0;
        for (int j = S::L - 1; j > l; --j)
            o += split(j) ? S::dw_tiles(j) : 0;
        return o;
    }
    static constexpr int slots = (item_start(-1) + 3) / 4;
};

// ---- weight preparation (the workgroup prologue) ----------------------------------------
//
// Each workgroup builds its LDS weight image itself from the fp16 weights: the matrices are
// first staged in LDS as they lie in memory (W_l[n * kin + k], padded), the last layer's
// rows already in output-row order, then read back as MFMA fragments. The image depends on
// the weights only, so every workgroup builds the same one; there is no separate
// preparation launch per step.

// Half offset of layer l's matrix in the staged copy.
template <class S>
__host__ __device__ constexpr int raw_off(int l)
{
    int o = 0;
    for (int j = 0; j < l; ++j)
        o += S::kout(j) * S::kin(j);
    return o;
}

// Layer-0 input feature of element e of k-step fragment q in lane group g. 16 channels:
// grid_feature (grids g and g + 2, eight consecutive channels per fragment). 3 channels
// (four grids, one k-step): lane group g holds grid g's channels (e = 0..2), grid g + 2's
// (e = 3..5) and two of the padding features 12..15 (e = 6, 7), so that each lane samples
// two grids and the two groups together cover all sixteen inputs.
template <int C>
__host__ __device__ constexpr int input_feature(int q, int g, int e)
{
    if constexpr (C == 16)
        return grid_feature(q, g, e);
    else
        return e < 3 ? 3 * g + e : e < 6 ? 3 * (g + 2) + (e - 3) : 12 + 2 * g + (e - 6);
}

// Output index of output row r (r < 16): nibble r of the packed permutation.
__device__ __forceinline__ int perm_row(uint64_t perm, int r) { return (int)((perm >> (4 * r)) & 15u); }

// Stage the weight matrices (16-byte loads; every matrix is a whole number of 16-byte
// rows) and the fp32 bias rows. All global loads are issued before the first LDS store, so
// the copy costs one memory round trip.
template <class S, int NT>
__device__ __forceinline__ void stage_weights16(const Train16Desc &d, uint16_t *raw, float *bias, int tid)
{
    constexpr int L = S::L;
    static_assert(L <= 4, "train16 networks have at most four layers");
    constexpr int I0 = (S::kout(0) * S::kin(0) / 8 + NT - 1) / NT;
    constexpr int I1 = (S::kout(1) * S::kin(1) / 8 + NT - 1) / NT;
    constexpr int I2 = L > 2 ? (S::kout(2) * S::kin(2) / 8 + NT - 1) / NT : 0;
    constexpr int I3 = L > 3 ? (S::kout(3) * S::kin(3) / 8 + NT - 1) / NT : 0;
    constexpr int it[4] = {I0, I1, I2, I3};
    constexpr int first[4] = {0, I0, I0 + I1, I0 + I1 + I2};
    uint4 v[I0 + I1 + I2 + I3 > 0 ? I0 + I1 + I2 + I3 : 1];
    uint16_t bv[L];
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const uint4 *W = (const uint4 *)d.mlp.W[l];
        const int n4 = S::kout(l) * S::kin(l) / 8;
        // Loads from clamped (always valid) addresses, so that none sits under a branch.
#pragma unroll
        for (int j = 0; j < it[l]; ++j)
            v[first[l] + j] = load_global(W + min(tid + j * NT, n4 - 1));
        // Bias row tid of layer l (output-row order on the last layer); 0 past the outputs.
        const int n = l == L - 1 ? (tid < NT_MAX_OUTPUTS ? perm_row(d.perm, tid) : NT_MAX_OUTPUTS) : tid;
        const uint16_t b = load_global(d.mlp.B[l] + min(n, d.mlp.sizes[l + 1] - 1));
        bv[l] = n < d.mlp.sizes[l + 1] ? b : (uint16_t)0;
    }
    // Keeps the loads above the conditional stores below (the compiler would otherwise sink
    // each load to its store and wait for it there).
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
#pragma unroll
    for (int l = 0; l < L; ++l) {
        const int n4 = S::kout(l) * S::kin(l) / 8;
        uint4 *dst = (uint4 *)(raw + raw_off<S>(l));
#pragma unroll
        for (int j = 0; j < it[l]; ++j) {
            const int i = tid + j * NT;
            if (i < n4)
                dst[i] = v[first[l] + j];
        }
        if (tid < 32 * S::t32(S::kout(l)))
            bias[S::bias_off(l) + tid] = h2f(bv[l]);
    }
}

// Fragment f (wave-uniform) for lane (c, g), read from the staged matrices.
template <class S, int C>
__device__ __forceinline__ h8 weight_fragment16(const uint16_t *raw, uint64_t perm, int f, int lane)
{
    const int c = lane & 31, g = lane >> 5;
    const bool fwd = f < S::fwd_total();
    int l = 0;
    if (fwd) {
        while (l + 1 < S::L && f >= S::fwd_off(l + 1))
            ++l;
    } else {
        while (l + 1 < S::L && f >= S::bwd_off(l + 1))
            ++l;
    }
    const int kin = S::kin(l), kout = S::kout(l);
    const bool last = l == S::L - 1;
    const uint16_t *W = raw + raw_off<S>(l);
    h8 v;
    if (fwd) {
        // Forward fragment (a, q): A[row][kk] = W_l[n][k], row = 32a + c, n the output of that
        // row (permuted on the last layer), k = the input of (q, g, e): eight consecutive
        // inputs on layer 0, two runs of four on the others.
        const int local = f - S::fwd_off(l), qn = kin / 16;
        const int a = local / qn, q = local % qn;
        const int row = 32 * a + c;
        if (row < kout) {
            const int n = last ? perm_row(perm, row) : row;
            const uint16_t *wr = W + n * kin;
            if (l == 0 && C == 16) {
                v = *(const h8 *)(wr + grid_feature(q, g, 0));
            } else if (l == 0) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    v[e] = bits_h(wr[input_feature<C>(q, g, e)]);
            } else {
                const h4 lo = *(const h4 *)(wr + chained_feature(q, g, 0));
                const h4 hi = *(const h4 *)(wr + chained_feature(q, g, 4));
                v = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
            }
        } else {
            v = (h8)(_Float16)0.f;
        }
    } else {
        // Backward fragment (mt, q): A[k][kk] = W_l[n][k], k = 32mt + c, n the output of the
        // chained row (q, g, e).
        const int local = f - S::bwd_off(l), qn = kout / 16;
        const int mt = local / qn, q = local % qn;
        const int k = 32 * mt + c;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int row = chained_feature(q, g, e);
            const int n = last ? perm_row(perm, row) : row;
            v[e] = k < kin ? bits_h(W[n * kin + k]) : (_Float16)0.f;
        }
    }
    return v;
}

// ---- device pieces ---------------------------------------------------------------------

__device__ __forceinline__ h4 lds_read_tr16(const _Float16 *p)
{
    typedef short s4 __attribute__((ext_vector_type(4)));
    const s4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s4 *)p);
    return __builtin_bit_cast(h4, v);
}

// Start the copy of the chunk's target tile (texels [cx0-2, cx0+18) x [cy0-2, cy0+10) of
// every texture, wrapped like the reference's texture objects, main.cpp:613-621) into the
// group's LDS tile with global_load_lds_dwordx4: wave w copies slots 64(w + 4k) + lane of
// each texture, each wave instruction filling 64 consecutive float4 slots (two tile rows;
// the 12 padding slots of a row repeat its last texel). No registers are held; the caller
// waits for vmcnt(0) before the barrier that publishes it.
// A 16-byte copy from global memory into LDS (at the wave-uniform dst + 16 lane) issued
// from inline assembly, so that the compiler does not track it as an LDS write: it then
// adds no wait for all outstanding memory operations before the next LDS read (it cannot
// tell LDS buffers apart), and the kernel waits for these copies itself (vmcnt) before any
// read of what they write. M0 (the copy's LDS address) is saved and restored around it,
// so the compiler's own use of M0 is undisturbed; one wait state separates the M0 write
// from the copy, and one the copy from the restore.
__device__ __forceinline__ void dma16_untracked(const void *src, void *dst)
{
    const uint32_t m0 = __builtin_amdgcn_readfirstlane(
        (uint32_t)(uintptr_t)(__attribute__((address_space(3))) void *)dst);
    uint32_t saved;
    asm volatile("s_mov_b32 %0, m0\n\ts_mov_b32 m0, %2\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, off\n\t"
                 "s_nop 0\n\ts_mov_b32 m0, %0"
                 : "=&s"(saved)
                 : "v"(src), "s"(m0)
                 : "memory");
}

template <bool UNTRACKED = false>
__device__ __forceinline__ void tile_fetch_async(const Train16Desc &d, float4 *tile, int cx0, int cy0,
                                                 int wave, int lane)
{
    static_assert(kT16TileSlots % 64 == 0, "whole wave instructions");
    for (int base = 64 * wave; base < kT16TileSlots; base += 64 * 4) {
        const int i = base + lane;
        const int ty = i / kT16TileStride, tx = min(i % kT16TileStride, kT16TileW - 1);
        int gx = cx0 - kT16TileX0 + tx, gy = cy0 - kT16TileX0 + ty;
        gx = (unsigned)gx < (unsigned)d.image_w ? gx : wrap_coord(gx, d.image_w);
        gy = (unsigned)gy < (unsigned)d.image_h ? gy : wrap_coord(gy, d.image_h);
        const int64_t off = ((int64_t)gy * d.image_w + gx) * 4; // same texel of every texture
        // Unrolled over the (at most four) textures so that their pointers stay in SGPRs.
#pragma unroll
        for (int t = 0; t < 4; ++t)
            if (t < d.ntex) {
                if constexpr (UNTRACKED)
                    dma16_untracked((const void *)(d.tex[t] + off), (void *)(tile + t * kT16TileSlots + base));
                else
                    __builtin_amdgcn_global_load_lds((const void *)(d.tex[t] + off),
                                                     (__attribute__((address_space(3))) void *)(tile + t * kT16TileSlots + base),
                                                     16, 0, 0);
            }
    }
}

// The 16 Catmull-Rom taps of one texture from the LDS tile, fp32 fma in tap order; the
// fourth channel only where some texture has one.
template <bool FOUR, bool PF>
__device__ __forceinline__ void cr_taps(const float4 *base, const float (&wx)[4], const float (&wy)[4],
                                        float (&acc)[4])
{
    if constexpr (!PF) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float4 p = base[jj * kT16TileStride + i];
                const float wxy = wx[i] * wy[jj];
                acc[0] = fmaf(p.x, wxy, acc[0]);
                acc[1] = fmaf(p.y, wxy, acc[1]);
                acc[2] = fmaf(p.z, wxy, acc[2]);
                if (FOUR)
                    acc[3] = fmaf(p.w, wxy, acc[3]);
            }
        return;
    }
    // With registers to spare, all 16 tap reads are issued before the first fma (one LDS
    // round trip, not sixteen).
    float4 p[4][4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            p[jj][i] = base[jj * kT16TileStride + i];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float wxy = wx[i] * wy[jj];
            acc[0] = fmaf(p[jj][i].x, wxy, acc[0]);
            acc[1] = fmaf(p[jj][i].y, wxy, acc[1]);
            acc[2] = fmaf(p[jj][i].z, wxy, acc[2]);
            if (FOUR)
                acc[3] = fmaf(p[jj][i].w, wxy, acc[3]);
        }
}

// Two channels (an 8-byte half of each tap's float4, `half` 0 or 1) of one texture.
template <bool PF>
__device__ __forceinline__ void cr_taps2(const float4 *base, int half, const float (&wx)[4], const float (&wy)[4],
                                         float (&acc)[4])
{
    const float2 *b2 = (const float2 *)base + half;
    if constexpr (!PF) {
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float2 q = b2[2 * (jj * kT16TileStride + i)];
                const float wxy = wx[i] * wy[jj];
                acc[0] = fmaf(q.x, wxy, acc[0]);
                acc[1] = fmaf(q.y, wxy, acc[1]);
            }
        return;
    }
    float2 p[4][4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            p[jj][i] = b2[2 * (jj * kT16TileStride + i)];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float wxy = wx[i] * wy[jj];
            acc[0] = fmaf(p[jj][i].x, wxy, acc[0]);
            acc[1] = fmaf(p[jj][i].y, wxy, acc[1]);
        }
}

// Catmull-Rom targets and loss weights of the lane's eight output rows 8j + 4g + ch,
// j = 0, 1: texture t = g + 2j, channel ch; with three textures (split3) rows 8 + 4g + ch
// are channels 2g + ch of texture 2 (train.cu:105-157; 16 taps, exact weights, the fp32
// fma order of the scalar restatement). Rows without a texture channel are the
// reference's unused outputs: target 0, weight 1.
template <bool PF>
__device__ __forceinline__ void lane_targets16(const Train16Desc &d, const float4 *tile, int cx0, int cy0,
                                               float u, float v, int g, float (&t)[8], float (&wt)[8])
{
    float wx[4], wy[4];
    const int gx0 = cr_axis(u, d.image_w, wx), gy0 = cr_axis(v, d.image_h, wy);
    const int x0 = gx0 - (cx0 - kT16TileX0), y0 = gy0 - (cy0 - kT16TileX0);
    const bool inside = x0 >= 0 && x0 + 3 < kT16TileW && y0 >= 0 && y0 + 3 < kT16TileH;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const bool half = PF && j == 1 && d.split3; // channels 2g, 2g + 1 of texture 2 (one group)
        const int ti = half ? 2 : g + 2 * j;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        if (half) {
            if (inside) {
                cr_taps2<PF>(tile + 2 * kT16TileSlots + y0 * kT16TileStride + x0, g, wx, wy, acc);
            } else {
                const float *tex = sreg(d.tex[2]);
                for (int jj = 0; jj < 4; ++jj) {
                    const int y = wrap_coord(gy0 + jj, d.image_h);
                    for (int i = 0; i < 4; ++i) {
                        const int x = wrap_coord(gx0 + i, d.image_w);
                        const float2 p = load_global((const float2 *)(tex + ((int64_t)y * d.image_w + x) * 4) + g);
                        const float wxy = wx[i] * wy[jj];
                        acc[0] = fmaf(p.x, wxy, acc[0]);
                        acc[1] = fmaf(p.y, wxy, acc[1]);
                    }
                }
            }
        } else if (ti < d.ntex) {
            if (inside) {
                const float4 *base = tile + ti * kT16TileSlots + y0 * kT16TileStride + x0;
                if (d.four_channels)
                    cr_taps<true, PF>(base, wx, wy, acc);
                else
                    cr_taps<false, PF>(base, wx, wy, acc);
            } else {
                const float *tex = g ? sreg(d.tex[2 * j + 1]) : sreg(d.tex[2 * j]);
                for (int jj = 0; jj < 4; ++jj) {
                    const int y = wrap_coord(gy0 + jj, d.image_h);
                    for (int i = 0; i < 4; ++i) {
                        const int x = wrap_coord(gx0 + i, d.image_w);
                        const float4 p = load_global((const float4 *)(tex + ((int64_t)y * d.image_w + x) * 4));
                        const float wxy = wx[i] * wy[jj];
                        acc[0] = fmaf(p.x, wxy, acc[0]);
                        acc[1] = fmaf(p.y, wxy, acc[1]);
                        acc[2] = fmaf(p.z, wxy, acc[2]);
                        acc[3] = fmaf(p.w, wxy, acc[3]);
                    }
                }
            }
        }
        int nch = ti < d.ntex ? (g ? sreg(d.tex_nch[2 * j + 1]) : sreg(d.tex_nch[2 * j])) : 0;
        float lw = g ? sreg(d.tex_w[2 * j + 1]) : sreg(d.tex_w[2 * j]);
        if (half) {
            nch = min(max(sreg(d.tex_nch[2]) - 2 * g, 0), 2);
            lw = sreg(d.tex_w[2]);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            t[4 * j + r] = r < nch ? acc[r] : 0.f;
            wt[4 * j + r] = r < nch ? lw : 1.f;
        }
    }
}

// NT_SAMPLES_RANDOM: the lane's Catmull-Rom taps straight from the textures (textures g and
// g + 2, wrapped like the reference's texture objects, main.cpp:613-621). All loads are
// issued at the start of the chunk and consumed after the forward pass, so their latency
// overlaps the gathers and the MLP.
struct LaneTaps {
    float4 p[2][16];
    float wx[4], wy[4];
};

__device__ __forceinline__ void issue_taps(const Train16Desc &d, float u, float v, int g, LaneTaps &tp)
{
    const int gx0 = cr_axis(u, d.image_w, tp.wx), gy0 = cr_axis(v, d.image_h, tp.wy);
    int xo[4], yo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xo[i] = wrap_near(gx0 + i, d.image_w);
        yo[i] = wrap_near(gy0 + i, d.image_h) * d.image_w;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const float4 *tex = (const float4 *)(g ? sreg(d.tex[2 * j + 1]) : sreg(d.tex[2 * j]));
        if (g + 2 * j < d.ntex) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    tp.p[j][4 * jj + i] = load_global(tex + (uint32_t)(yo[jj] + xo[i]));
        }
    }
}

// Targets and loss weights of the lane's eight output rows from its prefetched taps (same
// fma order as lane_targets16).
__device__ __forceinline__ void taps_targets(const Train16Desc &d, const LaneTaps &tp, int g, float (&t)[8],
                                             float (&wt)[8])
{
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int ti = g + 2 * j;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        if (ti < d.ntex) {
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float4 p = tp.p[j][4 * jj + i];
                    const float wxy = tp.wx[i] * tp.wy[jj];
                    acc[0] = fmaf(p.x, wxy, acc[0]);
                    acc[1] = fmaf(p.y, wxy, acc[1]);
                    acc[2] = fmaf(p.z, wxy, acc[2]);
                    acc[3] = fmaf(p.w, wxy, acc[3]);
                }
        }
        const int nch = ti < d.ntex ? (g ? sreg(d.tex_nch[2 * j + 1]) : sreg(d.tex_nch[2 * j])) : 0;
        const float lw = g ? sreg(d.tex_w[2 * j + 1]) : sreg(d.tex_w[2 * j]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            t[4 * j + r] = r < nch ? acc[r] : 0.f;
            wt[4 * j + r] = r < nch ? lw : 1.f;
        }
    }
}

// Two groups (256 registers a wave): the same targets with each texture's 16 taps loaded
// just before its fmas, so that only one texture's taps are live at a time.
__device__ __forceinline__ void taps_targets_late(const Train16Desc &d, float u, float v, int g, float (&t)[8],
                                                  float (&wt)[8])
{
    float wx[4], wy[4];
    const int gx0 = cr_axis(u, d.image_w, wx), gy0 = cr_axis(v, d.image_h, wy);
    int xo[4], yo[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        xo[i] = wrap_near(gx0 + i, d.image_w);
        yo[i] = wrap_near(gy0 + i, d.image_h) * d.image_w;
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int ti = g + 2 * j;
        float acc[4] = {0.f, 0.f, 0.f, 0.f};
        if (ti < d.ntex) {
            const float4 *tex = (const float4 *)(g ? sreg(d.tex[2 * j + 1]) : sreg(d.tex[2 * j]));
            float4 p[16];
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    p[4 * jj + i] = load_global(tex + (uint32_t)(yo[jj] + xo[i]));
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float wxy = wx[i] * wy[jj];
                    acc[0] = fmaf(p[4 * jj + i].x, wxy, acc[0]);
                    acc[1] = fmaf(p[4 * jj + i].y, wxy, acc[1]);
                    acc[2] = fmaf(p[4 * jj + i].z, wxy, acc[2]);
                    acc[3] = fmaf(p[4 * jj + i].w, wxy, acc[3]);
                }
        }
        const int nch = ti < d.ntex ? (g ? sreg(d.tex_nch[2 * j + 1]) : sreg(d.tex_nch[2 * j])) : 0;
        const float lw = g ? sreg(d.tex_w[2 * j + 1]) : sreg(d.tex_w[2 * j]);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            t[4 * j + r] = r < nch ? acc[r] : 0.f;
            wt[4 * j + r] = r < nch ? lw : 1.f;
        }
    }
}

// Bilinear footprint at mip 0 of a w x h grid (train.cu:284-303, z = 0).
__device__ __forceinline__ Footprint footprint16(int w, int h, float u, float v)
{
    return bilinear_footprint(u, v, w, h, 1.f);
}

// Gather grids g + 2j of the lane into fragments 2j (channels 0-7) and 2j + 1 (8-15);
// corner contributions rounded to fp16 and summed in fp16, corner by corner
// (train.cu:293-310).
// With PF every corner load of every grid pair is issued before the first product (one
// memory round trip for the 4-grid network instead of two).
template <int G, bool PF = false>
__device__ __forceinline__ void gather16(const Train16Desc &d, float u, float v, int g, h8 (&x)[G])
{
    constexpr int J = G / 2, JL = PF ? J : 1; // grid pairs; pairs loaded at once
#pragma unroll
    for (int j0 = 0; j0 < J; j0 += JL) {
        float4 t[JL][4][4];
        Footprint f[JL];
#pragma unroll
        for (int jj = 0; jj < JL; ++jj) {
            const int j = j0 + jj;
            const Grid16 &ga = d.grid[2 * j], &gb = d.grid[2 * j + 1];
            const float *vals = g ? sreg(gb.values) : sreg(ga.values);
            const int w = g ? sreg(gb.w) : sreg(ga.w), h = g ? sreg(gb.h) : sreg(ga.h);
            f[jj] = bilinear_footprint(u, v, w, h, 1.f);
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int tx = wrap_near(f[jj].x0 + (c & 1), w), ty = wrap_near(f[jj].y0 + (c >> 1), h);
                const float4 *p = (const float4 *)(vals + ((int64_t)ty * w + tx) * 16);
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    t[jj][c][k] = load_global(p + k);
            }
        }
#pragma unroll
        for (int jj = 0; jj < JL; ++jj) {
            h8 lo = (h8)(_Float16)0.f, hi = (h8)(_Float16)0.f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                lo = accumulate_products(lo, f[jj].w[c], t[jj][c][0], t[jj][c][1]);
                hi = accumulate_products(hi, f[jj].w[c], t[jj][c][2], t[jj][c][3]);
            }
            x[2 * (j0 + jj)] = lo;
            x[2 * (j0 + jj) + 1] = hi;
        }
    }
}

// The latent texels of a chunk's cell boxes (grid by grid, cb_w x cb_h cells from the box
// origin floor(c0 r - 1/2) that the scatter uses, wrapped into the grid) are copied into an
// LDS buffer without passing through registers: four float4 per cell, at most 64 cells, so
// one wave instruction per wave, lane l of wave w copying float4 64 w + l. What does not
// change from chunk to chunk is set once per launch: the lane's grid and its fields, and
// its cell's place in the box.
struct GboxLane {
    const float *vals; // the grid's mip 0, plus the float4's four floats within the texel
    float rx, ry;
    int w, h, cx, cy;
    bool on;           // the lane has a float4 to copy
};

template <int G>
__device__ __forceinline__ GboxLane gbox_lane(const Train16Desc &d, int wave, int lane)
{
    GboxLane q;
    const int i = 64 * wave + lane, cell = i >> 2;
    q.on = i < d.gbox_items;
    int gi = 0;
#pragma unroll
    for (int k = 1; k < G; ++k)
        gi += cell >= d.grid[k].gcell0 ? 1 : 0;
    const Grid16 &g = d.grid[gi];
    const int local = cell - g.gcell0, cbw = g.cb_w > 0 ? g.cb_w : 1;
    q.cy = local / cbw;
    q.cx = local - q.cy * cbw;
    q.vals = g.values + 4 * (i & 3);
    q.rx = g.rx;
    q.ry = g.ry;
    q.w = g.w;
    q.h = g.h;
    return q;
}

__device__ __forceinline__ void gbox_fetch_async(const GboxLane &q, float4 *buf, int cx0, int cy0, int wave)
{
    if (q.on) {
        int tx = (int)floorf(fmaf((float)cx0, q.rx, -0.5f)) + q.cx;
        int ty = (int)floorf(fmaf((float)cy0, q.ry, -0.5f)) + q.cy;
        tx = (unsigned)tx < (unsigned)q.w ? tx : wrap_coord(tx, q.w);
        ty = (unsigned)ty < (unsigned)q.h ? ty : wrap_coord(ty, q.h);
        dma16_untracked((const void *)(q.vals + (uint32_t)(ty * q.w + tx) * 16u), (void *)(buf + 64 * wave));
    }
}

// gather16 with the corners read from the chunk's gather boxes in LDS: the same values,
// products and fp16 sums. A wave with a footprint outside its grid's box (not expected: the
// box covers every corner a chunk position can reach) reads global memory instead.
template <int G>
__device__ __forceinline__ void gather16_box(const Train16Desc &d, const float4 *box, const Grid16 (&own)[G / 2],
                                             int cx0, int cy0, float u, float v, int g, h8 (&x)[G])
{
    constexpr int J = G / 2;
    Footprint f[J];
    int a[J];
    bool in = true;
#pragma unroll
    for (int j = 0; j < J; ++j) {
        const int cbw = own[j].cb_w;
        f[j] = bilinear_footprint(u, v, own[j].w, own[j].h, 1.f);
        const int lx = f[j].x0 - (int)floorf(fmaf((float)cx0, own[j].rx, -0.5f));
        const int ly = f[j].y0 - (int)floorf(fmaf((float)cy0, own[j].ry, -0.5f));
        in = in && lx >= 0 && lx + 1 < cbw && ly >= 0 && ly + 1 < own[j].cb_h;
        a[j] = 4 * (own[j].gcell0 + ly * cbw + lx);
    }
    if (__ballot(!in) != 0) {
        gather16<G, true>(d, u, v, g, x);
        return;
    }
    typedef float nf4 __attribute__((ext_vector_type(4)));
    typedef __attribute__((address_space(3))) const nf4 lds_nf4;
    lds_nf4 *lb = (lds_nf4 *)box;
    // Grid pair by grid pair: the next pair's 16 reads are issued before this pair's
    // products, so that their latency overlaps them.
    float4 t[J][4][4];
    auto load = [&](int j) {
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int o = a[j] + ((c >> 1) ? 4 * own[j].cb_w : 0) + ((c & 1) ? 4 : 0);
#pragma unroll
            for (int k = 0; k < 4; ++k)
                t[j][c][k] = __builtin_bit_cast(float4, lb[o + k]);
        }
    };
    load(0);
#pragma unroll
    for (int j = 0; j < J; ++j) {
        if (j + 1 < J) {
            // This pair's data first (s_waitcnt lgkmcnt(0), which the compiler's own wait
            // placement then counts), then the next pair's reads, kept ahead of the products.
            __builtin_amdgcn_s_waitcnt(0xC07F);
            load(j + 1);
            __builtin_amdgcn_sched_barrier(0);
        }
        h8 lo = (h8)(_Float16)0.f, hi = (h8)(_Float16)0.f;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            lo = accumulate_products(lo, f[j].w[c], t[j][c][0], t[j][c][1]);
            hi = accumulate_products(hi, f[j].w[c], t[j][c][2], t[j][c][3]);
        }
        x[2 * j] = lo;
        x[2 * j + 1] = hi;
    }
}

// The reference network's gather (four 3-channel grids): lane group g samples grids g and
// g + 2 into elements 0-2 and 3-5 of its one fragment (input_feature<3>), elements 6 and 7
// (padding features) zero. All 24 corner loads are issued before the first product; each
// channel's corner products are rounded to fp16 and summed in fp16, corner by corner
// (train.cu:293-310).
__device__ __forceinline__ void gather3(const Train16Desc &d, float u, float v, int g, h8 (&x)[1])
{
    float t[2][4][3];
    Footprint f[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const Grid16 &ga = d.grid[2 * j], &gb = d.grid[2 * j + 1];
        const float *vals = g ? sreg(gb.values) : sreg(ga.values);
        const int w = g ? sreg(gb.w) : sreg(ga.w), h = g ? sreg(gb.h) : sreg(ga.h);
        f[j] = bilinear_footprint(u, v, w, h, 1.f);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            const int tx = wrap_near(f[j].x0 + (c & 1), w), ty = wrap_near(f[j].y0 + (c >> 1), h);
            const float *p = vals + (uint32_t)(ty * w + tx) * 3u;
#pragma unroll
            for (int k = 0; k < 3; ++k)
                t[j][c][k] = load_global(p + k);
        }
    }
    h8 acc = (h8)(_Float16)0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            _Float16 a = (_Float16)0.f;
#pragma unroll
            for (int c = 0; c < 4; ++c)
                a = a + half_of_product(f[j].w[c], t[j][c][k]);
            acc[3 * j + k] = a;
        }
    x[0] = acc;
}

// Write the layer-0 inputs transposed, rows in natural feature order.
template <int G>
__device__ __forceinline__ void store_inputs_transposed(_Float16 *buf, const h8 (&v)[G], int col, int g)
{
#pragma unroll
    for (int q = 0; q < G; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e)
            buf[grid_feature(q, g, e) * kRowStride + col] = v[q][e];
}

// ---- sample-row tiles for the dW products --------------------------------------------------
//
// The group's layer inputs and output gradients are stored as sample rows
// ([sample][kFeatStride] fp16: 8-byte stores of the chained runs of four features) and read
// back transposed with ds_read_b64_tr_b16, which hands each lane of a 16-lane group four
// consecutive samples of one feature: the K-major operands of dW = X^T dY.

// Chained fragments q of the lane's sample: features 16q + 4g + (0..3), 16q + 8 + 4g + (0..3).
template <int NQ, int STRIDE = kFeatStride>
__device__ __forceinline__ void store_rows(_Float16 *buf, const h8 (&v)[NQ], int col, int g)
{
    _Float16 *row = buf + col * STRIDE + 4 * g;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        *(h4 *)(row + 16 * q) = __builtin_shufflevector(v[q], v[q], 0, 1, 2, 3);
        *(h4 *)(row + 16 * q + 8) = __builtin_shufflevector(v[q], v[q], 4, 5, 6, 7);
    }
}

// Layer-0 inputs at their natural feature positions. 16 channels (grid_feature order):
// eight consecutive features per fragment, two 8-byte stores (rows are 8-byte aligned);
// 3 channels: eight scalar stores.
template <int C, int NQ>
__device__ __forceinline__ void store_input_rows(_Float16 *buf, const h8 (&v)[NQ], int col, int g)
{
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        if constexpr (C == 16) {
            _Float16 *p = buf + col * kFeatStride + grid_feature(q, g, 0);
            *(h4 *)p = __builtin_shufflevector(v[q], v[q], 0, 1, 2, 3);
            *(h4 *)(p + 4) = __builtin_shufflevector(v[q], v[q], 4, 5, 6, 7);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                buf[col * kFeatStride + input_feature<C>(q, g, e)] = v[q][e];
        }
    }
}

// Samples s0 .. s0 + 7 of feature f0 + i16 (i16 = lane within its 16-lane group; s0 and f0
// uniform over the group) from rows of STRIDE halves.
template <int STRIDE = kFeatStride>
__device__ __forceinline__ h8 read_cols8(const _Float16 *buf, int s0, int f0, int i16)
{
    const _Float16 *p = buf + (s0 + (i16 >> 2)) * STRIDE + f0 + 4 * (i16 & 3);
    const h4 a = lds_read_tr16(p), b = lds_read_tr16(p + 4 * STRIDE);
    return __builtin_shufflevector(a, b, 0, 1, 2, 3, 4, 5, 6, 7);
}

// dW += X^T dY over the group's 128 samples for the dW tiles this wave owns (mlp.h:101-220).
// A tile (a, 0) also sums its A operand (the output gradient of feature 32a + c over the
// lane group's samples) into the tile's bias accumulator: fp32 sums of fp16 values, two per
// v_dot2_f32_f16.
template <class S, int l, bool PF = false>
__device__ __forceinline__ void dw_rows(const _Float16 *xs, const _Float16 *dys, f16v (&acc)[T16Layout<S, 1>::slots],
                                        float (&db)[T16Layout<S, 1>::slots], int wave, int lane)
{
    using LY = T16Layout<S, 1>;
    constexpr int kin = S::kin(l), kout = S::kout(l);
    constexpr int KB = S::t32(kin);
    constexpr bool SPLIT = LY::split(l);
    constexpr int start = LY::item_start(l), nitems = LY::items(l);
    constexpr int QN = SPLIT ? kChunk / 32 : kChunk / 16; // 16-sample k-steps per item
    const int c = lane & 31, g = lane >> 5, i16 = lane & 15, half = 16 * (c >> 4);
    const h2 one = {(_Float16)1.f, (_Float16)1.f};
#pragma unroll
    for (int j = 0; j < LY::slots; ++j) {
        const int it = 4 * j + wave - start;
        if (it >= 0 && it < nitems) {
            const int t = SPLIT ? it >> 1 : it, q0 = SPLIT ? (it & 1) * QN : 0;
            const int a = t / KB, b = t % KB;
            const bool arow = 32 * a + c < kout, brow = 32 * b + c < kin;
            if constexpr (PF) {
                // every k-step's operands first, then the MFMA chain
                h8 A[QN], B[QN];
#pragma unroll
                for (int qq = 0; qq < QN; ++qq) {
                    A[qq] = read_cols8(dys, 16 * (q0 + qq) + 8 * g, 32 * a + half, i16);
                    B[qq] = read_cols8(xs, 16 * (q0 + qq) + 8 * g, 32 * b + half, i16);
                }
#pragma unroll
                for (int qq = 0; qq < QN; ++qq) {
                    if (!arow)
                        A[qq] = (h8)(_Float16)0.f;
                    if (!brow)
                        B[qq] = (h8)(_Float16)0.f;
                    acc[j] = mfma32(A[qq], B[qq], acc[j]);
                    if (b == 0) {
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const h2 pair = {A[qq][e], A[qq][e + 1]};
                            db[j] = __builtin_amdgcn_fdot2(pair, one, db[j], false);
                        }
                    }
                }
                continue;
            }
#pragma unroll
            for (int qq = 0; qq < QN; ++qq) {
                const int q = q0 + qq;
                h8 A = read_cols8(dys, 16 * q + 8 * g, 32 * a + half, i16);
                h8 B = read_cols8(xs, 16 * q + 8 * g, 32 * b + half, i16);
                if (!arow)
                    A = (h8)(_Float16)0.f;
                if (!brow)
                    B = (h8)(_Float16)0.f;
                acc[j] = mfma32(A, B, acc[j]);
                if (b == 0) {
#pragma unroll
                    for (int e = 0; e < 8; e += 2) {
                        const h2 pair = {A[e], A[e + 1]};
                        db[j] = __builtin_amdgcn_fdot2(pair, one, db[j], false);
                    }
                }
            }
        }
    }
}

// Backward through hidden layer l (its input is hidden activation l-1), then l-1 ... 1.
template <class S, int l, bool PF>
__device__ __forceinline__ void backward_hidden_rows(_Float16 *xs, _Float16 *dys, const h8 *frags,
                                                     const h8 (&xh)[S::NH][S::H / 16], h8 (&dyh)[S::H / 16],
                                                     f16v (&dwacc)[T16Layout<S, 1>::slots],
                                                     float (&dbt)[T16Layout<S, 1>::slots], int col, int wave,
                                                     int lane)
{
    if constexpr (l >= 1) {
        constexpr int HQ = S::H / 16, HA = S::t32(S::H);
        const int g = lane >> 5;
        store_rows<HQ>(dys, dyh, col, g);
        store_rows<HQ>(xs, xh[l - 1], col, g);
        f16v acc[HA];
        layer_backward_dx<HQ, HA, PF>(frags + S::bwd_off(l) * kWave, dyh, acc, lane);
        relu_backward<HQ, HA>(acc, xh[l - 1], dyh);
        __syncthreads();
        dw_rows<S, l, PF>(xs, dys, dwacc, dbt, wave, lane);
        __syncthreads();
        backward_hidden_rows<S, l - 1, PF>(xs, dys, frags, xh, dyh, dwacc, dbt, col, wave, lane);
    }
}

// First dX0 feature of the 16 columns the scatter reduction reads for grid gi: the grid's
// own 16 channels, or (3 channels) the 8-byte-aligned feature at or below 3gi, whose 16
// columns include the grid's three (a transposing LDS read starts on an 8-byte boundary).
template <int C>
__device__ __forceinline__ int dx_col0(int gi)
{
    return C == 16 ? 16 * gi : (C * gi) & ~3;
}

// Column of chunk cell `cell` in the scatter weight rows: within each 16-cell tile the two
// 2-bit halves of the index are swapped, so that D row 4grp + r of the reduction's MFMA
// (lane group grp, element r) holds cell 16t + 4r + grp, and the four cells one atomic
// instruction covers are consecutive (neighbouring texel records) instead of four apart.
__device__ __forceinline__ int cell_column(int cell)
{
    return (cell & ~15) | ((cell & 3) << 2) | ((cell >> 2) & 3);
}

// ---- the kernel ----------------------------------------------------------------------------

// One box texel (X, Y) of a grid of 1/K the image's size (gather_records): the NC x NC
// candidate records (positions [KX - c0, KX - c0 + NC) x [KY - c0, KY - c0 + NC) of the
// chunk pair, read from clamped indices and masked, a block of rows' loads first), the weight of the
// corner that lands on the texel (the footprint's own arithmetic) times the sample's
// gradient, fp32 products summed in candidate order, added to the box texel.
template <int K, int NG>
__device__ __forceinline__ void gather_texel(const uint4 *rec, float *box, int X, int Y, int lx, int ly, int x0,
                                             int y0) // box: the texel's three floats
{
    constexpr int c0 = (K + 1) / 2, NC = (3 * K + 1) / 2 + c0;
    constexpr int RB = K == 1 ? NC : NC / 2; // candidate rows loaded at once (registers)
    const int i0 = K * X - c0 - x0, j0 = K * Y - c0 - y0;
    float s0 = 0.f, s1 = 0.f, s2 = 0.f;
#pragma unroll
    for (int a0 = 0; a0 < NC; a0 += RB) {
        uint4 r[RB][NC];
#pragma unroll
        for (int a = 0; a < RB; ++a)
#pragma unroll
            for (int b = 0; b < NC; ++b) {
                const int jr = min(max(j0 + a0 + a, 0), kChunkH * NG - 1), ir = min(max(i0 + b, 0), kChunkW - 1);
                r[a][b] = rec[(jr / kChunkH) * kChunk + kChunkW * (jr % kChunkH) + ir];
            }
#pragma unroll
        for (int a = 0; a < RB; ++a)
#pragma unroll
            for (int b = 0; b < NC; ++b) {
                const bool in =
                    (unsigned)(j0 + a0 + a) < (unsigned)(kChunkH * NG) && (unsigned)(i0 + b) < (unsigned)kChunkW;
                const int ex = lx - (int)((r[a][b].w >> 16) & 0xFFu), ey = ly - (int)(r[a][b].w >> 24);
                if (!in || (unsigned)ex > 1u || (unsigned)ey > 1u)
                    continue;
                const float fx = __uint_as_float(r[a][b].x), fy = __uint_as_float(r[a][b].y);
                const float wu = ex ? fx : 1.f - fx, wv = ey ? fy : 1.f - fy;
                const float wgt = wu * wv;
                s0 += wgt * (float)bits_h((uint16_t)(r[a][b].z & 0xFFFFu));
                s1 += wgt * (float)bits_h((uint16_t)(r[a][b].z >> 16));
                s2 += wgt * (float)bits_h((uint16_t)(r[a][b].w & 0xFFFFu));
            }
    }
    if (s0 != 0.f || s1 != 0.f || s2 != 0.f) {
        box[0] += s0;
        box[1] += s1;
        box[2] += s2;
    }
}

// The box texels of the chunk pair (positions x0 .. x0 + 15, rows y0 .. y0 + 8NG - 1) for
// the grids with records: texel (x, y) of a grid of 1/k the image's size is reached only by
// the footprints of the positions in [kx - c0, kx - c0 + nc) x [ky - c0, ky - c0 + nc)
// (c0 = ceil(k/2), nc = ceil(3k/2) + c0: 3 for k = 1, 4 for k = 2), and gathers from their
// records (gather_texel). The texels of all such grids are dealt out over the workgroup's
// waves together (whole waves per grid), one thread per texel.
template <int NG>
__device__ __forceinline__ void gather_records(const Train16Desc &d, float *sbox, int x0, int y0, int tx0, int ty0,
                                               int tid)
{
    // Whole waves per grid: grid gi's texels go to wave slots [w_gi, w_gi+1), 64 texels
    // each, so that a wave's grid (and its fields) is uniform.
    auto slots = [&](const Grid16 &q) {
        const int k = max(sreg(q.gk), 1); // 1 or 2 where there are records
        return sreg(q.slot_off) >= 0 ? ((kChunkW / k + 2) * (kChunkH * NG / k + 2) + kWave - 1) / kWave : 0;
    };
    const int w1 = slots(d.grid[0]), w2 = w1 + slots(d.grid[1]), w3 = w2 + slots(d.grid[2]);
    const int w4 = w3 + slots(d.grid[3]);
    const int lane = tid & (kWave - 1);
    for (int ws = tid / kWave; ws < w4; ws += kTrainThreads * NG / kWave) {
        const int gi = __builtin_amdgcn_readfirstlane((ws >= w1) + (ws >= w2) + (ws >= w3));
        const int wbase = gi == 0 ? 0 : gi == 1 ? w1 : gi == 2 ? w2 : w3;
        const Grid16 &q = d.grid[gi];
        const int k = max(q.gk, 1), so = q.slot_off, bw = q.box_w, boff = q.box_off;
        const float rx = q.rx, ry = q.ry;
        const int cell = (ws - wbase) * kWave + lane;
        if (cell >= (kChunkW / k + 2) * (kChunkH * NG / k + 2))
            continue;
        const int ox = (int)floorf(fmaf((float)(d.off_x + tx0), rx, -0.5f)) - 1;
        const int oy = (int)floorf(fmaf((float)(d.off_y + ty0), ry, -0.5f)) - 1;
        // The chunk pair's texels: those its positions' footprints reach.
        const int bx = (int)floorf(fmaf((float)x0, rx, -0.5f)), by = (int)floorf(fmaf((float)y0, ry, -0.5f));
        const int gw = kChunkW / k + 2;
        const int cy = cell / gw, cx = cell - cy * gw;
        const int X = bx + cx, Y = by + cy, lx = X - ox, ly = Y - oy;
        const uint4 *rec = (const uint4 *)(sbox + so);
        float *box = sbox + boff + (ly * bw + lx) * 3;
        if (k == 1)
            gather_texel<1, NG>(rec, box, X, Y, lx, ly, x0, y0);
        else
            gather_texel<2, NG>(rec, box, X, Y, lx, ly, x0, y0);
    }
}

// dW slots per round of the end-of-kernel handoff between the two groups: all of them,
// except for the 4-grid network (random texels), whose group regions hold two.
template <class S>
constexpr int handoff_slots()
{
    return S::K0 == 64 ? 2 : T16Layout<S, 1>::slots;
}

template <class S, int C, int NG, bool RND, bool ORD = false>
__global__ __launch_bounds__(kTrainThreads *NG) void train16_kernel(Train16Desc d)
{
    static_assert(!RND || C == 16, "random texels are built for 16-channel grids");
    using LY = T16Layout<S, NG>;
    // Grids: one per 16 inputs with 16 channels; the 3-channel network has four.
    constexpr int G = C == 16 ? LY::G : 4, L = S::L, NH = S::NH, KQ0 = S::K0 / 16, HQ = S::H / 16,
                  HA = S::t32(S::H);
    // One group (one wave per SIMD) leaves registers to spare: the MLP layers read all their
    // weight fragments and dW operands before their MFMAs (PFM), the target taps, both grid
    // pairs' corners and the scatter reduction's operands before use (PF). Two groups (two
    // waves per SIMD, 256 registers each) prefetch the MLP operands only.
    constexpr bool PF = NG == 1;
    constexpr bool PFM = true;
    static_assert(C == 16 ? KQ0 == G && (G == 2 || G == 4) : C == 3 && KQ0 == 1,
                  "16 channels: one grid per k-step; 3 channels: four grids in one k-step");
    extern __shared__ __align__(16) unsigned char smem[];
    h8 *frags = (h8 *)smem;
    float *bias = (float *)(smem + LY::frag_bytes);

    const int tid = threadIdx.x, t256 = tid & (kTrainThreads - 1), gr = tid >> 8;
    const int lane = tid & 63, wave = t256 >> 6, c = lane & 31, g = lane >> 5;
    unsigned char *gbase = smem + d.group_off + gr * d.group_bytes;
    float4 *tile = (float4 *)gbase;
    _Float16 *un = (_Float16 *)(gbase + d.tile_bytes);
    _Float16 *xs = un;                          // layer inputs, [sample][kFeatStride]
    _Float16 *dys = xs + kChunk * kFeatStride;  // layer output gradients, [sample][kFeatStride]
    _Float16 *dxs = un;                         // scatter: dX0 rows [sample][dx_stride(K0)]
    _Float16 *whi = un + kChunk * dx_stride(S::K0); // scatter weights [sample][wcols], hi
    _Float16 *wlo = whi + kChunk * d.wcols;     // ... lo

    // The tile of the workgroup's k-th turn (k = b0 / gridDim.x) and its origin.
    auto tile_origin = [&](int b0, int &tx0, int &ty0) {
        int b = b0;
        if (d.xcd_per > 0)
            b = (b & 7) * d.xcd_per + (b >> 3); // the workgroups of one XCD share an L2: give them neighbouring tiles
        tx0 = (b % d.tiles_x) * (kChunkW * 4);
        ty0 = (b / d.tiles_x) * (kChunkH * NG);
        return b;
    };
    // Gather boxes (one group): the first chunk's now, each later chunk's during the chunk
    // before it (two buffers).
    constexpr bool GBOX = PF && !RND && C == 16;
    float4 *gbox = (float4 *)(smem + d.gbox_off);
    const int gbox_step = d.gbox_bytes / 16;
    GboxLane gl{};
    if constexpr (GBOX) {
        if (d.gbox_off != 0) {
            gl = gbox_lane<G>(d, wave, lane);
            int fx0, fy0;
            tile_origin(blockIdx.x, fx0, fy0);
            gbox_fetch_async(gl, gbox, d.off_x + fx0, d.off_y + fy0, wave);
        }
    }
    {
        // Weight image (staged through the group regions, which the tile loop overwrites only
        // after the barriers below) and biases.
        constexpr int NT = kTrainThreads * NG;
        uint16_t *raw = (uint16_t *)(smem + d.group_off);
        stage_weights16<S, NT>(d, raw, bias, tid);
        __syncthreads();
        for (int f = __builtin_amdgcn_readfirstlane(tid >> 6); f < S::all_frags(); f += NT / kWave)
            frags[f * kWave + lane] = weight_fragment16<S, C>(raw, d.perm, f, lane);
        if constexpr (GBOX)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // the first gather boxes
        __syncthreads();
    }

    // NT_LATENT_TOUCHED: one thread logs the step and, for the first step since the
    // optimizer ran, its footprint rectangles.
    if (d.log && blockIdx.x == 0 && tid == 0) {
        UpdateLog *log = d.log;
        if (log->magic != kUpdateLogMagic) {
            log->magic = kUpdateLogMagic;
            log->count = log->consumed = 0u;
        } else if (log->consumed == log->count) {
            log->count = log->consumed = 0u;
        }
        const uint32_t count = log->count + (log->count < 0xffffffffu ? 1u : 0u);
        log->count = count;
        if (count == 1u) {
            log->kind = kUpdateLogTexels;
            for (int gi = 0; gi < NT_MAX_GRIDS; ++gi)
                for (int k = 0; k < 4; ++k)
                    log->rect[gi][k] = d.rect[gi][k];
        }
    }

    // The fields of the grids this lane's group scatters (grid 2j + g), selected once: a
    // lane-dependent select of kernel-argument fields inside the loop becomes per-lane loads
    // or branches.
    Grid16 own[G / 2];
#pragma unroll
    for (int j = 0; j < G / 2; ++j) {
        const Grid16 &qa = d.grid[2 * j], &qb = d.grid[2 * j + 1];
        own[j].w = g ? sreg(qb.w) : sreg(qa.w);
        own[j].h = g ? sreg(qb.h) : sreg(qa.h);
        own[j].cb_w = g ? sreg(qb.cb_w) : sreg(qa.cb_w);
        own[j].cb_h = g ? sreg(qb.cb_h) : sreg(qa.cb_h);
        own[j].ncell = g ? sreg(qb.ncell) : sreg(qa.ncell);
        own[j].wcol0 = g ? sreg(qb.wcol0) : sreg(qa.wcol0);
        own[j].gcell0 = g ? sreg(qb.gcell0) : sreg(qa.gcell0);
        own[j].rx = g ? sreg(qb.rx) : sreg(qa.rx);
        own[j].ry = g ? sreg(qb.ry) : sreg(qa.ry);
        own[j].grads = g ? sreg(qb.grads) : sreg(qa.grads);
        if constexpr (C == 3) {
            own[j].box_off = g ? sreg(qb.box_off) : sreg(qa.box_off);
            own[j].box_w = g ? sreg(qb.box_w) : sreg(qa.box_w);
            own[j].box_h = g ? sreg(qb.box_h) : sreg(qa.box_h);
            own[j].slot_off = g ? sreg(qb.slot_off) : sreg(qa.slot_off);
            own[j].gk = g ? sreg(qb.gk) : sreg(qa.gk);
        }
    }
    float *sbox = (float *)(smem + d.box_lds_off); // per-sample scatter boxes (box_floats)

    // The scatter reduction's tasks (one per grid and 16-cell tile of its chunk cell box,
    // at most eight: the planner keeps no more) go to wave k % 4, so this wave runs tasks
    // wave and wave + 4. Lane group grp of a task holds cells 16 t + 4 r + grp, r = 0..3;
    // their offsets in the cell box are the same for every chunk. With registers to spare
    // (one group) they are computed once: one byte each of cx and cy (the planner keeps at
    // most 128 cells per grid, so both are below 255), two cells per register, 0xFFFF for a
    // cell past the box; two groups (256 registers a wave) compute them per chunk.
    int ntask = 0, task_g[2] = {0, 0}, task_t[2] = {0, 0};
    uint32_t task_cell[2][2] = {{0u, 0u}, {0u, 0u}};
    if constexpr (!RND && PF) {
#pragma unroll
        for (int gi = 0; gi < G; ++gi)
            ntask += (d.grid[gi].ncell + 15) >> 4;
        const int grp = lane >> 4;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            int k = wave + 4 * j, gsel = 0;
#pragma unroll
            for (int gi = 0; gi + 1 < G; ++gi) {
                const int n = (d.grid[gi].ncell + 15) >> 4;
                if (gsel == gi && k >= n) {
                    k -= n;
                    gsel = gi + 1;
                }
            }
            task_g[j] = __builtin_amdgcn_readfirstlane(gsel);
            task_t[j] = __builtin_amdgcn_readfirstlane(k);
            const int cbw = sreg(d.grid[task_g[j]].cb_w), ncell = sreg(d.grid[task_g[j]].ncell);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int cell = 16 * task_t[j] + 4 * r + grp;
                const int cy = cbw > 0 ? cell / cbw : 0;
                const uint32_t e = cell < ncell ? (uint32_t)(cell - cy * cbw) | ((uint32_t)cy << 8) : 0xFFFFu;
                task_cell[j][r >> 1] |= e << (16 * (r & 1));
            }
        }
    }

    f16v dwacc[LY::slots];
#pragma unroll
    for (int j = 0; j < LY::slots; ++j)
        dwacc[j] = (f16v)0.f;
    float dbt[LY::slots]; // bias-gradient partial of the owned tile (a, 0): feature 32a + c
#pragma unroll
    for (int j = 0; j < LY::slots; ++j)
        dbt[j] = 0.f;
    const int col = 32 * wave + c; // this lane's sample column in the group's transposes

    // Tiles of the region, several per workgroup when there are more tiles than workgroups;
    // the MLP gradient accumulates over all of them.
    int gq = 0; // chunks done: the gather-box buffer of this one is gq & 1
    for (int b0 = blockIdx.x; b0 < d.ntiles; b0 += gridDim.x) {
    int tx0, ty0;
    const int b = tile_origin(b0, tx0, ty0);
    // Scatter boxes (the 3-channel network's fine grids; the planner places none for 16
    // channels): cleared here (the previous tile's flush ended with a barrier, and the
    // chunk's barriers order this before the first add); box origin of the lane's grids.
    int box_ox[G / 2], box_oy[G / 2];
    if constexpr (C == 3) {
        for (int i = tid; i < d.box_floats; i += kTrainThreads * NG)
            sbox[i] = 0.f;
#pragma unroll
        for (int j = 0; j < G / 2; ++j) {
            box_ox[j] = (int)floorf(fmaf((float)(d.off_x + tx0), own[j].rx, -0.5f)) - 1;
            box_oy[j] = (int)floorf(fmaf((float)(d.off_y + ty0), own[j].ry, -0.5f)) - 1;
        }
    }

    for (int chunk = 0; chunk < 4; ++chunk) {
        const int cx0 = d.off_x + tx0 + chunk * kChunkW, cy0 = d.off_y + ty0 + kChunkH * gr;
        // With gather boxes both copies are untracked: the gather's LDS reads (another buffer)
        // then wait for neither.
        if constexpr (GBOX)
            tile_fetch_async<true>(d, tile, cx0, cy0, wave, lane);
        else if constexpr (!RND)
            tile_fetch_async(d, tile, cx0, cy0, wave, lane);
        const float4 *gcur = gbox + (gq & 1) * gbox_step;

        // ---- sample position (train.cu:827-844)
        const int sx = tx0 + chunk * kChunkW + (c & 15);
        const int sy = ty0 + kChunkH * gr + 2 * wave + (c >> 4);
        uint32_t sidx = (uint32_t)sy * (uint32_t)d.region_w + (uint32_t)sx;
        bool valid = sx < d.region_w && sidx < (uint32_t)d.num_samples;
        if constexpr (RND) {
            // Slot 512 (NG b + gr) + 128 chunk + 32 wave + c: tiles of consecutive slots; with
            // ORD each holds the sample the bin-sorted order gives it, else slot i is sample i.
            sidx = (((((uint32_t)b * NG + (uint32_t)gr) * 4u + (uint32_t)chunk) * 4u + (uint32_t)wave) * 32u) +
                   (uint32_t)c;
            valid = sidx < (uint32_t)d.num_samples;
            if constexpr (ORD) {
                if (valid)
                    sidx = d.order[sidx];
            }
        }
        uint32_t st = mix_seed(sidx, d.step);
        uint32_t tx = (uint32_t)(d.off_x + sx), ty = (uint32_t)(d.off_y + sy);
        if constexpr (RND) // a uniformly random texel of the image, then the jitter
            random_texel(st, d.image_w, d.image_h, tx, ty);
        const float jx = uniform01(st) - 0.5f;
        const float jy = uniform01(st) - 0.5f;
        const float px = clampf((float)tx + 0.5f + jx, 0.5f, (float)d.image_w - 0.5f);
        const float py = clampf((float)ty + 0.5f + jy, 0.5f, (float)d.image_h - 0.5f);
        const float u = div_pow2(px, (float)d.image_w, d.inv_w);
        const float v = div_pow2(py, (float)d.image_h, d.inv_h);
        // One group (registers to spare) issues the taps here, so that their latency overlaps
        // the gathers and the MLP; two groups issue them before use and hide the latency with
        // the other group's wave.
        LaneTaps taps;
        if constexpr (RND && PF)
            issue_taps(d, u, v, g, taps);

        h8 x0[KQ0];
        if (valid) {
            if constexpr (GBOX) {
                if (d.gbox_off != 0)
                    gather16_box<G>(d, gcur, own, cx0, cy0, u, v, g, x0);
                else
                    gather16<G, PF>(d, u, v, g, x0);
            } else if constexpr (C == 16)
                gather16<G, PF>(d, u, v, g, x0);
            else
                gather3(d, u, v, g, x0);
        } else {
#pragma unroll
            for (int q = 0; q < KQ0; ++q)
                x0[q] = (h8)(_Float16)0.f;
        }

        // The next chunk's gather boxes (this tile's next chunk or the next tile's first),
        // issued once this chunk's gather is done; complete with the target tile at the
        // barrier before the targets.
        if constexpr (GBOX) {
            if (d.gbox_off != 0) {
                float4 *gnext = gbox + ((gq + 1) & 1) * gbox_step;
                if (chunk < 3) {
                    gbox_fetch_async(gl, gnext, cx0 + kChunkW, cy0, wave);
                } else if (b0 + (int)gridDim.x < d.ntiles) {
                    int nx0, ny0;
                    tile_origin(b0 + gridDim.x, nx0, ny0);
                    gbox_fetch_async(gl, gnext, d.off_x + nx0, d.off_y + ny0, wave);
                }
            }
        }

        // ---- forward (mlp.h:65-99)
        h8 xh[NH][HQ];
        {
            f16v acc[HA];
            layer_forward<KQ0, HA, PFM>(frags + S::fwd_off(0) * kWave, bias + S::bias_off(0), x0, acc, lane);
            to_fragments<HQ, HA, true>(acc, xh[0]);
#pragma unroll
            for (int l = 1; l < NH; ++l) {
                layer_forward<HQ, HA, PFM>(frags + S::fwd_off(l) * kWave, bias + S::bias_off(l), xh[l - 1], acc, lane);
                to_fragments<HQ, HA, true>(acc, xh[l]);
            }
        }
        f16v out[1];
        layer_forward<HQ, 1, PFM>(frags + S::fwd_off(L - 1) * kWave, bias + S::bias_off(L - 1), xh[NH - 1], out, lane);

        if constexpr (!RND)
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // Target tile staged; the previous chunk's scatter has read the union.
        __syncthreads();

        // ---- targets and loss gradient (train.cu:105-157, 876-888): dL/dy = fp16(2 w (y - t) / N)
        h8 dyo[1];
        {
            float tgt[8], tw[8];
            if constexpr (RND && PF)
                taps_targets(d, taps, g, tgt, tw);
            else if constexpr (RND)
                taps_targets_late(d, u, v, g, tgt, tw);
            else
                lane_targets16<PF>(d, tile, cx0, cy0, u, v, g, tgt, tw);
            float grd[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float y = (float)(_Float16)out[0][e];
                grd[e] = 2.f * tw[e] * (y - tgt[e]);
            }
            // One uniform branch: the product with the exact reciprocal of a power-of-two N,
            // else the quotient.
            if (d.inv_samples != 0.f) {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    grd[e] *= d.inv_samples;
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    grd[e] /= (float)d.num_samples;
            }
#pragma unroll
            for (int e = 0; e < 8; ++e)
                dyo[0][e] = valid ? (_Float16)grd[e] : (_Float16)0.f;
        }

        // ---- backward, last layer (mlp.h:302-362)
        h8 dyh[HQ];
        store_rows<1>(dys, dyo, col, g);
        store_rows<HQ>(xs, xh[NH - 1], col, g);
        {
            f16v acc[HA];
            layer_backward_dx<1, HA, PFM>(frags + S::bwd_off(L - 1) * kWave, dyo, acc, lane);
            relu_backward<HQ, HA>(acc, xh[NH - 1], dyh);
        }
        __syncthreads();
        dw_rows<S, L - 1, PFM>(xs, dys, dwacc, dbt, wave, lane);
        __syncthreads();

        // ---- hidden layers L-2 .. 1
        backward_hidden_rows<S, L - 2, PFM>(xs, dys, frags, xh, dyh, dwacc, dbt, col, wave, lane);

        // ---- first layer: dW with the gathered inputs, dX = latent gradient
        store_rows<HQ>(dys, dyh, col, g);
        store_input_rows<C, KQ0>(xs, x0, col, g);
        h8 dx0[KQ0];
        {
            constexpr int MA = S::t32(S::K0);
            f16v acc[MA];
            layer_backward_dx<HQ, MA, PFM>(frags + S::bwd_off(0) * kWave, dyh, acc, lane);
#pragma unroll
            for (int q = 0; q < KQ0; ++q) {
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const f2 pv = {acc[q >> 1][8 * (q & 1) + e], acc[q >> 1][8 * (q & 1) + e + 1]};
                    const h2 hv = __builtin_convertvector(pv, h2);
                    dx0[q][e] = hv[0];
                    dx0[q][e + 1] = hv[1];
                }
            }
        }
        __syncthreads();
        dw_rows<S, 0, PFM>(xs, dys, dwacc, dbt, wave, lane);
        __syncthreads();

        // ---- latent scatter (train.cu:460-509) as an MFMA reduction over the chunk
        // Part 1: dX0 rows; the sample's weight rows are cleared, then lane group g fills the
        // entries of grids g, g + 2 for its sample. A footprint not wholly inside the chunk
        // cell box (not expected: the box covers every corner a chunk position can reach, up
        // to fp32 rounding) goes straight to global memory, all C channels read back from
        // the dX0 row.
        store_rows<KQ0, dx_stride(S::K0)>(dxs, dx0, col, g);
        if constexpr (RND) {
            // Random texels: no two samples of a chunk are expected to share a texel, so each
            // sample's corners go straight to the gradients (train.cu:460-509's per-sample
            // atomics). The wave's lanes record each (sample, grid) corner's texel and weight
            // in the wave's own LDS slots, then walk the wave's 32 samples with lane =
            // 16 corner + channel: each atomic instruction adds four whole 64-byte texel
            // records. Only the wave's own rows and slots are read, so no barrier.
            int2 *slots = (int2 *)(dxs + kChunk * dx_stride(S::K0)) + wave * (32 * G * 4);
#pragma unroll
            for (int j = 0; j < G / 2; ++j) {
                const int gi = 2 * j + g, w = own[j].w, h = own[j].h;
                const Footprint f = footprint16(w, h, u, v);
#pragma unroll
                for (int corner = 0; corner < 4; ++corner) {
                    const int tx = wrap_near(f.x0 + (corner & 1), w), ty = wrap_near(f.y0 + (corner >> 1), h);
                    slots[(c * G + gi) * 4 + corner] = make_int2(valid ? ty * w + tx : -1, __float_as_int(f.w[corner]));
                }
            }
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const int corner = lane >> 4, ch = lane & 15;
            float *gptr[G];
#pragma unroll
            for (int gi = 0; gi < G; ++gi)
                gptr[gi] = sreg(d.grid[gi].grads);
#pragma unroll 2
            for (int s0 = 0; s0 < 32; s0 += 4) {
                int2 sl[4][G];
                float gv[4][G];
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int gi = 0; gi < G; ++gi) {
                        sl[s][gi] = slots[((s0 + s) * G + gi) * 4 + corner];
                        gv[s][gi] = (float)dxs[(32 * wave + s0 + s) * dx_stride(S::K0) + 16 * gi + ch];
                    }
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int gi = 0; gi < G; ++gi)
                        if (sl[s][gi].x >= 0 && gv[s][gi] != 0.f)
                            global_add(gptr[gi] + (uint32_t)sl[s][gi].x * 16u + (uint32_t)ch,
                                       __int_as_float(sl[s][gi].y) * gv[s][gi]);
            }
        } else {
        {
            _Float16 *rhi = whi + col * d.wcols, *rlo = wlo + col * d.wcols;
            {
                // The sample's two weight rows are cleared (their task columns; the
                // padding is never read), one by each lane group (hi by group 0, lo by
                // group 1): a uniform loop of 16-byte stores, ahead of the corner stores of
                // both groups in program order.
                uint4 *z = (uint4 *)(g ? rlo : rhi);
                const int n16 = d.wclear;
#pragma unroll 4
                for (int k = 0; k < n16; ++k)
                    z[k] = make_uint4(0u, 0u, 0u, 0u);
            }
#pragma unroll
            for (int j = 0; j < G / 2; ++j) {
                const int gi = 2 * j + g;
                const int w = own[j].w, h = own[j].h, cb_w = own[j].cb_w, cb_h = own[j].cb_h;
                const int wcol0 = own[j].wcol0;
                const float rx = own[j].rx, ry = own[j].ry;
                const int bx = (int)floorf(fmaf((float)cx0, rx, -0.5f));
                const int by = (int)floorf(fmaf((float)cy0, ry, -0.5f));
                const Footprint f = footprint16(w, h, u, v);
                const int cx = f.x0 - bx, cy = f.y0 - by;
                const bool inside = cx >= 0 && cx + 1 < cb_w && cy >= 0 && cy + 1 < cb_h;
                bool recorded = false;
                if constexpr (C == 3) {
                    if (own[j].slot_off >= 0) {
                        // The sample's record for the gather below (every sample of the chunk
                        // has one). Texel x of a grid of 1/k the image's size gathers from the
                        // positions [kx - c0, kx - c0 + nc) (gather_records); a footprint is
                        // regular when both of its texel columns (and rows) have the sample's
                        // position in their windows, which holds for every position but one
                        // clamped to the image edge (a region running past the image) or one
                        // on a texel edge whose fp32 arithmetic rounds across it. A position
                        // past the region, or an irregular one, records a zero gradient; an
                        // irregular one takes the per-sample path.
                        const int k = own[j].gk, c0 = (k + 1) >> 1, nc = ((3 * k + 1) >> 1) + c0;
                        const int ex = d.off_x + sx - (k * f.x0 - c0), ey = d.off_y + sy - (k * f.y0 - c0);
                        const bool regular = ex >= k && ex < nc && ey >= k && ey < nc;
                        const bool on = valid && regular;
                        uint4 *rec = (uint4 *)(sbox + own[j].slot_off) + gr * kChunk + col;
                        const float fx = fmaf(u, (float)w, -0.5f) - (float)f.x0;
                        const float fy = fmaf(v, (float)h, -0.5f) - (float)f.y0;
                        // The grid's three input gradients from the sample's dX0 row (natural
                        // feature order; this wave stored it above).
                        const _Float16 *gx = dxs + col * dx_stride(S::K0) + C * gi;
                        const uint32_t g0 = on ? h_bits(gx[0]) : 0u, g1 = on ? h_bits(gx[1]) : 0u;
                        const uint32_t g2 = on ? h_bits(gx[2]) : 0u;
                        // Box offsets of a regular footprint: 1 .. box size - 2 (< 256).
                        const uint32_t rel = on ? (uint32_t)(f.x0 - box_ox[j]) | ((uint32_t)(f.y0 - box_oy[j]) << 8) : 0u;
                        *rec = make_uint4(__float_as_uint(fx), __float_as_uint(fy), g0 | (g1 << 16), g2 | (rel << 16));
                        recorded = regular || !valid;
                    }
                }
                if (recorded) {
                } else if (valid && inside) {
#pragma unroll
                    for (int corner = 0; corner < 4; ++corner) {
                        const int k = wcol0 + cell_column((cy + (corner >> 1)) * cb_w + cx + (corner & 1));
                        const _Float16 hi = (_Float16)f.w[corner];
                        rhi[k] = hi;
                        rlo[k] = (_Float16)(f.w[corner] - (float)hi);
                    }
                } else if (valid) {
                    float *grads = own[j].grads;
                    if constexpr (C == 3) {
                        // Per-sample adds (a grid without a cell box, or a footprint outside
                        // it): the sample's three input gradients of the grid read once, every
                        // corner's place computed (the tile's scatter box, else global
                        // memory), then the adds without waits in between.
                        float gv[C];
#pragma unroll
                        for (int ch = 0; ch < C; ++ch)
                            gv[ch] = (float)dxs[col * dx_stride(S::K0) + C * gi + ch];
                        uint32_t tex[4];
                        int bx[4];
#pragma unroll
                        for (int corner = 0; corner < 4; ++corner) {
                            const int tx = wrap_near(f.x0 + (corner & 1), w), ty = wrap_near(f.y0 + (corner >> 1), h);
                            tex[corner] = (uint32_t)(ty * w + tx) * (uint32_t)C;
                            const int lx = f.x0 + (corner & 1) - box_ox[j], ly = f.y0 + (corner >> 1) - box_oy[j];
                            bx[corner] = lx >= 0 && lx < own[j].box_w && ly >= 0 && ly < own[j].box_h
                                             ? own[j].box_off + (ly * own[j].box_w + lx) * C
                                             : -1;
                        }
#pragma unroll
                        for (int corner = 0; corner < 4; ++corner)
#pragma unroll
                            for (int ch = 0; ch < C; ++ch)
                                if (gv[ch] != 0.f) {
                                    if (bx[corner] >= 0)
                                        lds_add(sbox + bx[corner] + ch, f.w[corner] * gv[ch]);
                                    else
                                        global_add(grads + tex[corner] + ch, f.w[corner] * gv[ch]);
                                }
                    } else {
                        // 16 channels: a compact loop (this path is not expected; the cell box
                        // covers every footprint, and the kernel's code size matters more).
                        for (int corner = 0; corner < 4; ++corner) {
                            const int tx = wrap_near(f.x0 + (corner & 1), w), ty = wrap_near(f.y0 + (corner >> 1), h);
                            for (int ch = 0; ch < C; ++ch) {
                                const float val = f.w[corner] * (float)dxs[col * dx_stride(S::K0) + C * gi + ch];
                                global_add(grads + ((int64_t)ty * w + tx) * C + ch, val);
                            }
                        }
                    }
                }
            }
        }
        __syncthreads();
        if constexpr (C == 3) {
            // Grids of the image's size: each texel of the chunk pair's footprint (18 x
            // (8NG + 2) texels: the groups' chunks side by side in y) sums the corners the
            // records of the samples at positions x - 1 .. x + 1, y - 1 .. y + 1 put on it
            // (no other sample's footprint reaches it), and adds the sums to its box texel.
            // One thread per texel and the chunk pairs in sequence: plain adds.
            if (d.gather_grids > 0)
                gather_records<NG>(d, sbox, d.off_x + tx0 + chunk * kChunkW, d.off_y + ty0, tx0, ty0, tid);
        }
        // Part 2: one task per (grid, 16-cell tile), this wave's two (above). A wave takes
        // its tasks two at a time with their LDS reads and MFMAs interleaved (the 4-grid
        // network has five tasks: one wave runs two, and their latencies overlap).
        {
            int total = ntask;
            if constexpr (!PF) {
                total = 0;
#pragma unroll
                for (int gi = 0; gi < G; ++gi)
                    total += (d.grid[gi].ncell + 15) >> 4;
            }
            const int i16 = lane & 15, grp = lane >> 4;
            // One pass with at most eight tasks (the planner's bound); two groups keep the
            // general loop.
            for (int k0 = wave; k0 < total; k0 += PF ? total : 8) {
                int tg[2] = {task_g[0], task_g[1]}, tt[2] = {task_t[0], task_t[1]};
                if constexpr (!PF) {
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        int k = k0 + 4 * j, gsel = 0;
#pragma unroll
                        for (int gi = 0; gi + 1 < G; ++gi) {
                            const int n = (d.grid[gi].ncell + 15) >> 4;
                            if (gsel == gi && k >= n) {
                                k -= n;
                                gsel = gi + 1;
                            }
                        }
                        tg[j] = __builtin_amdgcn_readfirstlane(gsel);
                        tt[j] = __builtin_amdgcn_readfirstlane(k);
                    }
                }
                const bool two = k0 + 4 < total;
                f4v acc[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
                if constexpr (PF) {
                    // every operand of both tasks first, then the MFMAs
                    constexpr int KS = kChunk / 32;
                    h8 bv[2][KS], wh[2][KS], wl[2][KS];
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (j == 1 && !two)
                            break;
                        const int acol = d.grid[tg[j]].wcol0 + 16 * tt[j] + 4 * (i16 & 3);
#pragma unroll
                        for (int kk = 0; kk < KS; ++kk) {
                            const int arow = 32 * kk + 8 * grp + (i16 >> 2);
                            bv[j][kk] = read_cols8<dx_stride(S::K0)>(dxs, 32 * kk + 8 * grp, dx_col0<C>(tg[j]), i16);
                            const h4 h0 = lds_read_tr16(whi + arow * d.wcols + acol);
                            const h4 h1 = lds_read_tr16(whi + (arow + 4) * d.wcols + acol);
                            const h4 l0 = lds_read_tr16(wlo + arow * d.wcols + acol);
                            const h4 l1 = lds_read_tr16(wlo + (arow + 4) * d.wcols + acol);
                            wh[j][kk] = __builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7);
                            wl[j][kk] = __builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7);
                        }
                    }
#pragma unroll
                    for (int kk = 0; kk < KS; ++kk)
#pragma unroll
                        for (int j = 0; j < 2; ++j) {
                            if (j == 1 && !two)
                                break;
                            acc[j] = mfma16(wh[j][kk], bv[j][kk], acc[j]);
                            acc[j] = mfma16(wl[j][kk], bv[j][kk], acc[j]);
                        }
                } else {
#pragma unroll
                for (int kk = 0; kk < kChunk / 32; ++kk) {
                    const int arow = 32 * kk + 8 * grp + (i16 >> 2);
#pragma unroll
                    for (int j = 0; j < 2; ++j) {
                        if (j == 1 && !two)
                            break;
                        const int acol = d.grid[tg[j]].wcol0 + 16 * tt[j] + 4 * (i16 & 3);
                        const h8 bv = read_cols8<dx_stride(S::K0)>(dxs, 32 * kk + 8 * grp, dx_col0<C>(tg[j]), i16);
                        const h4 h0 = lds_read_tr16(whi + arow * d.wcols + acol);
                        const h4 h1 = lds_read_tr16(whi + (arow + 4) * d.wcols + acol);
                        const h4 l0 = lds_read_tr16(wlo + arow * d.wcols + acol);
                        const h4 l1 = lds_read_tr16(wlo + (arow + 4) * d.wcols + acol);
                        acc[j] = mfma16(__builtin_shufflevector(h0, h1, 0, 1, 2, 3, 4, 5, 6, 7), bv, acc[j]);
                        acc[j] = mfma16(__builtin_shufflevector(l0, l1, 0, 1, 2, 3, 4, 5, 6, 7), bv, acc[j]);
                    }
                }
                }
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    if (j == 1 && !two)
                        break;
                    // The task's grid fields once, every address before any atomic (no
                    // reloads of the fields inside the guarded stores).
                    const Grid16 &q = d.grid[tg[j]];
                    const int w = sreg(q.w), h = sreg(q.h), cbw = sreg(q.cb_w), cbh = sreg(q.cb_h);
                    const int ncell = sreg(q.ncell);
                    const float icbw = sreg(q.inv_cb_w);
                    float *grads = sreg(q.grads);
                    const int bx = (int)floorf(fmaf((float)cx0, sreg(q.rx), -0.5f));
                    const int by = (int)floorf(fmaf((float)cy0, sreg(q.ry), -0.5f));
                    uint32_t off[4];
                    bool ok[4];
                    // D column i16 is dX0 feature dx_col0(grid) + i16, channel cl of this grid.
                    const int cl = i16 - (C * tg[j] - dx_col0<C>(tg[j]));
                    if constexpr (PF) {
                        // The lane's cells from the launch's table; a cell box wholly inside
                        // the grid (the chunk is not at a wrapping edge) needs no wrap.
                        const bool inside = bx >= 0 && by >= 0 && bx + cbw <= w && by + cbh <= h;
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            // D row 4grp + r: cell 16t + 4r + grp
                            const uint32_t e = task_cell[j][r >> 1] >> (16 * (r & 1));
                            int tx = bx + (int)(e & 0xFFu), ty = by + (int)((e >> 8) & 0xFFu);
                            if (!inside) {
                                tx = wrap_near(tx, w);
                                ty = wrap_near(ty, h);
                            }
                            off[r] = __umul24((uint32_t)ty, (uint32_t)w) * (uint32_t)C + (uint32_t)(tx * C + cl);
                            ok[r] = (e & 0xFFFFu) != 0xFFFFu && (C == 16 || (unsigned)cl < (unsigned)C) && acc[j][r] != 0.f;
                        }
                    } else {
#pragma unroll
                        for (int r = 0; r < 4; ++r) {
                            const int cell = 16 * tt[j] + 4 * r + grp; // D row 4grp + r holds column 16t + 4grp + r
                            const int cy = (int)(((float)cell + 0.5f) * icbw);
                            const int cxx = cell - cy * cbw;
                            const int tx = wrap_near(bx + cxx, w), ty = wrap_near(by + cy, h);
                            off[r] = (uint32_t)(ty * w + tx) * (uint32_t)C + (uint32_t)cl;
                            ok[r] = cell < ncell && (C == 16 || (unsigned)cl < (unsigned)C) && acc[j][r] != 0.f;
                        }
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (ok[r])
                            global_add(grads + off[r], acc[j][r]);
                }
            }
        }
        } // region scatter
        // The next chunk writes the union only after its first barrier.
        ++gq;
    }

    // Flush the tile's scatter boxes: grid by grid, the non-zero sums added to the
    // gradients once (wrapped like the corners they hold).
    if (C == 3 && d.box_floats > 0) {
        __syncthreads();
#pragma unroll
        for (int gi = 0; gi < G; ++gi) {
            const Grid16 &q = d.grid[gi];
            const int bw = q.box_w, n = bw * q.box_h * C;
            const int w = q.w, h = q.h;
            const int ox = (int)floorf(fmaf((float)(d.off_x + tx0), q.rx, -0.5f)) - 1;
            const int oy = (int)floorf(fmaf((float)(d.off_y + ty0), q.ry, -0.5f)) - 1;
            for (int i = tid; i < n; i += kTrainThreads * NG) {
                const float v = sbox[q.box_off + i];
                if (v == 0.f)
                    continue;
                const int cell = i / C, ch = i - cell * C;
                const int ly = cell / bw, lx = cell - ly * bw;
                const int tx = wrap_near(ox + lx, w), ty = wrap_near(oy + ly, h);
                global_add(q.grads + (uint32_t)(ty * w + tx) * (uint32_t)C + ch, v);
            }
        }
        __syncthreads();
    }

    } // tiles
    __syncthreads(); // group 1's last scatter reads are done before its region is reused below

    // ---- the workgroup's MLP gradient partial (output rows of the last layer un-permuted):
    // group 1 hands its accumulators to group 0 through its own (now idle) LDS region, then
    // the owner of the second half of a split dW tile hands it to the owner of the first
    // half through group 0's region. Every wave takes part in every barrier.
    if constexpr (NG == 2) {
        // In rounds of HS slots (17 floats per slot and thread), as many as group 1's region
        // holds.
        constexpr int HS = handoff_slots<S>();
        float *xch = (float *)(smem + d.group_off + d.group_bytes);
#pragma unroll
        for (int r0 = 0; r0 < LY::slots; r0 += HS) {
            if (r0 > 0)
                __syncthreads(); // group 0 has read the previous round
            if (gr == 1) {
#pragma unroll
                for (int j = r0; j < r0 + HS && j < LY::slots; ++j) {
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        xch[((j - r0) * 17 + e) * kTrainThreads + t256] = dwacc[j][e];
                    xch[((j - r0) * 17 + 16) * kTrainThreads + t256] = dbt[j];
                }
            }
            __syncthreads();
            if (gr == 0) {
#pragma unroll
                for (int j = r0; j < r0 + HS && j < LY::slots; ++j) {
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        dwacc[j][e] += xch[((j - r0) * 17 + e) * kTrainThreads + t256];
                    dbt[j] += xch[((j - r0) * 17 + 16) * kTrainThreads + t256];
                }
            }
        }
    }
    float *xfer = (float *)(smem + d.group_off); // [split tile][17][64 lanes]
    float *part = d.partial + (int64_t)blockIdx.x * S::grad_total();
#pragma unroll
    for (int pass = 0; pass < 2; ++pass) {
        if (pass == 1)
            __syncthreads();
#pragma unroll
        for (int j = 0; j < LY::slots; ++j) {
#pragma unroll
            for (int l = 0; l < L; ++l) {
                const int it = 4 * j + wave - LY::item_start(l);
                if (gr != 0 || it < 0 || it >= LY::items(l))
                    continue;
                const bool split = LY::split(l);
                const int t = split ? it >> 1 : it;
                float *x = xfer + (LY::split_start(l) + t) * 17 * kWave + lane;
                if (pass == 0) {
                    // second halves of split tiles: to the merge buffer
                    if (split && (it & 1)) {
#pragma unroll
                        for (int e = 0; e < 16; ++e)
                            x[e * kWave] = dwacc[j][e];
                        x[16 * kWave] = dbt[j];
                    }
                    continue;
                }
                if (split && (it & 1))
                    continue;
                f16v acc = dwacc[j];
                float dbj = dbt[j];
                if (split) {
#pragma unroll
                    for (int e = 0; e < 16; ++e)
                        acc[e] += x[e * kWave];
                    dbj += x[16 * kWave];
                }
                const int kin = S::kin(l), kout = S::kout(l), off = S::grad_off(l), kb = S::t32(S::kin(l));
                const int a = t / kb, bb = t % kb;
#pragma unroll
                for (int e = 0; e < 16; ++e) {
                    const int row = 32 * a + 8 * (e >> 2) + 4 * g + (e & 3);
                    const int k = 32 * bb + c;
                    if (row < kout && k < kin) {
                        const int n = l == L - 1 ? perm_row(d.perm, row) : row;
                        part[off + n * kin + k] = acc[e];
                    }
                }
                // Tile (a, 0) carries the bias gradient of rows 32a + c: lane groups 0 and 1
                // summed disjoint halves of every sample block.
                const float db = dbj + __shfl_xor(dbj, 32);
                if (bb == 0 && g == 0 && 32 * a + c < kout) {
                    const int row = 32 * a + c;
                    const int n = l == L - 1 ? perm_row(d.perm, row) : row;
                    part[off + kout * kin + n] = db;
                }
            }
        }
    }
}

// ---- launchers ---------------------------------------------------------------------------

using ShapeRef = Shape<16, 32, 2>;
using ShapeC2 = Shape<32, 64, 2>;
using ShapeC4 = Shape<64, 64, 3>;

template <class S, int C, int NG, bool RND, bool ORD = false>
static hipError_t launch16(const Train16Desc &d, size_t lds, hipStream_t s)
{
    auto k = train16_kernel<S, C, NG, RND, ORD>;
    // Raise the kernel's dynamic LDS limit to the whole 160 KB once (thread-safe).
    static std::once_flag once;
    static hipError_t configured = hipSuccess;
    std::call_once(once, [&] {
        configured = hipFuncSetAttribute((const void *)k, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
    });
    if (lds > 65536 && configured != hipSuccess)
        return configured;
    hipLaunchKernelGGL(k, dim3(d.nwg), dim3(kTrainThreads * NG), lds, s, d);
    return hipGetLastError();
}

// This file is compiled twice: once for the region kernels and the host functions below,
// and once with NT_TRAIN16_RANDOM_UNIT for the random-texel kernels alone, under the
// scheduler that groups memory instructions into clauses
// (-amdgpu-sched-strategy=max-memory-clause): the random-texel kernels wait on their
// gathers, taps and atomics, and that schedule runs the config-2 one 4 % faster (214 -> 205
// us in alternating runs) while the region kernels run as fast or slower with it.
#ifdef NT_TRAIN16_RANDOM_UNIT
hipError_t launch_train16_random(int shape, const Train16Desc &d, size_t lds, hipStream_t s)
{
    switch (shape) {
    case kShapeC2:
        return d.order ? launch16<ShapeC2, 16, 2, true, true>(d, lds, s) : launch16<ShapeC2, 16, 2, true>(d, lds, s);
    case kShapeC4:
        return d.order ? launch16<ShapeC4, 16, 2, true, true>(d, lds, s) : launch16<ShapeC4, 16, 2, true>(d, lds, s);
    default:
        return hipErrorInvalidValue;
    }
}
#else
int train16_groups(int shape, bool random_texels)
{
    if (random_texels)
        return shape == kShapeC2 || shape == kShapeC4 ? 2 : 0;
    return shape == kShapeRef || shape == kShapeC2 ? 2 : shape == kShapeC4 ? 1 : 0;
}

size_t train16_head_bytes(int shape)
{
    switch (shape) {
    case kShapeRef:
        return T16Layout<ShapeRef, 2>::head_bytes;
    case kShapeC2:
        return T16Layout<ShapeC2, 2>::head_bytes;
    case kShapeC4:
        return T16Layout<ShapeC4, 1>::head_bytes;
    default:
        return 0;
    }
}

int train16_slots(int shape)
{
    switch (shape) {
    case kShapeRef:
        return handoff_slots<ShapeRef>();
    case kShapeC2:
        return handoff_slots<ShapeC2>();
    case kShapeC4:
        return handoff_slots<ShapeC4>();
    default:
        return 0;
    }
}

size_t train16_raw_bytes(int shape)
{
    switch (shape) {
    case kShapeRef:
        return raw_off<ShapeRef>(ShapeRef::L) * 2;
    case kShapeC2:
        return raw_off<ShapeC2>(ShapeC2::L) * 2;
    case kShapeC4:
        return raw_off<ShapeC4>(ShapeC4::L) * 2;
    default:
        return 0;
    }
}

size_t train16_transpose_bytes(int shape)
{
    // Layer inputs and output gradients as sample rows.
    return shape == kShapeRef || shape == kShapeC2 || shape == kShapeC4 ? 2 * kChunk * kFeatStride * 2 : 0;
}

hipError_t launch_train16(int shape, const Train16Desc &d, size_t lds, hipStream_t s)
{
    switch (shape) {
    case kShapeRef:
        return d.random_texels ? hipErrorInvalidValue : launch16<ShapeRef, 3, 2, false>(d, lds, s);
    case kShapeC2:
        return d.random_texels ? launch_train16_random(shape, d, lds, s)
                               : launch16<ShapeC2, 16, 2, false>(d, lds, s);
    case kShapeC4:
        return d.random_texels ? launch_train16_random(shape, d, lds, s)
                               : launch16<ShapeC4, 16, 1, false>(d, lds, s);
    default:
        return hipErrorInvalidValue;
    }
}
#endif

} // namespace ntk
