// nt_forward.hip — forward-only passes on gfx950: the tiny-MLP forward
// (mlp.h:18-99, the path tests/forward_pass_test.cu exercises), latent sample + MLP at
// given coordinates, full-image inference (train.cu:917-961) and decode from
// codec-quantized latents.
//
// Each wave runs 32-sample MFMA tiles in a grid-stride loop; forward weight fragments are
// staged in LDS once per workgroup. Lane group g of sample c (lane = 32g + c) gathers the
// network-input features 16q + 8g + e and ends with output rows o = chained_feature(0,g,e).
#include "nt_internal.hpp"

namespace ntk {


template <class S>
struct FwdLayout {
    static constexpr int frag_bytes = S::fwd_total() * kWave * 16;
    static constexpr int bias_off = frag_bytes;
    static constexpr int bytes = frag_bytes + ((S::bias_total() * 4 + 15) / 16) * 16;
};

// Corner coordinate wrap for positions clamped into the image: every bilinear corner lies
// in [-1, size], so one compare per side replaces the modulo of wrap_coord.
__device__ __forceinline__ int wrap_edge(int c, int size)
{
    return c < 0 ? c + size : (c >= size ? c - size : c);
}

// Mip pair for mip coordinate z (train.cu:266-281).
__device__ __forceinline__ int mip_pair(int num_mips, float z, int (&mips)[2], float (&w)[2])
{
    const float fz = floorf(z);
    const int base = (int)fz;
    const float frac = z - fz;
    const int max_mip = num_mips > 0 ? num_mips - 1 : 0;
    const int n = frac > 0.f ? 2 : 1;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        int m = base + i < max_mip ? base + i : max_mip;
        mips[i] = m < 0 ? 0 : m;
        w[i] = i ? frac : 1.f - frac;
    }
    return n;
}

// Trilinear unconstrained latent sample of the lane's natural-layout features
// (train.cu:263-314): fp16 rounding of every corner contribution, fp16 accumulation.
template <int C, int KQ>
__device__ __forceinline__ void sample_bilinear(const FwdDesc &d, float u, float v, float z, int g,
                                                h8 (&x)[KQ])
{
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[q][e] = (_Float16)0.f;
        if constexpr (C == 16 || C == 8) {
            const int gi = C == 16 ? q : 2 * q + g;
            if (gi >= d.G)
                continue;
            const GridDesc &gr = d.grid[C == 16 ? q : (g ? ((2 * q + 1) & 3) : 2 * q)];
            const int cb = C == 16 ? 8 * g : 0;
            int mips[2];
            float mw[2];
            const int nm = mip_pair(gr.num_mips, z, mips, mw);
            for (int mi = 0; mi < nm; ++mi) {
                const int w = mip_dim(gr.w, mips[mi]), h = mip_dim(gr.h, mips[mi]);
                const Footprint f = bilinear_footprint(u, v, w, h, mw[mi]);
                const float *vals = gr.values + gr.mip_off[mips[mi]] * C + cb;
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    const int tx = wrap_coord(f.x0 + (c & 1), w), ty = wrap_coord(f.y0 + (c >> 1), h);
                    const float4 *p = (const float4 *)(vals + ((int64_t)ty * w + tx) * C);
                    x[q] = accumulate_products(x[q], f.w[c], p[0], p[1]);
                }
            }
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int feat = 16 * q + 8 * g + e;
                if (feat >= d.G * C)
                    continue;
                const GridDesc &gr = d.grid[feat / C];
                const int ch = feat % C;
                int mips[2];
                float mw[2];
                const int nm = mip_pair(gr.num_mips, z, mips, mw);
                _Float16 a = (_Float16)0.f;
                for (int mi = 0; mi < nm; ++mi) {
                    const int w = mip_dim(gr.w, mips[mi]), h = mip_dim(gr.h, mips[mi]);
                    const Footprint f = bilinear_footprint(u, v, w, h, mw[mi]);
                    const float *vals = gr.values + gr.mip_off[mips[mi]] * C;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        const int tx = wrap_coord(f.x0 + (c & 1), w), ty = wrap_coord(f.y0 + (c >> 1), h);
                        a = a + half_of_product(f.w[c], vals[((int64_t)ty * w + tx) * C + ch]);
                    }
                }
                x[q][e] = a;
            }
        }
    }
}

// 16-tap Catmull-Rom latent sample on mip 0: fp32 accumulation, one fp16 rounding.
template <int C, int KQ>
__device__ __forceinline__ void sample_catmull_rom(const FwdDesc &d, float u, float v, int g,
                                                   h8 (&x)[KQ])
{
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
        float acc[8];
#pragma unroll
        for (int e = 0; e < 8; ++e)
            acc[e] = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int feat = 16 * q + 8 * g + e;
            if (feat >= d.G * C)
                continue;
            const GridDesc &gr = d.grid[feat / C];
            const int ch = feat % C;
            float wx[4], wy[4];
            const int x0 = cr_axis(u, gr.w, wx);
            const int y0 = cr_axis(v, gr.h, wy);
            const float *vals = gr.values + gr.mip_off[0] * C;
            for (int j = 0; j < 4; ++j) {
                const int ty = wrap_coord(y0 + j, gr.h);
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int tx = wrap_coord(x0 + i, gr.w);
                    acc[e] = fmaf(vals[((int64_t)ty * gr.w + tx) * C + ch], wx[i] * wy[j], acc[e]);
                }
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[q][e] = (_Float16)acc[e];
    }
}

// Trilinear sample of codec-quantized latents (C multiple of 8 per lane group).
template <int C, int KQ>
__device__ __forceinline__ void sample_codec(const FwdDesc &d, float u, float v, float z, int g,
                                             h8 (&x)[KQ])
{
    static_assert(C == 16 || C == 8, "codec decode expects 8 or 16 channels");
#pragma unroll
    for (int q = 0; q < KQ; ++q) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
            x[q][e] = (_Float16)0.f;
        const int gi = C == 16 ? q : 2 * q + g;
        if (gi >= d.G)
            continue;
        const CodecGrid &gr = d.cgrid[C == 16 ? q : (g ? ((2 * q + 1) & 3) : 2 * q)];
        const int cb = C == 16 ? 8 * g : 0;
        int mips[2];
        float mw[2];
        const int nm = mip_pair(gr.num_mips, z, mips, mw);
        for (int mi = 0; mi < nm; ++mi) {
            const int w = mip_dim(gr.w, mips[mi]), h = mip_dim(gr.h, mips[mi]);
            const int bw = (w + 3) >> 2;
            const Footprint f = bilinear_footprint(u, v, w, h, mw[mi]);
            const uint8_t *base = gr.blocks + gr.byte_off[mips[mi]];
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const int tx = wrap_edge(f.x0 + (c & 1), w), ty = wrap_edge(f.y0 + (c >> 1), h);
                const uint8_t *rec = base + ((int64_t)(ty >> 2) * bw + (tx >> 2)) * (12 * C);
                const int pix = ((ty & 3) << 2) + (tx & 3);
                const uint4 e01 = *(const uint4 *)(rec + 4 * cb);
                const uint4 e23 = *(const uint4 *)(rec + 4 * cb + 16);
                const uint32_t idx = *(const uint32_t *)(rec + 4 * C + pix * (C / 2) + cb / 2);
                const uint32_t ends[8] = {e01.x, e01.y, e01.z, e01.w, e23.x, e23.y, e23.z, e23.w};
                const float wc = f.w[c];
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const float val = codec_value(ends[e] & 0xFFFFu, ends[e] >> 16, (idx >> (4 * e)) & 15);
                    x[q][e] = x[q][e] + half_of_product(wc, val);
                }
            }
        }
    }
}

// ---- decode (16 channels per grid) ---------------------------------------------------
// Lane group g samples grids g and g + 2 (all 16 channels; the layer-0 weights are staged in
// grid_feature order), so each lane evaluates one footprint per grid and mip. A corner
// contribution is accumulated as one fp16 fma per channel, weight rounded to fp16
// (v_pk_fma_f16, two channels per instruction): within an fp16 rounding of the training
// path's fp32-product-then-round accumulation, which decode does not need to reproduce.
// Mip offsets come from a per-workgroup LDS table (the mip index differs per pixel).

__device__ __forceinline__ void fma_corner16(h8 &lo, h8 &hi, float w, h8 vlo, h8 vhi)
{
    const h8 w8 = (h8)(_Float16)w;
    lo = __builtin_elementwise_fma(w8, vlo, lo);
    hi = __builtin_elementwise_fma(w8, vhi, hi);
}

// The sixteen decoded fp16 channels of texel (tx, ty) of one codec mip level.
__device__ __forceinline__ void codec_texel16(const uint8_t *base, int bw, int tx, int ty, h8 &lo, h8 &hi)
{
    const uint8_t *rec = base + ((int64_t)(ty >> 2) * bw + (tx >> 2)) * (12 * 16);
    const int pix = ((ty & 3) << 2) + (tx & 3);
    const uint4 *r4 = (const uint4 *)rec;
    const uint4 e0 = load_global(r4), e1 = load_global(r4 + 1), e2 = load_global(r4 + 2), e3 = load_global(r4 + 3);
    const uint2 ix = load_global((const uint2 *)(rec + 64 + pix * 8));
    const uint32_t ends[16] = {e0.x, e0.y, e0.z, e0.w, e1.x, e1.y, e1.z, e1.w,
                               e2.x, e2.y, e2.z, e2.w, e3.x, e3.y, e3.z, e3.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        lo[e] = bits_h((uint16_t)codec_unkey(codec_interp(ends[e] & 0xFFFFu, ends[e] >> 16, (ix.x >> (4 * e)) & 15)));
        hi[e] = bits_h((uint16_t)codec_unkey(
            codec_interp(ends[8 + e] & 0xFFFFu, ends[8 + e] >> 16, (ix.y >> (4 * e)) & 15)));
    }
}

// EXPANDED: sample the fp16 texels of the first decode pass; else decode the blocks.
template <int G, bool EXPANDED>
__device__ __forceinline__ void sample_decode16(const FwdDesc &d, const int64_t *mip_tab, float u, float v,
                                                float z, int g, h8 (&x)[G])
{
#pragma unroll
    for (int j = 0; j < G / 2; ++j) {
        const int gi = 2 * j + g;
        const GridDesc &ga = d.grid[2 * j], &gb = d.grid[2 * j + 1];
        const int gw = g ? sreg(gb.w) : sreg(ga.w), gh = g ? sreg(gb.h) : sreg(ga.h);
        const int nmips = g ? sreg(gb.num_mips) : sreg(ga.num_mips);
        const uint16_t *hv = g ? sreg(d.half_values[2 * j + 1]) : sreg(d.half_values[2 * j]);
        const uint8_t *blocks = g ? sreg(d.cgrid[2 * j + 1].blocks) : sreg(d.cgrid[2 * j].blocks);
        int mips[2];
        float mw[2];
        const int nm = mip_pair(nmips, z, mips, mw);
        h8 lo = (h8)(_Float16)0.f, hi = (h8)(_Float16)0.f;
        for (int mi = 0; mi < nm; ++mi) {
            const int w = mip_dim(gw, mips[mi]), h = mip_dim(gh, mips[mi]);
            const Footprint f = bilinear_footprint(u, v, w, h, mw[mi]);
            const int x0 = wrap_edge(f.x0, w), x1 = wrap_edge(f.x0 + 1, w);
            const int y0 = wrap_edge(f.y0, h), y1 = wrap_edge(f.y0 + 1, h);
            const int64_t off = mip_tab[gi * NT_MAX_MIPS + mips[mi]];
            h8 v0l, v0h, v1l, v1h, v2l, v2h, v3l, v3h;
            if constexpr (EXPANDED) {
                const uint4 *t = (const uint4 *)(hv + off * 16);
                const uint4 a0 = load_global(t + 2 * (y0 * w + x0)), a1 = load_global(t + 2 * (y0 * w + x0) + 1);
                const uint4 b0 = load_global(t + 2 * (y0 * w + x1)), b1 = load_global(t + 2 * (y0 * w + x1) + 1);
                const uint4 c0 = load_global(t + 2 * (y1 * w + x0)), c1 = load_global(t + 2 * (y1 * w + x0) + 1);
                const uint4 e0 = load_global(t + 2 * (y1 * w + x1)), e1 = load_global(t + 2 * (y1 * w + x1) + 1);
                v0l = __builtin_bit_cast(h8, a0), v0h = __builtin_bit_cast(h8, a1);
                v1l = __builtin_bit_cast(h8, b0), v1h = __builtin_bit_cast(h8, b1);
                v2l = __builtin_bit_cast(h8, c0), v2h = __builtin_bit_cast(h8, c1);
                v3l = __builtin_bit_cast(h8, e0), v3h = __builtin_bit_cast(h8, e1);
            } else {
                const uint8_t *base = blocks + off;
                const int bw = (w + 3) >> 2;
                codec_texel16(base, bw, x0, y0, v0l, v0h);
                codec_texel16(base, bw, x1, y0, v1l, v1h);
                codec_texel16(base, bw, x0, y1, v2l, v2h);
                codec_texel16(base, bw, x1, y1, v3l, v3h);
            }
            fma_corner16(lo, hi, f.w[0], v0l, v0h);
            fma_corner16(lo, hi, f.w[1], v1l, v1h);
            fma_corner16(lo, hi, f.w[2], v2l, v2h);
            fma_corner16(lo, hi, f.w[3], v3l, v3h);
            // One mip level's eight 16-byte loads at a time keeps the wave within 128 VGPRs.
            __builtin_amdgcn_sched_barrier(0);
        }
        x[2 * j] = lo;
        x[2 * j + 1] = hi;
    }
}

// Decode keeps its per-tile state within 128 VGPRs, so it asks for four waves per SIMD
// (16 per CU) to hide the gather latency; the other modes keep the default.
template <int MODE>
constexpr int fwd_min_blocks() { return MODE == kFwdDecode || MODE == kFwdDecode16 ? 4 : 1; }

template <class S, int C, int MODE>
__global__ __launch_bounds__(kFwdThreads, fwd_min_blocks<MODE>()) void forward_kernel(FwdDesc d)
{
    using LY = FwdLayout<S>;
    constexpr int L = S::L, NH = S::NH, KQ0 = S::K0 / 16, HQ = S::H / 16, HA = S::t32(S::H);
    extern __shared__ __align__(16) unsigned char smem[];
    h8 *frags = (h8 *)smem;
    float *bias = (float *)(smem + LY::bias_off);
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 31, g = lane >> 5;
    constexpr bool kDecode16 = (MODE == kFwdDecode || MODE == kFwdDecode16) && C == 16;
    __shared__ int64_t mip_tab[kDecode16 ? NT_MAX_GRIDS * NT_MAX_MIPS : 1];
    stage_weights<S, true, kDecode16>(d.mlp, frags, bias, tid, kFwdThreads);
    if constexpr (kDecode16) {
        // Texel (expanded pass) or byte (blocks) offset of every (grid, mip) level.
        if (tid < NT_MAX_GRIDS * NT_MAX_MIPS) {
            const int gi = tid / NT_MAX_MIPS, m = tid % NT_MAX_MIPS;
            mip_tab[tid] = gi < d.G ? (MODE == kFwdDecode16 ? d.grid[gi].mip_off[m] : d.cgrid[gi].byte_off[m]) : 0;
        }
    }
    __syncthreads();

    float sse = 0.f;
    const int ntiles = (d.count + 31) / 32;
    for (int tile = blockIdx.x * 4 + wave; tile < ntiles; tile += gridDim.x * 4) {
        const int s = tile * 32 + c;
        const bool valid = s < d.count;
        h8 x0[KQ0];
        float u = 0.f, v = 0.f;
        if constexpr (MODE == kFwdMlp) {
            const int in = d.mlp.sizes[0];
#pragma unroll
            for (int q = 0; q < KQ0; ++q)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int feat = natural_feature(q, g, e);
                    x0[q][e] = (valid && feat < in) ? bits_h(d.inputs[(int64_t)s * in + feat])
                                                    : (_Float16)0.f;
                }
        } else if constexpr (MODE == kFwdBilinear || MODE == kFwdCatmullRom) {
            const int sc = valid ? s : 0;
            u = d.uvz[3 * (int64_t)sc];
            v = d.uvz[3 * (int64_t)sc + 1];
            const float z = d.uvz[3 * (int64_t)sc + 2];
            if constexpr (MODE == kFwdBilinear)
                sample_bilinear<C, KQ0>(d, u, v, z, g, x0);
            else
                sample_catmull_rom<C, KQ0>(d, u, v, g, x0);
        } else if constexpr (MODE == kFwdInference) {
            const int sc = valid ? s : 0;
            const int px = sc % d.image_w, py = sc / d.image_w;
            u = div_pow2((float)px + 0.5f, (float)d.image_w, d.inv_w); // train.cu:926-933
            v = div_pow2((float)py + 0.5f, (float)d.image_h, d.inv_h);
            sample_bilinear<C, KQ0>(d, u, v, 0.f, g, x0);
        } else { // kFwdDecode, kFwdDecode16
            const int sc = valid ? s : 0;
            const int px = sc % d.image_w, py = sc / d.image_w;
            uint32_t st = mix_seed((uint32_t)sc, d.seed);
            const float jx = uniform01(st) - 0.5f;
            const float jy = uniform01(st) - 0.5f;
            const float zu = uniform01(st);
            const float posx = clampf(fmaf(d.jitter, jx, (float)px + 0.5f), 0.5f, (float)d.image_w - 0.5f);
            const float posy = clampf(fmaf(d.jitter, jy, (float)py + 0.5f), 0.5f, (float)d.image_h - 0.5f);
            u = div_pow2(posx, (float)d.image_w, d.inv_w);
            v = div_pow2(posy, (float)d.image_h, d.inv_h);
            const float z = fmaf(d.mip_max - d.mip_min, zu, d.mip_min);
            if constexpr (kDecode16)
                sample_decode16<KQ0, MODE == kFwdDecode16>(d, mip_tab, u, v, z, g, x0);
            else
                sample_codec<C, KQ0>(d, u, v, z, g, x0);
        }
        if (d.features != nullptr && valid) {
            const int nf = d.G * C;
#pragma unroll
            for (int q = 0; q < KQ0; ++q)
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int feat = natural_feature(q, g, e);
                    if (feat < nf)
                        d.features[(int64_t)s * nf + feat] = h_bits(x0[q][e]);
                }
        }

        // MLP forward (mlp.h:65-99)
        h8 xh[HQ];
        {
            f16v acc[HA];
            layer_forward<KQ0, HA>(frags + S::fwd_off(0) * kWave, bias + S::bias_off(0), x0, acc, lane);
            to_fragments<HQ, HA, true>(acc, xh);
#pragma unroll
            for (int l = 1; l < NH; ++l) {
                layer_forward<HQ, HA>(frags + S::fwd_off(l) * kWave, bias + S::bias_off(l), xh, acc, lane);
                to_fragments<HQ, HA, true>(acc, xh);
            }
        }
        f16v out[1];
        layer_forward<HQ, 1>(frags + S::fwd_off(L - 1) * kWave, bias + S::bias_off(L - 1), xh, out, lane);

        if (!valid)
            continue;
        if constexpr (MODE == kFwdInference) {
            // Targets for the SSE (train.cu:935-960).
            float tgt[8];
#pragma unroll
            for (int e = 0; e < 8; ++e)
                tgt[e] = 0.f;
            for (int ti = 0; ti < d.ntex; ++ti) {
                bool need = false;
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    need |= d.out_tex[chained_feature(0, g, e)] == ti;
                if (!need)
                    continue;
                const TexDesc tx = d.tex[ti];
                float wx[4], wy[4];
                const int x0t = cr_axis(u, tx.w, wx), y0t = cr_axis(v, tx.h, wy);
                float acc[4] = {0.f, 0.f, 0.f, 0.f};
                for (int j = 0; j < 4; ++j) {
                    const int y = wrap_coord(y0t + j, tx.h);
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int x = wrap_coord(x0t + i, tx.w);
                        const float wxy = wx[i] * wy[j];
                        const int64_t base = ((int64_t)y * tx.w + x) * tx.pitch;
                        if (tx.pitch == 4) {
                            const float4 p = *(const float4 *)(tx.texels + base);
                            acc[0] = fmaf(p.x, wxy, acc[0]);
                            if (tx.nch > 1)
                                acc[1] = fmaf(p.y, wxy, acc[1]);
                            if (tx.nch > 2)
                                acc[2] = fmaf(p.z, wxy, acc[2]);
                            if (tx.nch > 3)
                                acc[3] = fmaf(p.w, wxy, acc[3]);
                        } else {
                            acc[0] = fmaf(tx.texels[base], wxy, acc[0]);
                        }
                    }
                }
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int o = chained_feature(0, g, e);
                    if (d.out_tex[o] == ti) {
                        const int ch = d.out_ch[o];
                        tgt[e] = ch == 0 ? acc[0] : ch == 1 ? acc[1] : ch == 2 ? acc[2] : acc[3];
                    }
                }
            }
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int o = chained_feature(0, g, e);
                if (o < d.out_stride) {
                    const float y = (float)(_Float16)out[0][e];
                    d.out32[(int64_t)s * d.out_stride + o] = y;
                    const float err = y - tgt[e];
                    sse = fmaf(err, err, sse);
                }
            }
        } else {
            // Lane group g holds output rows 4g .. 4g+3 and 8+4g .. 8+4g+3: with a row stride
            // that is a multiple of 4 each run of four is one 8-byte store.
            uint16_t *orow = d.out16 + (int64_t)s * d.out_stride;
            const bool quads = (d.out_stride & 3) == 0; // uniform: one of the two paths runs
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                const int o = 8 * j + 4 * g;
                const f2 v0 = {out[0][4 * j], out[0][4 * j + 1]}, v1 = {out[0][4 * j + 2], out[0][4 * j + 3]};
                const h2 h0 = __builtin_convertvector(v0, h2), h1 = __builtin_convertvector(v1, h2);
                if (quads) {
                    if (o < d.out_stride)
                        *(uint2 *)(orow + o) = make_uint2(__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1));
                } else {
                    const _Float16 hv[4] = {h0[0], h0[1], h1[0], h1[1]};
#pragma unroll
                    for (int r = 0; r < 4; ++r)
                        if (o + r < d.out_stride)
                            orow[o + r] = h_bits(hv[r]);
                }
            }
        }
    }
    if constexpr (MODE == kFwdInference) {
#pragma unroll
        for (int off = 32; off >= 1; off >>= 1)
            sse += __shfl_xor(sse, off);
        if (lane == 0) {
            if (d.sse_partial)
                d.sse_partial[blockIdx.x * kFwdWaves + wave] = sse;
            else if (sse != 0.f)
                global_add(d.sse, sse);
        }
    }
}

// The fixed-order SSE reduction: thread t sums partial[t], partial[t + 256], ... in index
// order, then a pairwise tree over the 256 sums; the result is the same bits on every run.
__global__ __launch_bounds__(256) void sse_reduce_kernel(const float *partial, int n, float *sse)
{
    __shared__ float part[256];
    const int t = threadIdx.x;
    float s = 0.f;
    for (int i = t; i < n; i += 256)
        s += partial[i];
    part[t] = s;
    __syncthreads();
    for (int w = 128; w > 0; w >>= 1) {
        if (t < w)
            part[t] += part[t + w];
        __syncthreads();
    }
    if (t == 0)
        sse[0] = sse[0] + part[0];
}

hipError_t launch_sse_reduce(const float *partial, int n, float *sse, hipStream_t s)
{
    hipLaunchKernelGGL(sse_reduce_kernel, dim3(1), dim3(256), 0, s, partial, n, sse);
    return hipGetLastError();
}

// ---- LDS-staged decode (second pass of the two-pass decode) ----------------------------
// Same per-pixel arithmetic as forward_kernel<..., Decode16> (and so the same bits): the
// corner texels come from per-block LDS boxes instead of HBM/L2. Box entry of (grid, mip):
// {first texel, width | height << 16, origin x, origin y}.

__device__ __forceinline__ int wrap_mod(int c, int size)
{
    const int r = c % size;
    return r < 0 ? r + size : r;
}

// Sampling record of (grid, mip), built per block: the LDS byte address of box texel
// (0, 0) of the unwrapped grid (the box's first texel minus its origin, so that a
// footprint origin (x0, y0) is at base + 32 x0 + y0 row), the box row in bytes, and the
// mip's dimensions as floats (exact: they are below 2^24).
struct BoxSample {
    int base, row;
    float w, h;
};

typedef __attribute__((address_space(3))) const uint4 lds_uint4;

template <int G>
__device__ __forceinline__ void sample_box16(const int *max_mip, const BoxSample *samp, float u, float v, float z,
                                             int g, h8 (&x)[G])
{
    // Mip pair (train.cu:266-281, as mip_pair) with the grids' clamp bound precomputed.
    const float fz = floorf(z);
    const int base = (int)fz;
    const float frac = z - fz;
#pragma unroll
    for (int j = 0; j < G / 2; ++j) {
        const int gi = 2 * j + g, top = max_mip[gi];
        const int mips[2] = {min(max(base, 0), top), min(max(base + 1, 0), top)};
        const float mw[2] = {1.f - frac, frac};
        h8 lo = (h8)(_Float16)0.f, hi = (h8)(_Float16)0.f;
        const int nm = frac > 0.f ? 2 : 1;
        for (int mi = 0; mi < nm; ++mi) {
            const BoxSample q = samp[gi * NT_MAX_MIPS + mips[mi]];
            const Footprint f = bilinear_footprint(u, v, q.w, q.h, mw[mi]);
            // In the box by construction: the box origin is the footprint origin of the
            // block's lowest position and its size covers the highest one's (box_origin,
            // box_last, the same float operations), and the origin is monotone in the
            // position (fma, a division by the image size, floor), so the footprint's
            // 2 x 2 texels lie in the box (x0 and y0 are at least -1: 24-bit products).
            const int a = q.base + 32 * f.x0 + __mul24(f.y0, q.row);
            const lds_uint4 *t = (const lds_uint4 *)(size_t)(uint32_t)a;
            const lds_uint4 *t2 = (const lds_uint4 *)(size_t)(uint32_t)(a + q.row);
            fma_corner16(lo, hi, f.w[0], __builtin_bit_cast(h8, t[0]), __builtin_bit_cast(h8, t[1]));
            fma_corner16(lo, hi, f.w[1], __builtin_bit_cast(h8, t[2]), __builtin_bit_cast(h8, t[3]));
            fma_corner16(lo, hi, f.w[2], __builtin_bit_cast(h8, t2[0]), __builtin_bit_cast(h8, t2[1]));
            fma_corner16(lo, hi, f.w[3], __builtin_bit_cast(h8, t2[2]), __builtin_bit_cast(h8, t2[3]));
            // One mip level's reads at a time keeps the register peak down.
            __builtin_amdgcn_sched_barrier(0);
        }
        x[2 * j] = lo;
        x[2 * j + 1] = hi;
    }
}

template <class S>
__global__ __launch_bounds__(kFwdThreads, 4) void decode_box_kernel(DecodeBoxDesc d)
{
    using LY = FwdLayout<S>;
    constexpr int L = S::L, NH = S::NH, KQ0 = S::K0 / 16, HQ = S::H / 16, HA = S::t32(S::H);
    constexpr int kTiles = kBoxBlockW / 32 * kBoxBlockH;
    extern __shared__ __align__(16) unsigned char smem[];
    h8 *frags = (h8 *)smem;
    float *bias = (float *)(smem + LY::bias_off);
    uint4 *box = (uint4 *)(smem + d.lds_box_off);
    // The (grid, mip) entry of every box texel, after the boxes: the boxes' places do not
    // change from block to block, so it is found once per launch.
    uint8_t *owner = (uint8_t *)(box + 2 * d.box_texels);
    __shared__ int4 tab[NT_MAX_GRIDS * NT_MAX_MIPS];
    // Per (grid, mip): the mip's dimensions (w | h << 16), 1/box width (0: no box), the
    // mip's texels.
    __shared__ int4 tab2[NT_MAX_GRIDS * NT_MAX_MIPS];
    __shared__ BoxSample samp[NT_MAX_GRIDS * NT_MAX_MIPS];
    __shared__ int max_mip[NT_MAX_GRIDS];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6, c = lane & 31, g = lane >> 5;
    // LDS byte address of the boxes.
    const int box_addr = (int)(uint32_t)(size_t)(__attribute__((address_space(3))) unsigned char *)(smem + d.lds_box_off);
    stage_weights<S, true, true>(d.mlp, frags, bias, tid, kFwdThreads);
    if (tid < NT_MAX_GRIDS)
        max_mip[tid] = tid < d.G && d.grid[tid].num_mips > 0 ? d.grid[tid].num_mips - 1 : 0;
    // Per (grid, mip), once per launch: the box's place and size (tab.xy; the origins, tab.zw,
    // are each block's), and tab2 (mip dimensions, 1/box width, or 0 with no box, texels).
    if (tid < NT_MAX_GRIDS * NT_MAX_MIPS) {
        const int gi = tid / NT_MAX_MIPS, m = tid % NT_MAX_MIPS;
        int4 e = make_int4(0, 0x20002, 0, 0), f = make_int4(0, 0, 0, 0);
        if (gi < d.G) {
            const BoxGrid &q = d.grid[gi];
            const uintptr_t base = (uintptr_t)(q.texels + q.mip_off[m] * 16);
            f = make_int4(mip_dim(q.w, m) | (mip_dim(q.h, m) << 16), 0, (int)(uint32_t)base, (int)(uint32_t)(base >> 32));
            if (m >= q.mip_lo && m <= q.mip_hi) {
                e.x = q.box_off[m];
                e.y = q.box_w[m] | (q.box_h[m] << 16);
                f.y = __float_as_int(1.f / (float)q.box_w[m]);
            }
        }
        tab[tid] = e;
        tab2[tid] = f;
    }
    for (int k = tid; k < d.box_texels; k += kFwdThreads) {
        int o = 0;
        for (int a = 0; a < d.G; ++a) {
            const BoxGrid &q = d.grid[a];
            for (int b = q.mip_lo; b <= q.mip_hi; ++b)
                if (k >= q.box_off[b])
                    o = a * NT_MAX_MIPS + b;
        }
        owner[k] = (uint8_t)o;
    }

    const int nblocks = d.blocks_x * d.blocks_y;
    for (int blk = blockIdx.x; blk < nblocks; blk += gridDim.x) {
        const int bx0 = (blk % d.blocks_x) * kBoxBlockW, by0 = (blk / d.blocks_x) * kBoxBlockH;
        __syncthreads(); // the previous block's reads of the boxes (and the weight staging) are done
        if (tid < NT_MAX_GRIDS * NT_MAX_MIPS) {
            // The block's box origins, from the launch's table (LDS).
            int4 e = tab[tid];
            const int4 f = tab2[tid];
            const int mw = f.x & 0xFFFF, mh = (int)((uint32_t)f.x >> 16);
            if (f.y != 0) {
                e.z = box_origin(bx0, d.image_w, d.jitter, mw);
                e.w = box_origin(by0, d.image_h, d.jitter, mh);
                tab[tid] = e;
            }
            const int bw = e.y & 0xFFFF;
            samp[tid] = BoxSample{box_addr + 32 * (e.x - e.w * bw - e.z), 32 * bw, f.x != 0 ? (float)mw : 1.f,
                                  f.x != 0 ? (float)mh : 1.f};
        }
        __syncthreads();
        // Stage the boxes: texel k of box (gi, m) is global texel (origin + (k % bw, k / bw)),
        // wrapped; two 16-byte halves per texel, copied into LDS without passing through
        // registers (lane l of a wave instruction writes the l-th 16 bytes from its base).
        // k / bw by a float reciprocal and one correction (below 2^22).
        for (int i = tid; i < 2 * d.box_texels; i += kFwdThreads) {
            const int k = i >> 1, o = owner[k];
            const int4 e = tab[o], f = tab2[o];
            const int bw = e.y & 0xFFFF, local = k - e.x;
            int ly = (int)((float)local * __int_as_float(f.y));
            int lx = local - ly * bw;
            if (lx >= bw) {
                lx -= bw;
                ++ly;
            } else if (lx < 0) {
                lx += bw;
                --ly;
            }
            const int w = f.x & 0xFFFF, h = (int)((uint32_t)f.x >> 16);
            int gx = e.z + lx, gy = e.w + ly;
            if ((unsigned)gx >= (unsigned)w)
                gx = wrap_mod(gx, w);
            if ((unsigned)gy >= (unsigned)h)
                gy = wrap_mod(gy, h);
            const uint16_t *base = (const uint16_t *)(((uintptr_t)(uint32_t)f.w << 32) | (uint32_t)f.z);
            const uint4 *src = (const uint4 *)(base + ((int64_t)gy * w + gx) * 16) + (i & 1);
            __builtin_amdgcn_global_load_lds((const void *)src,
                                             (__attribute__((address_space(3))) void *)(box + (i & ~63)), 16, 0, 0);
        }
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();

        // Two tiles per wave at a time (t and t + kFwdWaves), sharing the weight reads.
        static_assert(kTiles % (2 * kFwdWaves) == 0, "whole tile pairs per wave");
        for (int t0 = wave; t0 < kTiles; t0 += 2 * kFwdWaves) {
            int s[2];
            bool valid[2];
            h8 x0[2][KQ0];
            // Both lane groups sample pixel c of both tiles. Lane group g computes the
            // position and mip of pixel c of tile g only (as forward_kernel<..., Decode16>,
            // pixel index s); one v_permlane32_swap of the wave's halves per value then hands
            // every lane both: the first result holds the lower half's values (tile 0) in
            // every lane, the second the upper half's (tile 1).
            float uvz[3][2];
            {
                const int t = t0 + g * kFwdWaves;
                const int px = bx0 + 32 * (t % (kBoxBlockW / 32)) + c, py = by0 + t / (kBoxBlockW / 32);
                const int cx = min(px, d.image_w - 1), cy = min(py, d.image_h - 1);
                uint32_t st = mix_seed((uint32_t)(cy * d.image_w + cx), d.seed);
                const float jx = uniform01(st) - 0.5f;
                const float jy = uniform01(st) - 0.5f;
                const float zu = uniform01(st);
                const float posx = clampf(fmaf(d.jitter, jx, (float)cx + 0.5f), 0.5f, (float)d.image_w - 0.5f);
                const float posy = clampf(fmaf(d.jitter, jy, (float)cy + 0.5f), 0.5f, (float)d.image_h - 0.5f);
                const float mine[3] = {div_pow2(posx, (float)d.image_w, d.inv_w),
                                       div_pow2(posy, (float)d.image_h, d.inv_h),
                                       fmaf(d.mip_max - d.mip_min, zu, d.mip_min)};
#pragma unroll
                for (int i = 0; i < 3; ++i) {
                    const uint32_t b = __float_as_uint(mine[i]);
                    const auto r = __builtin_amdgcn_permlane32_swap(b, b, false, false);
                    uvz[i][0] = __uint_as_float(r[0]);
                    uvz[i][1] = __uint_as_float(r[1]);
                }
            }
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                const int t = t0 + k * kFwdWaves;
                const int px = bx0 + 32 * (t % (kBoxBlockW / 32)) + c, py = by0 + t / (kBoxBlockW / 32);
                valid[k] = px < d.image_w && py < d.image_h;
                s[k] = min(py, d.image_h - 1) * d.image_w + min(px, d.image_w - 1);
                sample_box16<KQ0>(max_mip, samp, uvz[0][k], uvz[1][k], uvz[2][k], g, x0[k]);
            }

            f16v out[2][1];
            {
                h8 xh[2][HQ];
                f16v acc[2][HA];
                layer_forward2<KQ0, HA>(frags + S::fwd_off(0) * kWave, bias + S::bias_off(0), x0[0], x0[1], acc[0],
                                        acc[1], lane);
                to_fragments<HQ, HA, true>(acc[0], xh[0]);
                to_fragments<HQ, HA, true>(acc[1], xh[1]);
#pragma unroll
                for (int l = 1; l < NH; ++l) {
                    layer_forward2<HQ, HA>(frags + S::fwd_off(l) * kWave, bias + S::bias_off(l), xh[0], xh[1], acc[0],
                                           acc[1], lane);
                    to_fragments<HQ, HA, true>(acc[0], xh[0]);
                    to_fragments<HQ, HA, true>(acc[1], xh[1]);
                }
                layer_forward2<HQ, 1>(frags + S::fwd_off(L - 1) * kWave, bias + S::bias_off(L - 1), xh[0], xh[1],
                                      out[0], out[1], lane);
            }
            const bool quads = (d.out_stride & 3) == 0;
#pragma unroll
            for (int k = 0; k < 2; ++k) {
                if (!valid[k])
                    continue;
                uint16_t *orow = d.out16 + (int64_t)s[k] * d.out_stride;
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int o = 8 * j + 4 * g;
                    const f2 v0 = {out[k][0][4 * j], out[k][0][4 * j + 1]}, v1 = {out[k][0][4 * j + 2], out[k][0][4 * j + 3]};
                    const h2 h0 = __builtin_convertvector(v0, h2), h1 = __builtin_convertvector(v1, h2);
                    if (quads) {
                        if (o < d.out_stride)
                            *(uint2 *)(orow + o) = make_uint2(__builtin_bit_cast(uint32_t, h0), __builtin_bit_cast(uint32_t, h1));
                    } else {
                        const _Float16 hv[4] = {h0[0], h0[1], h1[0], h1[1]};
#pragma unroll
                        for (int r = 0; r < 4; ++r)
                            if (o + r < d.out_stride)
                                orow[o + r] = h_bits(hv[r]);
                    }
                }
            }
        }
    }
}

template <class S>
static hipError_t launch_box(const DecodeBoxDesc &d, hipStream_t s)
{
    const int nblocks = d.blocks_x * d.blocks_y;
    const int grid = nblocks < 2048 ? nblocks : 2048;
    const size_t lds = (size_t)d.lds_box_off + (size_t)d.box_texels * 33; // the boxes and their owner bytes
    if ((size_t)d.lds_box_off < FwdLayout<S>::bytes)
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(decode_box_kernel<S>, dim3(grid), dim3(kFwdThreads), lds, s, d);
    return hipGetLastError();
}

hipError_t launch_decode_box(int shape, const DecodeBoxDesc &d, hipStream_t s)
{
    switch (shape) {
    case kShapeC2:
        return launch_box<Shape<32, 64, 2>>(d, s);
    case kShapeC4:
        return launch_box<Shape<64, 64, 3>>(d, s);
    default:
        return hipErrorInvalidValue;
    }
}

size_t decode_box_weight_bytes(int shape)
{
    switch (shape) {
    case kShapeC2:
        return FwdLayout<Shape<32, 64, 2>>::bytes;
    case kShapeC4:
        return FwdLayout<Shape<64, 64, 3>>::bytes;
    default:
        return 0;
    }
}

template <class S, int C, int MODE>
static hipError_t launch_fwd(const FwdDesc &d, hipStream_t s)
{
    const int blocks = forward_blocks(d.count);
    hipLaunchKernelGGL((forward_kernel<S, C, MODE>), dim3(blocks), dim3(kFwdThreads),
                       FwdLayout<S>::bytes, s, d);
    return hipGetLastError();
}

template <class S, int C>
static hipError_t launch_modes(int mode, const FwdDesc &d, hipStream_t s)
{
    switch (mode) {
    case kFwdBilinear:
        return launch_fwd<S, C, kFwdBilinear>(d, s);
    case kFwdCatmullRom:
        return launch_fwd<S, C, kFwdCatmullRom>(d, s);
    case kFwdInference:
        return launch_fwd<S, C, kFwdInference>(d, s);
    case kFwdDecode:
        if constexpr (C == 16 || C == 8)
            return launch_fwd<S, C, kFwdDecode>(d, s);
        return hipErrorInvalidValue;
    case kFwdDecode16:
        if constexpr (C == 16)
            return launch_fwd<S, C, kFwdDecode16>(d, s);
        return hipErrorInvalidValue;
    default:
        return hipErrorInvalidValue;
    }
}

hipError_t launch_forward(int shape, int mode, const FwdDesc &d, hipStream_t s)
{
    if (mode == kFwdMlp) {
        switch (shape) {
        case kShapeRef:
            return launch_fwd<Shape<16, 32, 2>, 0, kFwdMlp>(d, s);
        case kShapeFpt:
            return launch_fwd<Shape<16, 16, 1>, 0, kFwdMlp>(d, s);
        case kShapeC1:
            return launch_fwd<Shape<16, 64, 2>, 0, kFwdMlp>(d, s);
        case kShapeC2:
            return launch_fwd<Shape<32, 64, 2>, 0, kFwdMlp>(d, s);
        case kShapeC4:
            return launch_fwd<Shape<64, 64, 3>, 0, kFwdMlp>(d, s);
        default:
            return hipErrorInvalidValue;
        }
    }
    switch (shape) {
    case kShapeRef:
        return launch_modes<Shape<16, 32, 2>, 3>(mode, d, s);
    case kShapeC1:
        return launch_modes<Shape<16, 64, 2>, 8>(mode, d, s);
    case kShapeC2:
        return launch_modes<Shape<32, 64, 2>, 16>(mode, d, s);
    case kShapeC4:
        return launch_modes<Shape<64, 64, 3>, 16>(mode, d, s);
    default:
        return hipErrorInvalidValue;
    }
}

} // namespace ntk
