/*
 * nt_oracle.c — scalar CPU restatement of the reference train/decode path.
 *
 * TEST INFRASTRUCTURE ONLY (parity checker and CPU baseline); see nt_oracle.h for the
 * floating-point policy. Build: oracle/build.sh (gcc -O2 -ffp-contract=off -fopenmp).
 * Citations are to mavenkim2/neural_textures.
 */
#include "nt_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

#define PAD16(x) (((x) + 15) & ~15)
#define MAXW 64

/* ---- fp16 ------------------------------------------------------------------------- */

/* Round a double to IEEE binary16, nearest-even, subnormals kept. The sum of two fp16
 * values is exact in double, so ntref_f16_add rounds exactly once, like __hadd. */
static uint16_t f64_to_f16(double d)
{
    uint64_t x;
    memcpy(&x, &d, 8);
    const uint16_t sign = (uint16_t)((x >> 48) & 0x8000u);
    const uint64_t absx = x & 0x7FFFFFFFFFFFFFFFull;
    if (absx >= 0x7FF0000000000000ull) {
        if (absx > 0x7FF0000000000000ull)
            return (uint16_t)(sign | 0x7E00u | ((absx >> 42) & 0x3FFu));
        return (uint16_t)(sign | 0x7C00u);
    }
    const int e = (int)(absx >> 52);
    if (e == 0)
        return sign; /* double subnormals are far below the fp16 range */
    const uint64_t mant = (absx & 0xFFFFFFFFFFFFFull) | (1ull << 52);
    const int he = e - 1023 + 15;
    if (he >= 31)
        return (uint16_t)(sign | 0x7C00u);
    if (he <= 0) {
        /* fp16 subnormal: value = mant * 2^(e-1075) = q * 2^-24 */
        const int s = 1051 - e;
        if (s >= 64)
            return sign;
        uint64_t q = mant >> s;
        const uint64_t rem = mant & ((1ull << s) - 1);
        const uint64_t half = 1ull << (s - 1);
        if (rem > half || (rem == half && (q & 1)))
            ++q;
        return (uint16_t)(sign | (uint16_t)q);
    }
    const uint64_t rem = mant & ((1ull << 42) - 1);
    const uint64_t half = 1ull << 41;
    uint32_t h = ((uint32_t)he << 10) + (uint32_t)((mant >> 42) & 0x3FFu);
    if (rem > half || (rem == half && (h & 1)))
        ++h;
    if (h >= 0x7C00u)
        return (uint16_t)(sign | 0x7C00u);
    return (uint16_t)(sign | h);
}

uint16_t ntref_f32_to_f16(float f) { return f64_to_f16((double)f); }

float ntref_f16_to_f32(uint16_t h)
{
    const uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    const uint32_t e = ((uint32_t)h >> 10) & 0x1Fu;
    const uint32_t m = (uint32_t)h & 0x3FFu;
    uint32_t x;
    if (e == 0) {
        float v = (float)m * 5.9604644775390625e-8f; /* m * 2^-24, exact */
        memcpy(&x, &v, 4);
        x |= sign;
    } else if (e == 31) {
        x = sign | 0x7F800000u | (m << 13);
    } else {
        x = sign | ((e + 112u) << 23) | (m << 13);
    }
    float f;
    memcpy(&f, &x, 4);
    return f;
}

uint16_t ntref_f16_add(uint16_t a, uint16_t b)
{
    return f64_to_f16((double)ntref_f16_to_f32(a) + (double)ntref_f16_to_f32(b));
}

static double h2d(uint16_t h) { return (double)ntref_f16_to_f32(h); }

/* With this switch on, the MLP's forward sums and its backward dY W^T sums accumulate in
 * fp32 (in index order, the fp16 products exact) instead of float64: a second, equally
 * valid accumulation order, with which the tests measure how sensitive each gradient
 * element is to the order of the fp32 sums (the GPU's MFMA order is a third). */
static int g_mlp_accum_f32 = 0;

void ntref_set_mlp_accum_f32(int on)
{
    g_mlp_accum_f32 = on != 0;
}

/* ---- RNG and sample positions (train.cu:37-58, 818-844) --------------------------- */

uint32_t ntref_xorshift32(uint32_t *state)
{
    uint32_t x = *state;
    x ^= x << 13;
    x ^= x >> 17;
    x ^= x << 5;
    *state = x;
    return x;
}

float ntref_uniform(uint32_t *state)
{
    return (float)(ntref_xorshift32(state) & 0x00FFFFFFu) * (1.0f / 16777216.0f);
}

uint32_t ntref_sample_seed(uint32_t sample_index, int step)
{
    const uint32_t seed = sample_index ^ ((uint32_t)step * 747796405u + 2891336453u);
    return seed ? seed : 1u; /* RNG(0) starts at 1 (train.cu:41) */
}

static float clampf(float x, float lo, float hi) { return x < lo ? lo : (x > hi ? hi : x); }

static int wrap_coord(int c, int size)
{
    int w = c % size; /* WrapTexelCoord, train.cu:65-69 */
    return w < 0 ? w + size : w;
}

static int mip_dim(int size, int mip)
{
    int d = size >> mip; /* GetMipDimension, train.cu:214-218 */
    return d > 0 ? d : 1;
}

uint32_t ntref_fmix32(uint32_t h)
{
    /* MurmurHash3's 32-bit finalizer (public domain, Austin Appleby). */
    h ^= h >> 16;
    h *= 0x85EBCA6Bu;
    h ^= h >> 13;
    h *= 0xC2B2AE35u;
    h ^= h >> 16;
    return h;
}

void ntref_sample_uvz(const nt_params *p, uint32_t i, float uvz[3])
{
    const uint32_t rw = p->region_width > 0 ? (uint32_t)p->region_width : NT_DEFAULT_REGION;
    uint32_t sx = (uint32_t)p->texel_offset_x + i % rw;
    uint32_t sy = (uint32_t)p->texel_offset_y + i / rw;
    uint32_t st = ntref_sample_seed(i, p->step);
    if (p->sample_mode == NT_SAMPLES_RANDOM) {
        /* A uniformly random texel of the image (nt.h nt_sample_mode), then the jitter. */
        const uint32_t h1 = ntref_fmix32(st), h2 = ntref_fmix32(h1);
        const uint32_t x = (uint32_t)((float)(h1 & 0x00FFFFFFu) * (1.0f / 16777216.0f) * (float)p->image_width);
        const uint32_t y = (uint32_t)((float)(h2 & 0x00FFFFFFu) * (1.0f / 16777216.0f) * (float)p->image_height);
        sx = x < (uint32_t)p->image_width ? x : (uint32_t)p->image_width - 1;
        sy = y < (uint32_t)p->image_height ? y : (uint32_t)p->image_height - 1;
    }
    const float jx = ntref_uniform(&st) - 0.5f;
    const float jy = ntref_uniform(&st) - 0.5f;
    const float px = clampf((float)sx + 0.5f + jx, 0.5f, (float)p->image_width - 0.5f);
    const float py = clampf((float)sy + 0.5f + jy, 0.5f, (float)p->image_height - 0.5f);
    uvz[0] = px / (float)p->image_width;
    uvz[1] = py / (float)p->image_height;
    uvz[2] = p->sample_mip; /* 0 in the reference (train.cu:844) */
}

/* ---- latent sampling -------------------------------------------------------------- */

/* Bilinear footprint of one mip (train.cu:284-291). */
typedef struct {
    int w, h, x0, y0;
    float fx, fy;
} footprint;

static footprint make_footprint(int gw, int gh, int mip, float u, float v)
{
    footprint f;
    f.w = mip_dim(gw, mip);
    f.h = mip_dim(gh, mip);
    const float tu = fmaf(u, (float)f.w, -0.5f);
    const float tv = fmaf(v, (float)f.h, -0.5f);
    const float bu = floorf(tu), bv = floorf(tv);
    f.x0 = (int)bu;
    f.y0 = (int)bv;
    f.fx = tu - bu;
    f.fy = tv - bv;
    return f;
}

static float corner_weight(const footprint *f, int corner, float mip_weight)
{
    const int cx = corner & 1, cy = corner >> 1;
    const float wu = cx ? f->fx : 1.f - f->fx; /* BilinearWeight, train.cu:71-76 */
    const float wv = cy ? f->fy : 1.f - f->fy;
    return mip_weight * (wu * wv);
}

/* Mips visited for mip coordinate z (train.cu:266-281). Returns the count (1 or 2). */
static int mip_pair(const nt_grid *g, float z, int mips[2], float weights[2])
{
    const int base = (int)floorf(z);
    const float frac = z - floorf(z);
    const int max_mip = g->num_mips > 0 ? g->num_mips - 1 : 0;
    const int n = frac > 0.f ? 2 : 1;
    for (int i = 0; i < n; ++i) {
        int m = base + i < max_mip ? base + i : max_mip;
        mips[i] = m < 0 ? 0 : m;
        weights[i] = i ? frac : 1.f - frac;
    }
    return n;
}

void ntref_sample_latents_bilinear(const nt_latents *lat, const float uvz[3], uint16_t *out)
{
    const int C = lat->channels;
    for (int i = 0; i < lat->num_grids * C; ++i)
        out[i] = 0;
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid *g = &lat->grids[gi];
        int mips[2];
        float mw[2];
        const int n = mip_pair(g, uvz[2], mips, mw);
        for (int mi = 0; mi < n; ++mi) {
            const footprint f = make_footprint(g->width, g->height, mips[mi], uvz[0], uvz[1]);
            for (int corner = 0; corner < 4; ++corner) {
                const int x = wrap_coord(f.x0 + (corner & 1), f.w);
                const int y = wrap_coord(f.y0 + (corner >> 1), f.h);
                const float w = corner_weight(&f, corner, mw[mi]);
                const float *t = g->values + (g->mip_offset[mips[mi]] + (int64_t)y * f.w + x) * C;
                for (int c = 0; c < C; ++c) /* train.cu:306-310 */
                    out[gi * C + c] = ntref_f16_add(out[gi * C + c], ntref_f32_to_f16(w * t[c]));
            }
        }
    }
}

void ntref_catmull_rom_weights(float f, float w[4])
{
    /* filter/catmull_rom.h:56-59 with nvcc's contraction made explicit */
    w[0] = f * fmaf(f, fmaf(f, -0.5f, 1.0f), -0.5f);
    w[1] = fmaf(f * f, fmaf(f, 1.5f, -2.5f), 1.0f);
    w[2] = f * fmaf(f, fmaf(f, -1.5f, 2.0f), 0.5f);
    w[3] = (f * f) * fmaf(f, 0.5f, -0.5f);
}

/* Catmull-Rom tap origin and weights along one axis (catmull_rom.h:43-59). */
static int cr_axis(float uv, int size, float w[4])
{
    const float s = uv * (float)size;
    const float b = floorf(s - 0.5f);
    ntref_catmull_rom_weights(s - (b + 0.5f), w);
    return (int)b - 1;
}

void ntref_sample_latents_catmull_rom(const nt_latents *lat, const float uvz[3], uint16_t *out)
{
    const int C = lat->channels;
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid *g = &lat->grids[gi];
        float wx[4], wy[4], acc[16] = {0};
        const int x0 = cr_axis(uvz[0], g->width, wx);
        const int y0 = cr_axis(uvz[1], g->height, wy);
        for (int j = 0; j < 4; ++j) {
            const int y = wrap_coord(y0 + j, g->height);
            for (int i = 0; i < 4; ++i) {
                const int x = wrap_coord(x0 + i, g->width);
                const float wxy = wx[i] * wy[j];
                const float *t = g->values + (g->mip_offset[0] + (int64_t)y * g->width + x) * C;
                for (int c = 0; c < C; ++c)
                    acc[c] = fmaf(t[c], wxy, acc[c]);
            }
        }
        for (int c = 0; c < C; ++c)
            out[gi * C + c] = ntref_f32_to_f16(acc[c]);
    }
}

/* ---- reference textures (train.cu:78-157, filter/catmull_rom.h:37-89) -------------- */

static void texture_mip_sample(const nt_texture *t, float u, float v, int mip, float out[4])
{
    const int w = mip_dim(t->width, mip), h = mip_dim(t->height, mip);
    const int nc = t->num_channels < 4 ? t->num_channels : 4;
    float wx[4], wy[4], acc[4] = {0.f, 0.f, 0.f, 0.f};
    const int x0 = cr_axis(u, w, wx);
    const int y0 = cr_axis(v, h, wy);
    for (int j = 0; j < 4; ++j) {
        const int y = wrap_coord(y0 + j, h);
        for (int i = 0; i < 4; ++i) {
            const int x = wrap_coord(x0 + i, w);
            const float wxy = wx[i] * wy[j];
            const float *px = t->texels + (t->mip_offset[mip] + (int64_t)y * w + x) * t->pitch;
            for (int c = 0; c < nc; ++c)
                acc[c] = fmaf(px[c], wxy, acc[c]);
        }
    }
    for (int c = 0; c < 4; ++c)
        out[c] = acc[c];
}

void ntref_sample_texture(const nt_texture *t, float u, float v, float z, float out[4])
{
    const int max_mip = t->num_mips > 0 ? t->num_mips - 1 : 0;
    const float mc = clampf(z, 0.f, (float)max_mip);
    const int m0 = (int)floorf(mc) < max_mip ? (int)floorf(mc) : max_mip;
    const int m1 = m0 + 1 < max_mip ? m0 + 1 : max_mip;
    const float frac = m1 > m0 ? mc - (float)m0 : 0.f;
    texture_mip_sample(t, u, v, m0, out);
    if (m1 == m0)
        return;
    float s1[4];
    texture_mip_sample(t, u, v, m1, s1);
    for (int c = 0; c < 4; ++c)
        out[c] = fmaf(s1[c], frac, out[c] * (1.f - frac));
}

int ntref_expected_values(const nt_params *p, const float uvz[3], float expected[16],
                          float weights[16])
{
    for (int i = 0; i < NT_MAX_OUTPUTS; ++i) {
        expected[i] = 0.f;
        if (weights)
            weights[i] = 1.f;
    }
    int oc = 0;
    const int count = p->num_textures < NT_MAX_TEXTURES ? p->num_textures : NT_MAX_TEXTURES;
    for (int ti = 0; ti < count && oc < NT_MAX_OUTPUTS; ++ti) {
        const nt_texture *t = &p->textures[ti];
        if (!t->texels || t->num_channels <= 0)
            continue;
        float s[4];
        ntref_sample_texture(t, uvz[0], uvz[1], uvz[2], s);
        const int nc = t->num_channels == 1 ? 1 : (t->num_channels < 4 ? t->num_channels : 4);
        for (int c = 0; c < nc && oc < NT_MAX_OUTPUTS; ++c) {
            expected[oc] = s[c];
            if (weights)
                weights[oc] = t->loss_weight;
            ++oc;
        }
    }
    return oc;
}

/* ---- BC6 emulation (train.cu:19-35, 159-261, 316-458) ------------------------------ */

const int ntref_bc6_partition_sets[32] = {
    0xCCCC, 0x8888, 0xEEEE, 0xECC8, 0xC880, 0xFEEC, 0xFEC8, 0xEC80,
    0xC800, 0xFFEC, 0xFE80, 0xE800, 0xFFE8, 0xFF00, 0xFFF0, 0xF000,
    0xF710, 0x008E, 0x7100, 0x08CE, 0x008C, 0x7310, 0x3100, 0x8CCE,
    0x088C, 0x3110, 0x6666, 0x366C, 0x17E8, 0x0FF0, 0x718E, 0x399C,
};
const int ntref_bc6_partition_bits[10] = {10, 7, 11, 11, 11, 9, 8, 8, 8, 6};

float ntref_bc6_unquantize(float e, int bits)
{
    return ldexpf(fmaf(31744.f, e, 32768.f), -bits); /* (31/64 * 65536) e + 32768 */
}

static float bc6_y(float q0, float q1, float x) { return fmaf(ldexpf(q1 - q0, 3), x, q0); }

static int bc6_hy(float y)
{
    return (int)fmaxf(floorf((y - 1.f) / 1024.f) - 1.f, 0.f);
}

float ntref_bc6_decompress(float e0, float e1, int bits, float x)
{
    const float y = bc6_y(ntref_bc6_unquantize(e0, bits), ntref_bc6_unquantize(e1, bits), x);
    const int hy = bc6_hy(y);
    return ldexpf(y / 1024.f - (float)hy, hy - 14);
}

typedef struct {
    const float *rec; /* block record */
    float *grad;      /* gradient record (may be NULL) */
    int pix, part, bits;
} bc6_texel;

static bc6_texel bc6_locate(const nt_grid *g, int C, int mip, int x, int y)
{
    const int w = mip_dim(g->width, mip);
    const int nbu = (w >> 2) > 0 ? (w >> 2) : 1;
    const int64_t idx = g->block_offset[mip] + (int64_t)(y >> 2) * nbu + (x >> 2);
    bc6_texel t;
    t.rec = g->block_params + idx * (4 * C + 18);
    t.grad = g->block_grads ? g->block_grads + idx * (4 * C + 16) : NULL;
    t.pix = ((y & 3) << 2) + (x & 3);
    int32_t partition, mode;
    memcpy(&partition, t.rec + 4 * C + 16, 4);
    memcpy(&mode, t.rec + 4 * C + 17, 4);
    t.part = (ntref_bc6_partition_sets[partition & 31] >> t.pix) & 1;
    t.bits = ntref_bc6_partition_bits[(unsigned)mode < 10u ? mode : 0];
    return t;
}

void ntref_sample_latents_bc6(const nt_latents *lat, const float uvz[3], uint16_t *out)
{
    const int C = lat->channels;
    for (int i = 0; i < lat->num_grids * C; ++i)
        out[i] = 0;
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid *g = &lat->grids[gi];
        int mips[2];
        float mw[2];
        const int n = mip_pair(g, uvz[2], mips, mw);
        for (int mi = 0; mi < n; ++mi) {
            const footprint f = make_footprint(g->width, g->height, mips[mi], uvz[0], uvz[1]);
            for (int corner = 0; corner < 4; ++corner) {
                const int x = wrap_coord(f.x0 + (corner & 1), f.w);
                const int y = wrap_coord(f.y0 + (corner >> 1), f.h);
                const float w = corner_weight(&f, corner, mw[mi]);
                const bc6_texel t = bc6_locate(g, C, mips[mi], x, y);
                const float *e0 = t.rec + (2 * t.part) * C, *e1 = e0 + C;
                const float xi = t.rec[4 * C + t.pix];
                for (int c = 0; c < C; ++c) {
                    /* half += float (train.cu:365-367) is operator+=(__half&, const __half&):
                     * the fp32 product is rounded to fp16, then added in fp16 */
                    const float v = w * ntref_bc6_decompress(e0[c], e1[c], t.bits, xi);
                    out[gi * C + c] = ntref_f16_add(out[gi * C + c], ntref_f32_to_f16(v));
                }
            }
        }
    }
}

static void scatter_bc6(const nt_latents *lat, const float uvz[3], const uint16_t *dinput)
{
    const int C = lat->channels;
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid *g = &lat->grids[gi];
        int mips[2];
        float mw[2];
        const int n = mip_pair(g, uvz[2], mips, mw);
        for (int mi = 0; mi < n; ++mi) {
            const footprint f = make_footprint(g->width, g->height, mips[mi], uvz[0], uvz[1]);
            for (int corner = 0; corner < 4; ++corner) {
                const int x = wrap_coord(f.x0 + (corner & 1), f.w);
                const int y = wrap_coord(f.y0 + (corner >> 1), f.h);
                const float w = corner_weight(&f, corner, mw[mi]);
                const bc6_texel t = bc6_locate(g, C, mips[mi], x, y);
                const int base = 2 * t.part;
                const float *e0 = t.rec + base * C, *e1 = e0 + C;
                const float xi = t.rec[4 * C + t.pix];
                const float alpha = ldexpf(xi, 3);
                const float deibar = ldexpf(31.f / 64.f, 16 - t.bits);
                float dl_dx = 0.f;
                for (int c = 0; c < C; ++c) { /* train.cu:434-454 */
                    const float q0 = ntref_bc6_unquantize(e0[c], t.bits);
                    const float q1 = ntref_bc6_unquantize(e1[c], t.bits);
                    const int hy = bc6_hy(bc6_y(q0, q1, xi));
                    const float fg = w * ntref_f16_to_f32(dinput[gi * C + c]);
                    const float dl_dy = ldexpf(fg, hy - 24);
                    const float dy_dx = ldexpf(q1 - q0, 3);
                    dl_dx = c == 0 ? dl_dy * dy_dx : fmaf(dl_dy, dy_dx, dl_dx);
                    t.grad[base * C + c] += ((1.f - alpha) * deibar) * dl_dy;
                    t.grad[(base + 1) * C + c] += (alpha * deibar) * dl_dy;
                }
                t.grad[4 * C + t.pix] += dl_dx;
            }
        }
    }
}

/* ---- latent gradient scatter (train.cu:460-509) ----------------------------------- */

static void scatter_unconstrained(const nt_latents *lat, const float uvz[3],
                                  const uint16_t *dinput, int atomic)
{
    const int C = lat->channels;
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid *g = &lat->grids[gi];
        int mips[2];
        float mw[2];
        const int n = mip_pair(g, uvz[2], mips, mw);
        for (int mi = 0; mi < n; ++mi) {
            const footprint f = make_footprint(g->width, g->height, mips[mi], uvz[0], uvz[1]);
            for (int corner = 0; corner < 4; ++corner) {
                const int x = wrap_coord(f.x0 + (corner & 1), f.w);
                const int y = wrap_coord(f.y0 + (corner >> 1), f.h);
                const float w = corner_weight(&f, corner, mw[mi]);
                float *gr = g->grads + (g->mip_offset[mips[mi]] + (int64_t)y * f.w + x) * C;
                for (int c = 0; c < C; ++c) {
                    const float v = w * ntref_f16_to_f32(dinput[gi * C + c]);
                    if (atomic) {
#pragma omp atomic
                        gr[c] += v;
                    } else {
                        gr[c] += v;
                    }
                }
            }
        }
    }
}

void ntref_scatter_unconstrained(const nt_latents *lat, const float uvz[3], const uint16_t *dinput)
{
    scatter_unconstrained(lat, uvz, dinput, 0);
}

void ntref_scatter_bc6(const nt_latents *lat, const float uvz[3], const uint16_t *dinput)
{
    scatter_bc6(lat, uvz, dinput);
}

/* ---- BC6 block initialisation from unconstrained latents ----------------------------
 * No reference counterpart: the reference zero-fills its block records
 * (main.cpp:689-694) and its schedule would switch to BLOCK_FEATURES from those
 * (main.cpp:1052-1060). This is the initialisation nt_bc6_init performs. */

float ntref_bc6_value_to_y(float v)
{
    /* Inverse of the decode y -> w of train.cu:167-181: for hy >= 1 the decode is
     * w = (y/1024 - hy) 2^(hy-14) with M = y/1024 - hy in [1 + 2^-10, 2 + 2^-10); for
     * hy = 0 (y < 2049) it is linear, w = y 2^-24. With v = f 2^e (f in [0.5, 1)): M = 2f
     * at hy = e + 13, or M = 4f at hy = e + 12 when 2f < 1 + 2^-11. Values in between
     * (2f in [1 + 2^-11, 1 + 2^-10)) have no exact y and map to the start of the upper
     * range (2^-10 relative error at most). */
    if (v < 2049.f * 0x1p-24f)
        return ldexpf(v, 24);
    int e;
    const float f = frexpf(v, &e);
    const float m = ldexpf(f, 1);
    if (m >= 1.f + 0x1p-10f)
        return 1024.f * (float)(e + 13) + ldexpf(f, 11);
    if (m < 1.f + 0x1p-11f)
        return 1024.f * (float)(e + 12) + ldexpf(f, 12);
    return 1024.f * (float)(e + 13) + 1025.f;
}

float ntref_bc6_fit_subset(const float *v, const float *y, int C, int pixels, int bits, float *e0,
                           float *e1, float *x)
{
    float sum[16], lo[16], hi[16], mean[16], cov[16], d[16], t[16];
    int n = 0;
    for (int c = 0; c < C; ++c) {
        sum[c] = 0.f;
        lo[c] = INFINITY;
        hi[c] = -INFINITY;
        cov[c] = 0.f;
    }
    for (int i = 0; i < 16; ++i) {
        if (!((pixels >> i) & 1))
            continue;
        ++n;
        for (int c = 0; c < C; ++c) {
            const float yy = y[i * C + c];
            sum[c] += yy;
            lo[c] = fminf(lo[c], yy);
            hi[c] = fmaxf(hi[c], yy);
        }
    }
    if (n == 0) {
        for (int c = 0; c < C; ++c)
            e0[c] = e1[c] = 0.f;
        return 0.f;
    }
    int k = 0;
    for (int c = 0; c < C; ++c) {
        mean[c] = sum[c] / (float)n;
        if (c > 0 && hi[c] - lo[c] > hi[k] - lo[k])
            k = c;
    }
    /* Regression of every channel on channel k (the widest), then the least-squares
     * parameter of each pixel along that direction. */
    float var = 0.f;
    for (int i = 0; i < 16; ++i) {
        if (!((pixels >> i) & 1))
            continue;
        const float dk = y[i * C + k] - mean[k];
        var = fmaf(dk, dk, var);
        for (int c = 0; c < C; ++c)
            cov[c] = fmaf(y[i * C + c] - mean[c], dk, cov[c]);
    }
    float dd = 0.f;
    for (int c = 0; c < C; ++c) {
        d[c] = var > 0.f ? cov[c] / var : 0.f;
        dd = fmaf(d[c], d[c], dd);
    }
    float tlo = INFINITY, thi = -INFINITY;
    for (int i = 0; i < 16; ++i) {
        if (!((pixels >> i) & 1))
            continue;
        float s = 0.f;
        for (int c = 0; c < C; ++c)
            s = fmaf(d[c], y[i * C + c] - mean[c], s);
        t[i] = dd > 0.f ? s / dd : 0.f;
        tlo = fminf(tlo, t[i]);
        thi = fmaxf(thi, t[i]);
    }
    /* Segment ends -> endpoints: y = q0 + 8 (q1 - q0) x with x in [0, 1] (train.cu:172),
     * q = (31744 e + 32768) 2^-bits (train.cu:161-166). */
    for (int c = 0; c < C; ++c) {
        const float plo = fmaf(d[c], tlo, mean[c]), phi = fmaf(d[c], thi, mean[c]);
        const float q1 = plo + ldexpf(phi - plo, -3);
        e0[c] = (ldexpf(plo, bits) - 32768.f) / 31744.f;
        e1[c] = (ldexpf(q1, bits) - 32768.f) / 31744.f;
    }
    const float span = thi - tlo;
    float sse = 0.f;
    for (int i = 0; i < 16; ++i) {
        if (!((pixels >> i) & 1))
            continue;
        x[i] = span > 0.f ? (t[i] - tlo) / span : 0.f;
        for (int c = 0; c < C; ++c) {
            const float r = ntref_bc6_decompress(e0[c], e1[c], bits, x[i]) - v[i * C + c];
            sse = fmaf(r, r, sse);
        }
    }
    return sse;
}

void ntref_bc6_init_block(const float *v, int C, int valid, float *rec)
{
    float y[16 * 16], e[2][2][16], x[2][16];
    const int bits = ntref_bc6_partition_bits[0];
    /* The decode reaches [0, 65504] (the unsigned half range; negative values only as
     * y < 0 in its tiny linear range): the fit targets the values clamped to it. */
    float vc[16 * 16];
    for (int i = 0; i < 16 * C; ++i) {
        vc[i] = fminf(fmaxf(v[i], 0.f), 65504.f);
        y[i] = ((valid >> (i / C)) & 1) ? ntref_bc6_value_to_y(vc[i]) : 0.f;
    }
    v = vc;
    int best = 0;
    float best_sse = INFINITY;
    for (int p = 0; p < 32; ++p) {
        const int mask = ntref_bc6_partition_sets[p];
        const float s0 = ntref_bc6_fit_subset(v, y, C, valid & ~mask & 0xFFFF, bits, e[0][0], e[0][1], x[0]);
        const float s1 = ntref_bc6_fit_subset(v, y, C, valid & mask, bits, e[1][0], e[1][1], x[1]);
        float tot = s0 + s1;
        if (tot != tot)
            tot = INFINITY;
        if (p == 0 || tot < best_sse) {
            best = p;
            best_sse = tot;
        }
    }
    const int mask = ntref_bc6_partition_sets[best];
    for (int s = 0; s < 2; ++s) {
        const int pixels = valid & (s ? mask : ~mask) & 0xFFFF;
        ntref_bc6_fit_subset(v, y, C, pixels, bits, e[s][0], e[s][1], x[s]);
        for (int c = 0; c < C; ++c) {
            rec[2 * s * C + c] = e[s][0][c];
            rec[(2 * s + 1) * C + c] = e[s][1][c];
        }
    }
    for (int i = 0; i < 16; ++i) {
        const int s = (mask >> i) & 1;
        rec[4 * C + i] = ((valid >> i) & 1) ? x[s][i] : 0.f;
    }
    const int32_t part = best, mode = 0;
    memcpy(rec + 4 * C + 16, &part, 4);
    memcpy(rec + 4 * C + 17, &mode, 4);
}

int ntref_bc6_init(const nt_latents *lat)
{
    const int C = lat->channels;
    if (C < 1 || C > 16)
        return 1;
    for (int g = 0; g < lat->num_grids; ++g) {
        const nt_grid *gr = &lat->grids[g];
        if (!gr->values || !gr->block_params)
            return 2;
        for (int m = 0; m < gr->num_mips; ++m) {
            const int w = mip_dim(gr->width, m), h = mip_dim(gr->height, m);
            const int nbu = (w >> 2) > 0 ? (w >> 2) : 1, nbv = (h >> 2) > 0 ? (h >> 2) : 1;
            for (int by = 0; by < nbv; ++by)
                for (int bx = 0; bx < nbu; ++bx) {
                    float v[16 * 16];
                    int valid = 0;
                    for (int i = 0; i < 16; ++i) {
                        const int tx = 4 * bx + (i & 3), ty = 4 * by + (i >> 2);
                        const int ok = tx < w && ty < h;
                        valid |= ok << i;
                        for (int c = 0; c < C; ++c)
                            v[i * C + c] = ok ? gr->values[(gr->mip_offset[m] + (int64_t)ty * w + tx) * C + c] : 0.f;
                    }
                    float *rec = gr->block_params + (gr->block_offset[m] + (int64_t)by * nbu + bx) * (4 * C + 18);
                    ntref_bc6_init_block(v, C, valid, rec);
                }
        }
    }
    return 0;
}

/* ---- MLP (mlp.h:18-362) ------------------------------------------------------------ */

void ntref_mlp_forward_one(const nt_mlp *mlp, const uint16_t *in, uint16_t *acts,
                           uint16_t *out)
{
    uint16_t cur[MAXW], nxt[MAXW];
    memset(cur, 0, sizeof(cur));
    memcpy(cur, in, (size_t)mlp->sizes[0] * 2);
    const int L = mlp->num_layers;
    for (int l = 0; l < L; ++l) {
        const int pin = PAD16(mlp->sizes[l]), pout = PAD16(mlp->sizes[l + 1]);
        if (acts) {
            memset(acts + l * MAXW, 0, MAXW * 2);
            memcpy(acts + l * MAXW, cur, (size_t)pin * 2);
        }
        const uint16_t *W = mlp->weights[l];
        for (int n = 0; n < pout; ++n) {
            float y;
            if (g_mlp_accum_f32) {
                /* products of two fp16 values are exact in fp32 */
                float a = n < mlp->sizes[l + 1] ? ntref_f16_to_f32(mlp->biases[l][n]) : 0.f;
                for (int k = 0; k < pin; ++k)
                    a += ntref_f16_to_f32(cur[k]) * ntref_f16_to_f32(W[n * pin + k]);
                y = a;
            } else {
                double acc = n < mlp->sizes[l + 1] ? h2d(mlp->biases[l][n]) : 0.0;
                for (int k = 0; k < pin; ++k)
                    acc += h2d(cur[k]) * h2d(W[n * pin + k]);
                y = (float)acc;
            }
            if (l < L - 1 && !(y > 0.f))
                y = 0.f; /* ReLU on hidden layers (mlp.h:35-38) */
            nxt[n] = ntref_f32_to_f16(y);
        }
        memset(cur, 0, sizeof(cur));
        memcpy(cur, nxt, (size_t)pout * 2);
    }
    memcpy(out, cur, (size_t)PAD16(mlp->sizes[L]) * 2);
}

void ntref_mlp_backward_one(const nt_mlp *mlp, const uint16_t *acts, const uint16_t *dy_in,
                            double **dw, double **db, uint16_t *dinput)
{
    uint16_t dy[MAXW], dx[MAXW];
    const int L = mlp->num_layers;
    memcpy(dy, dy_in, (size_t)PAD16(mlp->sizes[L]) * 2);
    for (int l = L - 1; l >= 0; --l) {
        const int pin = PAD16(mlp->sizes[l]), pout = PAD16(mlp->sizes[l + 1]);
        const uint16_t *x = acts + l * MAXW;
        const uint16_t *W = mlp->weights[l];
        for (int n = 0; n < mlp->sizes[l + 1]; ++n) /* SumRows, mlp.h:101-153 */
            db[l][n] += h2d(dy[n]);
        for (int n = 0; n < pout; ++n) { /* outer_product, mlp.h:249-254 */
            const double d = h2d(dy[n]);
            if (d != 0.0)
                for (int k = 0; k < pin; ++k)
                    dw[l][n * pin + k] += h2d(x[k]) * d;
        }
        for (int k = 0; k < pin; ++k) { /* dY W^T, then ReLU mask (mlp.h:243-247) */
            float g;
            if (g_mlp_accum_f32) {
                float a = 0.f;
                for (int n = 0; n < pout; ++n)
                    a += ntref_f16_to_f32(W[n * pin + k]) * ntref_f16_to_f32(dy[n]);
                g = a;
            } else {
                double s = 0.0;
                for (int n = 0; n < pout; ++n)
                    s += h2d(W[n * pin + k]) * h2d(dy[n]);
                g = (float)s;
            }
            if (l > 0 && !(ntref_f16_to_f32(x[k]) > 0.f))
                g = 0.f;
            dx[k] = ntref_f32_to_f16(g);
        }
        memcpy(dy, dx, (size_t)pin * 2);
    }
    memcpy(dinput, dy, (size_t)mlp->sizes[0] * 2);
}

static int mlp_valid(const nt_mlp *m)
{
    if (m->num_layers < 1 || m->num_layers > NT_MAX_LAYERS)
        return 0;
    for (int l = 0; l <= m->num_layers; ++l)
        if (m->sizes[l] < 1 || PAD16(m->sizes[l]) > MAXW)
            return 0;
    return m->sizes[m->num_layers] <= NT_MAX_OUTPUTS;
}

/* ---- passes ------------------------------------------------------------------------ */

static void sample_features(const nt_params *p, int type, const float uvz[3], uint16_t *f)
{
    if (type == NT_UNCONSTRAINED)
        ntref_sample_latents_bilinear(&p->latents, uvz, f);
    else
        ntref_sample_latents_bc6(&p->latents, uvz, f);
}

/* Loss gradient, train.cu:876-888: dL/dy = fp16(2 w (y - t) / N). */
static void loss_gradient(const nt_params *p, const uint16_t *out, const float *expected,
                          const float *weights, uint16_t *dy)
{
    const int pout = PAD16(p->mlp.sizes[p->mlp.num_layers]);
    for (int n = 0; n < pout; ++n) {
        const float err = ntref_f16_to_f32(out[n]) - expected[n];
        dy[n] = ntref_f32_to_f16(2.f * weights[n] * err / (float)p->num_samples);
    }
}

int ntref_train_intermediates(const nt_params *p, int type, uint16_t *features, uint16_t *dy,
                              float *target)
{
    if (!mlp_valid(&p->mlp))
        return NT_ERR_INVALID_ARGUMENT;
    const int F = p->latents.num_grids * p->latents.channels;
    for (int i = 0; i < p->num_samples; ++i) {
        float uvz[3], expected[16], weights[16];
        uint16_t f[MAXW], acts[NT_MAX_LAYERS * MAXW], out[16], d[16];
        ntref_sample_uvz(p, (uint32_t)i, uvz);
        sample_features(p, type, uvz, f);
        ntref_expected_values(p, uvz, expected, weights);
        ntref_mlp_forward_one(&p->mlp, f, acts, out);
        loss_gradient(p, out, expected, weights, d);
        if (features)
            memcpy(features + (size_t)i * F, f, (size_t)F * 2);
        if (dy)
            memcpy(dy + (size_t)i * 16, d, sizeof(d));
        if (target)
            memcpy(target + (size_t)i * 16, expected, sizeof(expected));
    }
    return NT_OK;
}

/* With this switch on, ntref_train_step rounds each warp's weight-gradient partial (the sum
 * over its 32 consecutive samples of x (x) dy) to fp16 before adding it to the total, as the
 * reference keeps the warp's outer product as __half2 registers before the fp32 atomics
 * (mlp.h:166-173, 249-254). How tcnn accumulates inside the outer product is not visible in
 * the reference; the partial is taken exactly and rounded once. Off (the default), the
 * partials are summed in double. Bias gradients are fp32 sums of fp16 dy in both modes
 * (SumRows, mlp.h:101-153). */
static int g_dw_partial_fp16 = 0;

void ntref_set_dw_partial_fp16(int on)
{
    g_dw_partial_fp16 = on != 0;
}

int ntref_train_step(const nt_params *p, int type, int num_threads)
{
    if (!mlp_valid(&p->mlp) || p->num_samples <= 0)
        return NT_ERR_INVALID_ARGUMENT;
    const nt_mlp *m = &p->mlp;
    const int L = m->num_layers;
    int nt = num_threads > 0 ? num_threads : 1;
#ifndef _OPENMP
    nt = 1;
#endif
    size_t per = 0;
    size_t off_w[NT_MAX_LAYERS], off_b[NT_MAX_LAYERS];
    for (int l = 0; l < L; ++l) {
        off_w[l] = per;
        per += (size_t)PAD16(m->sizes[l]) * PAD16(m->sizes[l + 1]);
        off_b[l] = per;
        per += (size_t)PAD16(m->sizes[l + 1]);
    }
    double *acc = (double *)calloc(per * (size_t)nt, sizeof(double));
    if (!acc)
        return NT_ERR_INVALID_ARGUMENT;

#pragma omp parallel num_threads(nt) if (nt > 1)
    {
        int tid = 0;
#ifdef _OPENMP
        tid = omp_get_thread_num();
#endif
        double *dw[NT_MAX_LAYERS], *db[NT_MAX_LAYERS], *wdw[NT_MAX_LAYERS];
        /* warp partials of the weight gradients, when they are rounded to fp16 */
        double *wbuf = g_dw_partial_fp16 ? (double *)malloc(per * sizeof(double)) : NULL;
        for (int l = 0; l < L; ++l) {
            dw[l] = acc + per * (size_t)tid + off_w[l];
            db[l] = acc + per * (size_t)tid + off_b[l];
            wdw[l] = wbuf ? wbuf + off_w[l] : dw[l];
        }
        const int nwarp = (p->num_samples + 31) / 32;
#pragma omp for schedule(static)
        for (int w = 0; w < nwarp; ++w) {
            if (wbuf)
                memset(wbuf, 0, per * sizeof(double));
            const int i1 = 32 * w + 32 < p->num_samples ? 32 * w + 32 : p->num_samples;
            for (int i = 32 * w; i < i1; ++i) {
                float uvz[3], expected[16], weights[16];
                uint16_t f[MAXW], acts[NT_MAX_LAYERS * MAXW], out[16], dy[16], din[MAXW];
                ntref_sample_uvz(p, (uint32_t)i, uvz);
                sample_features(p, type, uvz, f);
                ntref_expected_values(p, uvz, expected, weights);
                ntref_mlp_forward_one(m, f, acts, out);
                loss_gradient(p, out, expected, weights, dy);
                ntref_mlp_backward_one(m, acts, dy, wdw, db, din);
                if (type == NT_UNCONSTRAINED) {
                    scatter_unconstrained(&p->latents, uvz, din, nt > 1);
                } else if (type == NT_BLOCK_FEATURES) {
                    if (nt > 1) {
#pragma omp critical
                        scatter_bc6(&p->latents, uvz, din);
                    } else {
                        scatter_bc6(&p->latents, uvz, din);
                    }
                }
            }
            if (wbuf)
                for (int l = 0; l < L; ++l) {
                    const size_t nw = (size_t)PAD16(m->sizes[l]) * PAD16(m->sizes[l + 1]);
                    for (size_t k = 0; k < nw; ++k)
                        dw[l][k] += h2d(f64_to_f16(wdw[l][k]));
                }
        }
        free(wbuf);
    }
    for (int t = 1; t < nt; ++t)
        for (size_t i = 0; i < per; ++i)
            acc[i] += acc[per * (size_t)t + i];
    for (int l = 0; l < L; ++l) {
        const size_t nw = (size_t)PAD16(m->sizes[l]) * PAD16(m->sizes[l + 1]);
        for (size_t i = 0; i < nw; ++i)
            m->weight_grads[l][i] = (float)((double)m->weight_grads[l][i] + acc[off_w[l] + i]);
        for (int i = 0; i < m->sizes[l + 1]; ++i)
            m->bias_grads[l][i] = (float)((double)m->bias_grads[l][i] + acc[off_b[l] + i]);
    }
    free(acc);
    return NT_OK;
}

/* ---- Adam (train.cu:521-816) ------------------------------------------------------ */

typedef struct {
    nt_adam a;
    float bc1, bc2;
} adam_step;

static adam_step make_adam(const nt_adam *a, int step)
{
    adam_step s;
    s.a = *a;
    const int t = step > 0 ? step : 1;
    s.bc1 = 1.f - powf(a->beta1, (float)t);
    s.bc2 = 1.f - powf(a->beta2, (float)t);
    return s;
}

/* AdamUpdateFloatParameter (train.cu:545-564); returns the new weight. */
static float adam_update(float *m1, float *m2, float g, const adam_step *s, float w)
{
    *m1 = fmaf(s->a.beta1, *m1, (1.f - s->a.beta1) * g);
    *m2 = fmaf(s->a.beta2, *m2, (1.f - s->a.beta2) * g * g);
    const float mhat = *m1 / s->bc1;
    const float vhat = *m2 / s->bc2;
    return w - s->a.learning_rate * mhat / (sqrtf(vhat) + s->a.epsilon);
}

/* Lazy update of one fp32 scalar (OptimizeFeatureScalar, train.cu:625-639). */
static void lazy_f32(float *w, float *g, float *m1, float *m2, const adam_step *s)
{
    if (*g == 0.f)
        return;
    *w = adam_update(m1, m2, *g, s, *w);
    *g = 0.f;
}

/* Lazy update of one fp16 parameter (AdamUpdateParameter, train.cu:521-543). */
static void lazy_f16(uint16_t *w, float *g, float *m1, float *m2, const adam_step *s)
{
    if (*g == 0.f)
        return;
    *w = ntref_f32_to_f16(adam_update(m1, m2, *g, s, ntref_f16_to_f32(*w)));
    *g = 0.f;
}

int ntref_optimize_network(const nt_params *p)
{
    const nt_mlp *m = &p->mlp;
    if (!mlp_valid(m))
        return NT_ERR_INVALID_ARGUMENT;
    const adam_step s = make_adam(&p->network_adam, p->step);
    for (int l = 0; l < m->num_layers; ++l) {
        const int rows = m->sizes[l], pin = PAD16(m->sizes[l]);
        const int cols = l == m->num_layers - 1 ? m->used_outputs : m->sizes[l + 1];
        for (int col = 0; col < cols; ++col) /* train.cu:590-623 */
            for (int row = 0; row < rows; ++row) {
                const int i = col * pin + row;
                lazy_f16(&m->weights[l][i], &m->weight_grads[l][i], &m->weight_moment1[l][i],
                         &m->weight_moment2[l][i], &s);
            }
        for (int i = 0; i < m->sizes[l + 1]; ++i) /* train.cu:566-588 */
            lazy_f16(&m->biases[l][i], &m->bias_grads[l][i], &m->bias_moment1[l][i],
                     &m->bias_moment2[l][i], &s);
    }
    return NT_OK;
}

int ntref_optimize_latents(const nt_params *p, int type)
{
    const nt_latents *lat = &p->latents;
    const int C = lat->channels;
    const adam_step s = make_adam(&p->feature_adam, p->step);
    for (int gi = 0; gi < lat->num_grids; ++gi) {
        const nt_grid *g = &lat->grids[gi];
        for (int mip = 0; mip < g->num_mips; ++mip) {
            const int w = mip_dim(g->width, mip), h = mip_dim(g->height, mip);
            if (type == NT_UNCONSTRAINED) { /* train.cu:764-803 */
                const int64_t base = g->mip_offset[mip] * C;
                const int64_t n = (int64_t)w * h * C;
                for (int64_t i = base; i < base + n; ++i)
                    lazy_f32(&g->values[i], &g->grads[i], &g->moment1[i], &g->moment2[i], &s);
            } else { /* train.cu:641-679, 728-762 */
                const int nb = ((w >> 2) > 0 ? (w >> 2) : 1) * ((h >> 2) > 0 ? (h >> 2) : 1);
                const int stride = 4 * C + 16;
                for (int b = 0; b < nb; ++b) {
                    const int64_t blk = g->block_offset[mip] + b;
                    float *pr = g->block_params + blk * (stride + 2);
                    float *gr = g->block_grads + blk * stride;
                    float *m1 = g->block_moment1 + blk * stride;
                    float *m2 = g->block_moment2 + blk * stride;
                    for (int i = 0; i < stride; ++i)
                        lazy_f32(&pr[i], &gr[i], &m1[i], &m2[i], &s);
                }
            }
        }
    }
    return NT_OK;
}

int ntref_inference(const nt_params *p)
{
    if (!mlp_valid(&p->mlp) || !p->inference_output || !p->inference_mse_accum)
        return NT_ERR_INVALID_ARGUMENT;
    const int W = p->image_width, H = p->image_height;
    const int no = p->mlp.sizes[p->mlp.num_layers];
    double sse_total = 0.0;
    for (int64_t i = 0; i < (int64_t)W * H; ++i) { /* train.cu:917-961 */
        const int x = (int)(i % W), y = (int)(i / W);
        const float uvz[3] = {((float)x + 0.5f) / (float)W, ((float)y + 0.5f) / (float)H, 0.f};
        uint16_t f[MAXW], out[16];
        float expected[16];
        ntref_sample_latents_bilinear(&p->latents, uvz, f);
        ntref_expected_values(p, uvz, expected, NULL);
        ntref_mlp_forward_one(&p->mlp, f, NULL, out);
        float sse = 0.f;
        for (int c = 0; c < no; ++c) {
            const float o = ntref_f16_to_f32(out[c]);
            p->inference_output[i * no + c] = o;
            const float e = o - expected[c];
            sse = fmaf(e, e, sse);
        }
        sse_total += sse;
    }
    *p->inference_mse_accum = (float)((double)*p->inference_mse_accum + sse_total);
    return NT_OK;
}

int ntref_mlp_forward(const nt_mlp *mlp, const uint16_t *inputs, uint16_t *outputs, int count)
{
    if (!mlp_valid(mlp))
        return NT_ERR_INVALID_ARGUMENT;
    const int in = mlp->sizes[0], no = mlp->sizes[mlp->num_layers];
    for (int i = 0; i < count; ++i) {
        uint16_t out[16];
        ntref_mlp_forward_one(mlp, inputs + (size_t)i * in, NULL, out);
        memcpy(outputs + (size_t)i * no, out, (size_t)no * 2);
    }
    return NT_OK;
}

int ntref_forward(const nt_latents *lat, const nt_mlp *mlp, int filter, const float *uvz,
                  int count, uint16_t *features, uint16_t *outputs)
{
    if (!mlp_valid(mlp))
        return NT_ERR_INVALID_ARGUMENT;
    const int F = lat->num_grids * lat->channels, no = mlp->sizes[mlp->num_layers];
    for (int i = 0; i < count; ++i) {
        uint16_t f[MAXW], out[16];
        if (filter == NT_FILTER_CATMULL_ROM)
            ntref_sample_latents_catmull_rom(lat, uvz + 3 * (size_t)i, f);
        else
            ntref_sample_latents_bilinear(lat, uvz + 3 * (size_t)i, f);
        ntref_mlp_forward_one(mlp, f, NULL, out);
        if (features)
            memcpy(features + (size_t)i * F, f, (size_t)F * 2);
        memcpy(outputs + (size_t)i * no, out, (size_t)no * 2);
    }
    return NT_OK;
}

/* ---- block codec (the build's own format; no reference counterpart) ---------------- */

/* BC6H 4-bit interpolation weights (public BC6H/BC7 specification). */
static const int kCodecWeights[16] = {0, 4, 9, 13, 17, 21, 26, 30, 34, 38, 43, 47, 51, 55, 60, 64};

uint16_t ntref_codec_key(uint16_t h)
{
    return (h & 0x8000u) ? (uint16_t)~h : (uint16_t)(h | 0x8000u);
}

uint16_t ntref_codec_unkey(uint16_t k)
{
    return (k & 0x8000u) ? (uint16_t)(k & 0x7FFFu) : (uint16_t)~k;
}

uint16_t ntref_codec_interp(uint16_t k0, uint16_t k1, int i)
{
    const int w = kCodecWeights[i & 15];
    return (uint16_t)(((uint32_t)k0 * (uint32_t)(64 - w) + (uint32_t)k1 * (uint32_t)w + 32u) >> 6);
}

static float codec_clamp(float v) { return fminf(fmaxf(v, -65504.f), 65504.f); }

int ntref_codec_encode(const float *values, int width, int height, int channels,
                       uint8_t *blocks)
{
    if (width <= 0 || height <= 0 || channels <= 0 || channels % 4 || channels > 16)
        return NT_ERR_INVALID_ARGUMENT;
    const int C = channels, bw = (width + 3) / 4, bh = (height + 3) / 4;
    const size_t rec = (size_t)12 * C;
    /* blocks are independent: the result does not depend on the thread count */
#pragma omp parallel for schedule(static)
    for (int by = 0; by < bh; ++by)
        for (int bx = 0; bx < bw; ++bx) {
            uint8_t *r = blocks + ((size_t)by * bw + bx) * rec;
            memset(r, 0, rec);
            uint16_t *ends = (uint16_t *)r;
            for (int c = 0; c < C; ++c) {
                uint16_t kmin = 0xFFFF, kmax = 0;
                for (int p = 0; p < 16; ++p) {
                    const int x = bx * 4 + (p & 3), y = by * 4 + (p >> 2);
                    if (x >= width || y >= height)
                        continue;
                    const float v = codec_clamp(values[((size_t)y * width + x) * C + c]);
                    const uint16_t k = ntref_codec_key(ntref_f32_to_f16(v));
                    kmin = k < kmin ? k : kmin;
                    kmax = k > kmax ? k : kmax;
                }
                ends[2 * c] = kmin;
                ends[2 * c + 1] = kmax;
                for (int p = 0; p < 16; ++p) {
                    const int x = bx * 4 + (p & 3), y = by * 4 + (p >> 2);
                    if (x >= width || y >= height)
                        continue;
                    const float v = codec_clamp(values[((size_t)y * width + x) * C + c]);
                    int best = 0;
                    float best_err = INFINITY;
                    for (int i = 0; i < 16; ++i) {
                        const float d =
                            ntref_f16_to_f32(ntref_codec_unkey(ntref_codec_interp(kmin, kmax, i)));
                        const float err = fabsf(v - d);
                        if (err < best_err) {
                            best_err = err;
                            best = i;
                        }
                    }
                    r[4 * C + p * (C / 2) + c / 2] |= (uint8_t)(best << ((c & 1) * 4));
                }
            }
        }
    return NT_OK;
}

static float codec_texel(const uint8_t *rec, int C, int pix, int c)
{
    const uint16_t *ends = (const uint16_t *)rec;
    const int idx = (rec[4 * C + pix * (C / 2) + c / 2] >> ((c & 1) * 4)) & 15;
    return ntref_f16_to_f32(ntref_codec_unkey(ntref_codec_interp(ends[2 * c], ends[2 * c + 1], idx)));
}

int ntref_codec_decode(const uint8_t *blocks, int width, int height, int channels,
                       float *values)
{
    if (width <= 0 || height <= 0 || channels <= 0 || channels % 4 || channels > 16)
        return NT_ERR_INVALID_ARGUMENT;
    const int C = channels, bw = (width + 3) / 4;
#pragma omp parallel for schedule(static)
    for (int y = 0; y < height; ++y)
        for (int x = 0; x < width; ++x) {
            const uint8_t *r = blocks + ((size_t)(y >> 2) * bw + (x >> 2)) * 12 * C;
            const int pix = ((y & 3) << 2) + (x & 3);
            for (int c = 0; c < C; ++c)
                values[((size_t)y * width + x) * C + c] = codec_texel(r, C, pix, c);
        }
    return NT_OK;
}

void ntref_set_threads(int n)
{
#ifdef _OPENMP
    omp_set_num_threads(n > 0 ? n : 1);
#else
    (void)n;
#endif
}

int ntref_decode(const nt_decode_params *p, int num_threads)
{
    return ntref_decode_rect(p, 0, 0, p->out_width, p->out_height, num_threads);
}

int ntref_decode_rect(const nt_decode_params *p, int x0, int y0, int rw, int rh, int num_threads)
{
    if (!mlp_valid(&p->mlp) || p->channels % 4 || p->num_grids < 1)
        return NT_ERR_INVALID_ARGUMENT;
    const int W = p->out_width, H = p->out_height, C = p->channels;
    const int no = p->mlp.used_outputs;
    if (x0 < 0 || y0 < 0 || rw < 0 || rh < 0 || x0 + rw > W || y0 + rh > H)
        return NT_ERR_INVALID_ARGUMENT;
    const int64_t n = (int64_t)rw * rh;
    (void)num_threads;
#pragma omp parallel for schedule(static) num_threads(num_threads > 0 ? num_threads : 1)
    for (int64_t k = 0; k < n; ++k) {
        /* pixel i of the full image; its output goes to row-major position k of the rectangle */
        const int px = x0 + (int)(k % rw), py = y0 + (int)(k / rw);
        const int64_t i = (int64_t)py * W + px;
        uint32_t st = (uint32_t)i ^ (p->seed * 747796405u + 2891336453u);
        st = st ? st : 1u;
        const float jx = ntref_uniform(&st) - 0.5f;
        const float jy = ntref_uniform(&st) - 0.5f;
        const float zu = ntref_uniform(&st);
        const float posx = clampf(fmaf(p->jitter, jx, (float)px + 0.5f), 0.5f, (float)W - 0.5f);
        const float posy = clampf(fmaf(p->jitter, jy, (float)py + 0.5f), 0.5f, (float)H - 0.5f);
        const float u = posx / (float)W, v = posy / (float)H;
        const float z = fmaf(p->mip_max - p->mip_min, zu, p->mip_min);
        uint16_t f[MAXW], out[16];
        for (int k = 0; k < p->num_grids * C; ++k)
            f[k] = 0;
        for (int gi = 0; gi < p->num_grids; ++gi) {
            const nt_codec_grid *g = &p->grids[gi];
            nt_grid tmp;
            tmp.num_mips = g->num_mips;
            int mips[2];
            float mw[2];
            const int nm = mip_pair(&tmp, z, mips, mw);
            for (int mi = 0; mi < nm; ++mi) {
                const footprint fp = make_footprint(g->width, g->height, mips[mi], u, v);
                const int bw = (fp.w + 3) / 4;
                const uint8_t *base = (const uint8_t *)g->blocks + g->byte_offset[mips[mi]];
                for (int corner = 0; corner < 4; ++corner) {
                    const int x = wrap_coord(fp.x0 + (corner & 1), fp.w);
                    const int y = wrap_coord(fp.y0 + (corner >> 1), fp.h);
                    const float w = corner_weight(&fp, corner, mw[mi]);
                    const uint8_t *r = base + ((size_t)(y >> 2) * bw + (x >> 2)) * 12 * C;
                    const int pix = ((y & 3) << 2) + (x & 3);
                    for (int c = 0; c < C; ++c)
                        f[gi * C + c] = ntref_f16_add(
                            f[gi * C + c], ntref_f32_to_f16(w * codec_texel(r, C, pix, c)));
                }
            }
        }
        ntref_mlp_forward_one(&p->mlp, f, NULL, out);
        for (int c = 0; c < no; ++c)
            p->output[k * no + c] = out[c];
    }
    return NT_OK;
}
