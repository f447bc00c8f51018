// nt_bc6.hip — BC6 block initialisation from unconstrained latents (nt_bc6_init).
//
// The reference zero-fills its BC6 block records (main.cpp:689-694); its schedule's
// BLOCK_FEATURES phase (main.cpp:1052-1060) would start from those. This kernel instead
// fits every 4x4 block of every mip to the unconstrained latents trained so far, through
// the reference's own BC6 decode (train.cu:159-181): values, clamped to the decode's
// range [0, 65504], are mapped to its linear "y" domain, each of the 32 two-subset
// partitions (train.cu:20-29) is tried with a
// line fit per subset, and the partition whose record decodes with the least squared
// error is written (mode 0: 10-bit endpoints; pixel indices in [0, 1]).
//
// One wave per block: lane p + 32 s fits subset s of partition p, the two halves add
// their errors with one shuffle and an argmin over the 32 partitions (ties to the lowest)
// picks the record; the two winning lanes write it. Every operation and its order match
// the oracle's restatement, so records are bit-identical to it.
#include "nt_internal.hpp"

namespace ntk {

// y whose BC6 decode is v (2^-10 relative at most): the decode is w = (y/1024 - hy)
// 2^(hy-14) with M = y/1024 - hy in [1 + 2^-10, 2 + 2^-10) for hy >= 1, and w = y 2^-24
// for y < 2049 (hy = 0).
__device__ __forceinline__ float bc6_value_to_y(float v)
{
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

// Line fit of the pixels in `pixels` (a 16-bit mask) of a block v / y [16][C] in LDS:
// regression of every channel on the widest one, least-squares pixel parameters, the
// segment's ends as endpoints. Returns the decoded squared error.
template <int C>
__device__ __forceinline__ float bc6_fit_subset(const float *v, const float *y, int pixels, int bits,
                                                float (&e0)[C], float (&e1)[C], float (&x)[16])
{
    float sum[C], lo[C], hi[C], mean[C], cov[C], d[C], t[16];
    int n = 0;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        sum[c] = 0.f;
        lo[c] = INFINITY;
        hi[c] = -INFINITY;
        cov[c] = 0.f;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if ((pixels >> i) & 1) {
            ++n;
#pragma unroll
            for (int c = 0; c < C; ++c) {
                const float yy = y[i * C + c];
                sum[c] += yy;
                lo[c] = fminf(lo[c], yy);
                hi[c] = fmaxf(hi[c], yy);
            }
        }
    }
    if (n == 0) {
#pragma unroll
        for (int c = 0; c < C; ++c)
            e0[c] = e1[c] = 0.f;
        return 0.f;
    }
    int k = 0;
    float rk = hi[0] - lo[0], mk = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        mean[c] = sum[c] / (float)n;
        const float r = hi[c] - lo[c];
        if (c > 0 && r > rk) {
            k = c;
            rk = r;
        }
    }
#pragma unroll
    for (int c = 0; c < C; ++c)
        mk = c == k ? mean[c] : mk;
    float var = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if ((pixels >> i) & 1) {
            const float dk = y[i * C + k] - mk;
            var = fmaf(dk, dk, var);
#pragma unroll
            for (int c = 0; c < C; ++c)
                cov[c] = fmaf(y[i * C + c] - mean[c], dk, cov[c]);
        }
    }
    float dd = 0.f;
#pragma unroll
    for (int c = 0; c < C; ++c) {
        d[c] = var > 0.f ? cov[c] / var : 0.f;
        dd = fmaf(d[c], d[c], dd);
    }
    float tlo = INFINITY, thi = -INFINITY;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        t[i] = 0.f;
        if ((pixels >> i) & 1) {
            float s = 0.f;
#pragma unroll
            for (int c = 0; c < C; ++c)
                s = fmaf(d[c], y[i * C + c] - mean[c], s);
            t[i] = dd > 0.f ? s / dd : 0.f;
            tlo = fminf(tlo, t[i]);
            thi = fmaxf(thi, t[i]);
        }
    }
    // y = q0 + 8 (q1 - q0) x, x in [0, 1] (train.cu:172); q = (31744 e + 32768) 2^-bits.
#pragma unroll
    for (int c = 0; c < C; ++c) {
        const float plo = fmaf(d[c], tlo, mean[c]), phi = fmaf(d[c], thi, mean[c]);
        const float q1 = plo + ldexpf(phi - plo, -3);
        e0[c] = (ldexpf(plo, bits) - 32768.f) / 31744.f;
        e1[c] = (ldexpf(q1, bits) - 32768.f) / 31744.f;
    }
    const float span = thi - tlo;
    float sse = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        x[i] = 0.f;
        if ((pixels >> i) & 1) {
            x[i] = span > 0.f ? (t[i] - tlo) / span : 0.f;
#pragma unroll
            for (int c = 0; c < C; ++c) {
                const float r = bc6_decompress(e0[c], e1[c], bits, x[i]) - v[i * C + c];
                sse = fmaf(r, r, sse);
            }
        }
    }
    return sse;
}

template <int C>
__global__ __launch_bounds__(256) void bc6_init_kernel(Bc6InitDesc d)
{
    __shared__ float sv[4][16 * C], sy[4][16 * C];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * 4 + wave;
    const bool active = b < d.start[d.levels];
    int lev = 0;
    while (active && lev + 1 < d.levels && b >= d.start[lev + 1])
        ++lev;
    const int64_t local = active ? b - d.start[lev] : 0;
    const int nbu = d.nbu[lev], w = d.w[lev], h = d.h[lev];
    const int bx = (int)(local % nbu), by = (int)(local / nbu);
    int valid = 0;
#pragma unroll
    for (int i = 0; i < 16; ++i)
        valid |= (4 * bx + (i & 3) < w && 4 * by + (i >> 2) < h) ? 1 << i : 0;
    if (active) {
        const float *vals = d.values[lev];
        for (int idx = lane; idx < 16 * C; idx += 64) {
            const int i = idx / C, c = idx % C;
            const int tx = 4 * bx + (i & 3), ty = 4 * by + (i >> 2);
            const bool ok = (valid >> i) & 1;
            // Target range of the decode: [0, 65504] (unsigned half).
            const float v = ok ? fminf(fmaxf(vals[((int64_t)ty * w + tx) * C + c], 0.f), 65504.f) : 0.f;
            sv[wave][idx] = v;
            sy[wave][idx] = ok ? bc6_value_to_y(v) : 0.f;
        }
    }
    __syncthreads();
    if (!active)
        return;
    constexpr int kBits = 10; // mode 0
    const int p = lane & 31, s = lane >> 5, mask = bc6_partition_mask(p);
    const int pixels = valid & (s ? mask : ~mask) & 0xFFFF;
    float e0[C], e1[C], x[16];
    const float sse = bc6_fit_subset<C>(sv[wave], sy[wave], pixels, kBits, e0, e1, x);
    float tot = sse + __shfl_xor(sse, 32);
    if (tot != tot)
        tot = INFINITY;
    float bt = tot;
    int bp = p;
#pragma unroll
    for (int off = 16; off >= 1; off >>= 1) {
        const float ot = __shfl_xor(bt, off);
        const int op = __shfl_xor(bp, off);
        if (ot < bt || (ot == bt && op < bp)) {
            bt = ot;
            bp = op;
        }
    }
    if (p != bp)
        return;
    float *rec = d.blocks[lev] + local * (4 * C + 18);
#pragma unroll
    for (int c = 0; c < C; ++c) {
        rec[2 * s * C + c] = e0[c];
        rec[(2 * s + 1) * C + c] = e1[c];
    }
#pragma unroll
    for (int i = 0; i < 16; ++i)
        if (((mask >> i) & 1) == s)
            rec[4 * C + i] = ((valid >> i) & 1) ? x[i] : 0.f;
    if (s == 0) {
        rec[4 * C + 16] = __int_as_float(p);
        rec[4 * C + 17] = __int_as_float(0);
    }
}

hipError_t launch_bc6_init(const Bc6InitDesc &d, hipStream_t s)
{
    const int64_t blocks = d.start[d.levels];
    if (blocks <= 0)
        return hipSuccess;
    const dim3 grid((unsigned)((blocks + 3) / 4));
    switch (d.C) {
    case 3:
        hipLaunchKernelGGL(bc6_init_kernel<3>, grid, dim3(256), 0, s, d);
        break;
    case 4:
        hipLaunchKernelGGL(bc6_init_kernel<4>, grid, dim3(256), 0, s, d);
        break;
    case 8:
        hipLaunchKernelGGL(bc6_init_kernel<8>, grid, dim3(256), 0, s, d);
        break;
    case 16:
        hipLaunchKernelGGL(bc6_init_kernel<16>, grid, dim3(256), 0, s, d);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

// ---- the BC6 block phase on the fused train kernel ------------------------------------

// The level of a launch-wide block number (levels take consecutive ranges of blocks).
__device__ __forceinline__ int bc6_phase_level(const Bc6PhaseDesc &d, int64_t b)
{
    int li = 0;
#pragma unroll
    for (int k = 1; k < 2 * NT_MAX_GRIDS; ++k)
        if (k < d.nlevels && b >= d.level[k].first_block)
            li = k;
    return li;
}

__device__ __forceinline__ int wrap_mod(int v, int n)
{
    const int r = v % n;
    return r < 0 ? r + n : r;
}

// Block (column, row) of block lb of a level's rectangle, wrapped into the level: the row by
// a float reciprocal and one correction step (exact for rows below 2^16, which the level's
// block rows are), the wrap by one compare each way (a rectangle narrower than the level
// starts at most one block outside it; wrap_mod for anything else).
__device__ __forceinline__ void bc6_block_of(const Bc6PhaseLevel &g, int lb, int &bx, int &by)
{
    int ry = (int)((float)lb * __builtin_amdgcn_rcpf((float)g.nbx));
    int rx = lb - ry * g.nbx;
    if (rx < 0) {
        ry -= 1;
        rx += g.nbx;
    } else if (rx >= g.nbx) {
        ry += 1;
        rx -= g.nbx;
    }
    bx = g.bx0 + rx;
    by = g.by0 + ry;
    bx = bx < 0 ? bx + g.nbu : (bx >= g.nbu ? bx - g.nbu : bx);
    by = by < 0 ? by + g.nbv : (by >= g.nbv ? by - g.nbv : by);
    if ((unsigned)bx >= (unsigned)g.nbu || (unsigned)by >= (unsigned)g.nbv) {
        bx = wrap_mod(g.bx0 + rx, g.nbu);
        by = wrap_mod(g.by0 + ry, g.nbv);
    }
}

// A block record's fields a pixel thread needs, all loads issued at once (the partition
// picks the endpoints afterwards): the four endpoints of every channel, the pixel's index
// on the segment, the partition and the mode.
template <int C>
struct Bc6Pixel {
    float q0[C], q1[C]; // the pixel's partition's endpoints, unquantized
    float xi;
    int part, bits;
};
template <int C>
__device__ __forceinline__ Bc6Pixel<C> bc6_pixel(const float *rec, int pix)
{
    float e[4][C];
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int ch = 0; ch < C; ++ch)
            e[k][ch] = rec[k * C + ch];
    Bc6Pixel<C> q;
    q.xi = rec[4 * C + pix];
    const int partition = __float_as_int(rec[4 * C + 16]);
    q.bits = bc6_mode_bits(__float_as_int(rec[4 * C + 17]));
    q.part = (bc6_partition_mask(partition) >> pix) & 1;
#pragma unroll
    for (int ch = 0; ch < C; ++ch) {
        q.q0[ch] = bc6_unquantize(q.part ? e[2][ch] : e[0][ch], q.bits);
        q.q1[ch] = bc6_unquantize(q.part ? e[3][ch] : e[1][ch], q.bits);
    }
    return q;
}

// Expansion: one thread per texel of a block rectangle, numbered block by block and, in a
// block, row-major, so that 16 consecutive threads share one record. Each texel's C values are the
// reference's BC6 decode of its block (train.cu:240-261, DecompressBC6 :169-182), the same
// arithmetic as the per-sample gather (bc6_decompress); its gradients are cleared.
template <int C>
__global__ __launch_bounds__(256) void bc6_expand_kernel(Bc6PhaseDesc d)
{
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = t >> 4;
    if (b >= d.total_blocks)
        return;
    const Bc6PhaseLevel &g = d.level[bc6_phase_level(d, b)];
    // A level's rectangle holds fewer than 2^31 blocks (its texels fit 32-bit offsets).
    const int lb = (int)(b - g.first_block);
    int bx, by;
    bc6_block_of(g, lb, bx, by);
    const int pix = (int)(t & 15);
    const int x = 4 * bx + (pix & 3), y = 4 * by + (pix >> 2);
    if (x >= g.w || y >= g.h)
        return; // a level narrower than a block (w or h < 4)
    const Bc6Pixel<C> q = bc6_pixel<C>(g.params + ((int64_t)by * g.nbu + bx) * (4 * C + 18), pix);
    const int64_t o = ((int64_t)y * g.w + x) * C;
#pragma unroll
    for (int ch = 0; ch < C; ++ch) {
        const float yv = bc6_y(q.q0[ch], q.q1[ch], q.xi);
        const int hy = bc6_hy(yv);
        g.values[o + ch] = ldexpf(yv / 1024.f - (float)hy, hy - 14);
        g.tgrads[o + ch] = 0.f;
    }
}

// Fold: one thread per texel of the block rectangle, as the expansion. The reference adds,
// for every corner that lands on texel (pixel p) of a block, with feature gradient w * g per
// channel (train.cu:405-455):
//   dl_dy = ldexp(w g, hy - 24),   hy from y = q0 + 8 (q1 - q0) x_p  (that texel's channel)
//   pixel index p:    += sum_ch dl_dy * 8 (q1 - q0)
//   endpoints of p's partition, channel ch:  e0 += (1 - 8 x_p) (31/64) 2^(16 - bits) dl_dy,
//                                            e1 += 8 x_p (31/64) 2^(16 - bits) dl_dy.
// Every factor but w g depends on the texel and channel only, and ldexp by an integer is
// exact, so the sums over corners equal these terms applied to the texel's gradient
// G = sum w g (which the fused kernel accumulated) up to the order of the fp32 additions
// (which the reference's atomics leave open as well). The pixel thread adds its pixel-index
// gradient; the endpoint terms are summed over the block's 16 threads with lane shuffles
// and added by its first thread. Texels with a zero gradient add nothing; each record field
// is read, added to and written by one thread only.
template <int C>
__global__ __launch_bounds__(256) void bc6_fold_kernel(Bc6PhaseDesc d)
{
    // NT_LATENT_TOUCHED: one thread logs the step (the protocol of the fused kernel's texel
    // log) and, for the first step since the optimizer ran, its block rectangles.
    if (d.log && blockIdx.x == 0 && threadIdx.x == 0) {
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
            log->kind = kUpdateLogBlocks;
            for (int gi = 0; gi < NT_MAX_GRIDS; ++gi)
                for (int k = 0; k < 4; ++k)
                    log->rect[gi][k] = d.rect[gi][k];
        }
    }
    // The 16 threads of a block are 16 consecutive lanes of one wave (the launch covers
    // whole blocks), so every cross-lane sum below stays within the block's lanes, and
    // a block's lanes leave only together.
    const int64_t t = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int64_t b = t >> 4;
    if (b >= d.total_blocks)
        return;
    const Bc6PhaseLevel &g = d.level[bc6_phase_level(d, b)];
    // A level's rectangle holds fewer than 2^31 blocks (its texels fit 32-bit offsets).
    const int lb = (int)(b - g.first_block);
    int bx, by;
    bc6_block_of(g, lb, bx, by);
    const int pix = (int)(t & 15);
    const int64_t blk = (int64_t)by * g.nbu + bx;
    const int x = 4 * bx + (pix & 3), y = 4 * by + (pix >> 2);
    const bool inside = x < g.w && y < g.h; // a level narrower than a block (w or h < 4)
    const int64_t o = ((int64_t)y * g.w + x) * C;
    float G[C];
    bool touched = false;
#pragma unroll
    for (int ch = 0; ch < C; ++ch) {
        G[ch] = inside ? g.tgrads[o + ch] : 0.f;
        touched |= G[ch] != 0.f;
    }
    // Lanes of the block with a non-zero gradient (the block's 16-bit slice of the wave's).
    const uint64_t vote = __ballot(touched);
    const int lane = (int)(threadIdx.x & 63);
    if (((vote >> (lane & ~15)) & 0xFFFFull) == 0)
        return; // the whole block untouched (all 16 lanes leave together)
    const Bc6Pixel<C> q = bc6_pixel<C>(g.params + blk * (4 * C + 18), pix);
    float *grec = g.grads + blk * (4 * C + 16);
    const float deibar = ldexpf(31.f / 64.f, 16 - q.bits);
    const float alpha = ldexpf(q.xi, 3);
    float dl_dx = 0.f;
    float de[4][C];
#pragma unroll
    for (int ch = 0; ch < C; ++ch) {
        const int hy = bc6_hy(bc6_y(q.q0[ch], q.q1[ch], q.xi));
        const float dl_dy = ldexpf(G[ch], hy - 24);
        dl_dx += dl_dy * ldexpf(q.q1[ch] - q.q0[ch], 3);
        const float a0 = touched ? ((1.f - alpha) * deibar) * dl_dy : 0.f;
        const float a1 = touched ? (alpha * deibar) * dl_dy : 0.f;
        de[0][ch] = q.part ? 0.f : a0;
        de[1][ch] = q.part ? 0.f : a1;
        de[2][ch] = q.part ? a0 : 0.f;
        de[3][ch] = q.part ? a1 : 0.f;
    }
    if (touched)
        grec[4 * C + pix] += dl_dx;
    // Sums over the block's 16 lanes by DPP within each row of 16: lanes xor 1, xor 2
    // (quad permutations), then the mirrors of each half row and of the row (after the
    // first two steps every lane of a quad holds the quad's sum, and each mirror pairs every
    // lane with one of the other half).
#pragma unroll
    for (int k = 0; k < 4; ++k)
#pragma unroll
        for (int ch = 0; ch < C; ++ch) {
            float v = de[k][ch];
            v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0xB1, 0xF, 0xF, false));
            v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x4E, 0xF, 0xF, false));
            v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x141, 0xF, 0xF, false));
            v += __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x140, 0xF, 0xF, false));
            de[k][ch] = v;
        }
    if (pix == 0) {
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
            for (int ch = 0; ch < C; ++ch)
                if (de[k][ch] != 0.f)
                    grec[k * C + ch] += de[k][ch];
    }
}

template <template <int> class K>
static hipError_t launch_phase(const Bc6PhaseDesc &d, hipStream_t s)
{
    if (d.total_blocks <= 0)
        return hipSuccess;
    const dim3 grid((unsigned)((d.total_blocks * 16 + 255) / 256));
    switch (d.C) {
    case 3:
        hipLaunchKernelGGL(K<3>::kernel, grid, dim3(256), 0, s, d);
        break;
    case 8:
        hipLaunchKernelGGL(K<8>::kernel, grid, dim3(256), 0, s, d);
        break;
    case 16:
        hipLaunchKernelGGL(K<16>::kernel, grid, dim3(256), 0, s, d);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}
template <int C>
struct ExpandK {
    static constexpr auto kernel = bc6_expand_kernel<C>;
};
template <int C>
struct FoldK {
    static constexpr auto kernel = bc6_fold_kernel<C>;
};

hipError_t launch_bc6_expand(const Bc6PhaseDesc &d, hipStream_t s) { return launch_phase<ExpandK>(d, s); }

hipError_t launch_bc6_fold(const Bc6PhaseDesc &d, hipStream_t s) { return launch_phase<FoldK>(d, s); }

} // namespace ntk
