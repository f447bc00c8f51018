// nt_adam.hip — lazy Adam as bandwidth-bound elementwise kernels (replaces
// OptimizeNetwork / OptimizeFeatures, train.cu:521-816, 963-972).
//
// Semantics kept from the reference: a parameter whose gradient is exactly zero is skipped
// (its moments do not decay), an updated parameter has its gradient re-zeroed, and the bias
// corrections use t = max(step, 1) (train.cu:528, 580-586). The corrections 1 - beta^t are
// computed once on the host and passed in. The latent kernel streams float4 gradient words
// and touches the parameter and moments only where a gradient is non-zero.
#include <algorithm>

#include "nt_device.hpp"
#include "nt_internal.hpp"

namespace ntk {

// AdamUpdateFloatParameter (train.cu:545-564), contraction as nvcc forms it.
__device__ __forceinline__ float adam_update(float &m1, float &m2, float g, const AdamDesc &a, float w)
{
    m1 = fmaf(a.beta1, m1, (1.f - a.beta1) * g);
    m2 = fmaf(a.beta2, m2, (1.f - a.beta2) * g * g);
    const float mhat = m1 / a.bc1;
    const float vhat = m2 / a.bc2;
    return w - a.lr * mhat / (sqrtf(vhat) + a.eps);
}

__global__ __launch_bounds__(256) void net_adam_kernel(NetAdamDesc d)
{
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= d.wstart[d.num_layers])
        return;
    // Layers start at multiples of 256 items: the layer is uniform per workgroup and its
    // pointers come from scalar loads.
    int l = 0;
    for (int k = 1; k < d.num_layers; ++k)
        if ((int)(blockIdx.x * 256) >= d.wstart[k])
            l = k;
    l = __builtin_amdgcn_readfirstlane(l);
    const int local = i - d.wstart[l];
    const int nw = d.rows[l] * d.cols[l];
    if (local >= nw + d.nbias[l])
        return; // padding to the next layer's start
    if (local < nw) {
        // OptimizePaddedParameterMatrix (train.cu:590-623): active rows x cols only.
        const int row = local % d.rows[l], col = local / d.rows[l];
        const int idx = col * d.pin[l] + row;
        // Network gradients are almost all non-zero: the moments and the weight are loaded
        // with the gradient, in one round trip.
        float *gp = d.g[l] + idx;
        const float g = *gp;
        float m1 = d.m1[l][idx], m2 = d.m2[l][idx];
        const uint16_t wb = d.w[l][idx];
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory"); // keeps the loads above the test
        if (g == 0.f)
            return;
        const float w = adam_update(m1, m2, g, d.a, h2f(wb));
        d.m1[l][idx] = m1;
        d.m2[l][idx] = m2;
        d.w[l][idx] = h_bits((_Float16)w);
        *gp = 0.f;
    } else {
        // OptimizeParameterBuffer (train.cu:566-588).
        const int idx = local - nw;
        float *gp = d.bg[l] + idx;
        const float g = *gp;
        float m1 = d.bm1[l][idx], m2 = d.bm2[l][idx];
        const uint16_t bb = d.b[l][idx];
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        if (g == 0.f)
            return;
        const float w = adam_update(m1, m2, g, d.a, h2f(bb));
        d.bm1[l][idx] = m1;
        d.bm2[l][idx] = m2;
        d.b[l][idx] = h_bits((_Float16)w);
        *gp = 0.f;
    }
}

// Segment (grid) of the workgroup's current work items: segments start at multiples of
// kAdamSpan items, so it is uniform and the segment's pointers come from scalar loads.
__device__ __forceinline__ int adam_segment(const LatentAdamDesc &d, int64_t block_first)
{
    int s = 0;
#pragma unroll
    for (int k = 1; k < NT_MAX_GRIDS; ++k)
        if (k < d.nseg && block_first >= d.start[k])
            s = k;
    return __builtin_amdgcn_readfirstlane(s);
}

// One work item: floats f0 .. f0 + 3 of an n-float segment (fewer at its end), their
// gradient already loaded when four are there.
__device__ __forceinline__ void adam_item(const AdamDesc &a, float *w, float *gp, float *m1p, float *m2p, int64_t n,
                                          int64_t f0, float4 gv)
{
    const int64_t rem = n - f0;
    float *g = gp + f0;
    if (rem >= 4) {
        if (gv.x == 0.f && gv.y == 0.f && gv.z == 0.f && gv.w == 0.f)
            return;
        float4 wv = *(const float4 *)(w + f0);
        float4 m1 = *(const float4 *)(m1p + f0);
        float4 m2 = *(const float4 *)(m2p + f0);
        if (gv.x != 0.f)
            wv.x = adam_update(m1.x, m2.x, gv.x, a, wv.x);
        if (gv.y != 0.f)
            wv.y = adam_update(m1.y, m2.y, gv.y, a, wv.y);
        if (gv.z != 0.f)
            wv.z = adam_update(m1.z, m2.z, gv.z, a, wv.z);
        if (gv.w != 0.f)
            wv.w = adam_update(m1.w, m2.w, gv.w, a, wv.w);
        *(float4 *)(w + f0) = wv;
        *(float4 *)(m1p + f0) = m1;
        *(float4 *)(m2p + f0) = m2;
        *(float4 *)g = make_float4(0.f, 0.f, 0.f, 0.f);
    } else {
        for (int k = 0; k < rem; ++k) {
            const float gs = g[k];
            if (gs == 0.f)
                continue;
            float m1 = m1p[f0 + k], m2 = m2p[f0 + k];
            w[f0 + k] = adam_update(m1, m2, gs, a, w[f0 + k]);
            m1p[f0 + k] = m1;
            m2p[f0 + k] = m2;
            g[k] = 0.f;
        }
    }
}

__device__ __forceinline__ void latent_adam_item(const LatentAdamDesc &d, int s, int64_t f0, float4 gv)
{
    adam_item(d.a, d.w[s], d.g[s], d.m1[s], d.m2[s], d.n[s], f0, gv);
}

// Unconstrained latents: work item = 4 consecutive floats of one grid's flattened mip chain
// (OptimizeUnconstrainedFeaturePass, train.cu:764-803). A workgroup takes kAdamSpan items
// at a time, thread t the items t + 256k: all four gradient loads are issued before any is
// tested (almost all gradients are zero; the scan is what costs).
// NT_LATENT_TOUCHED with one logged train step: only the texels of its footprint
// rectangles can hold non-zero gradients. The float4 items of all rectangles (16 channels:
// four per texel, rows of the rectangle one after another) are dealt out evenly, two per
// thread per pass; a thread issues the gradient, parameter and moment loads of all its items
// at once (one memory round trip: nearly every texel of a region's footprint has a non-zero
// gradient), then writes back the items with a non-zero gradient.
__device__ void latent_adam_rects(const LatentAdamDesc &d, const int32_t (&rect)[NT_MAX_GRIDS][4], int bid, int nb,
                                  int tid)
{
    // Two items per thread per pass: a region's rectangles are a few hundred thousand items,
    // and more items per thread would leave most CUs with one workgroup (measured: four per
    // thread 2-4 % slower steps on configs 2 and the reference network, equal on config 4).
    constexpr int K = 2;
    int start[NT_MAX_GRIDS + 1], nx4[NT_MAX_GRIDS];
    start[0] = 0;
#pragma unroll
    for (int s = 0; s < NT_MAX_GRIDS; ++s) {
        const bool on = s < d.nseg;
        nx4[s] = on ? 4 * (rect[s][1] - rect[s][0] + 1) : 1;
        start[s + 1] = start[s] + (on ? (rect[s][3] - rect[s][2] + 1) * nx4[s] : 0);
    }
    const int total = start[NT_MAX_GRIDS];
    for (int base = bid * (256 * K); base < total; base += nb * (256 * K)) {
        float4 gv[K], wv[K], m1[K], m2[K];
        float *W[K], *G[K], *M1[K], *M2[K];
        bool in[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int i = base + tid + 256 * k;
            in[k] = i < total;
            int s = 0;
#pragma unroll
            for (int q = 1; q < NT_MAX_GRIDS; ++q)
                s = i >= start[q] && q < d.nseg ? q : s;
            int x0 = rect[0][0], y0 = rect[0][2], n4 = nx4[0], w = d.gw[0], h = d.gh[0], st = start[0];
            float *pw = d.w[0], *pg = d.g[0], *pm1 = d.m1[0], *pm2 = d.m2[0];
#pragma unroll
            for (int q = 1; q < NT_MAX_GRIDS; ++q)
                if (s == q) {
                    x0 = rect[q][0], y0 = rect[q][2], n4 = nx4[q], w = d.gw[q], h = d.gh[q], st = start[q];
                    pw = d.w[q], pg = d.g[q], pm1 = d.m1[q], pm2 = d.m2[q];
                }
            const int local = in[k] ? i - st : 0;
            const int row = local / n4, xi = local - row * n4;
            const int x = wrap_coord(x0 + (xi >> 2), w), y = wrap_coord(y0 + row, h);
            const int64_t f = ((int64_t)y * w + x) * 16 + 4 * (xi & 3);
            W[k] = pw + f;
            G[k] = pg + f;
            M1[k] = pm1 + f;
            M2[k] = pm2 + f;
            if (in[k]) {
                gv[k] = *(const float4 *)G[k];
                wv[k] = *(const float4 *)W[k];
                m1[k] = *(const float4 *)M1[k];
                m2[k] = *(const float4 *)M2[k];
            }
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if (!in[k] || (gv[k].x == 0.f && gv[k].y == 0.f && gv[k].z == 0.f && gv[k].w == 0.f))
                continue;
            if (gv[k].x != 0.f)
                wv[k].x = adam_update(m1[k].x, m2[k].x, gv[k].x, d.a, wv[k].x);
            if (gv[k].y != 0.f)
                wv[k].y = adam_update(m1[k].y, m2[k].y, gv[k].y, d.a, wv[k].y);
            if (gv[k].z != 0.f)
                wv[k].z = adam_update(m1[k].z, m2[k].z, gv[k].z, d.a, wv[k].z);
            if (gv[k].w != 0.f)
                wv[k].w = adam_update(m1[k].w, m2[k].w, gv[k].w, d.a, wv[k].w);
            *(float4 *)W[k] = wv[k];
            *(float4 *)M1[k] = m1[k];
            *(float4 *)M2[k] = m2[k];
            *(float4 *)G[k] = make_float4(0.f, 0.f, 0.f, 0.f);
        }
    }
}

// Three channels (the reference network): one texel (three floats) per work item, the
// rectangles' rows one after another; two items per thread per pass, every load of them
// issued before the first update, and only channels with a non-zero gradient written back.
__device__ void latent_adam_rects3(const LatentAdamDesc &d, const int32_t (&rect)[NT_MAX_GRIDS][4], int bid, int nb,
                                   int tid)
{
    constexpr int K = 2, C = 3; // items per thread per pass, as latent_adam_rects
    int start[NT_MAX_GRIDS + 1], nx[NT_MAX_GRIDS];
    start[0] = 0;
#pragma unroll
    for (int s = 0; s < NT_MAX_GRIDS; ++s) {
        const bool on = s < d.nseg;
        nx[s] = on ? rect[s][1] - rect[s][0] + 1 : 1;
        start[s + 1] = start[s] + (on ? (rect[s][3] - rect[s][2] + 1) * nx[s] : 0);
    }
    const int total = start[NT_MAX_GRIDS];
    for (int base = bid * (256 * K); base < total; base += nb * (256 * K)) {
        float gv[K][C], wv[K][C], m1[K][C], m2[K][C];
        float *W[K], *G[K], *M1[K], *M2[K];
        bool in[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int i = base + tid + 256 * k;
            in[k] = i < total;
            int s = 0;
#pragma unroll
            for (int q = 1; q < NT_MAX_GRIDS; ++q)
                s = i >= start[q] && q < d.nseg ? q : s;
            int x0 = rect[0][0], y0 = rect[0][2], n = nx[0], w = d.gw[0], h = d.gh[0], st = start[0];
            float *pw = d.w[0], *pg = d.g[0], *pm1 = d.m1[0], *pm2 = d.m2[0];
#pragma unroll
            for (int q = 1; q < NT_MAX_GRIDS; ++q)
                if (s == q) {
                    x0 = rect[q][0], y0 = rect[q][2], n = nx[q], w = d.gw[q], h = d.gh[q], st = start[q];
                    pw = d.w[q], pg = d.g[q], pm1 = d.m1[q], pm2 = d.m2[q];
                }
            const int local = in[k] ? i - st : 0;
            const int row = local / n, xi = local - row * n;
            const int x = wrap_coord(x0 + xi, w), y = wrap_coord(y0 + row, h);
            const int64_t f = ((int64_t)y * w + x) * C;
            W[k] = pw + f;
            G[k] = pg + f;
            M1[k] = pm1 + f;
            M2[k] = pm2 + f;
            if (in[k]) {
#pragma unroll
                for (int c = 0; c < C; ++c) {
                    gv[k][c] = G[k][c];
                    wv[k][c] = W[k][c];
                    m1[k][c] = M1[k][c];
                    m2[k][c] = M2[k][c];
                }
            }
        }
#pragma unroll
        for (int k = 0; k < K; ++k) {
            if (!in[k])
                continue;
#pragma unroll
            for (int c = 0; c < C; ++c) {
                if (gv[k][c] == 0.f)
                    continue;
                W[k][c] = adam_update(m1[k][c], m2[k][c], gv[k][c], d.a, wv[k][c]);
                M1[k][c] = m1[k][c];
                M2[k][c] = m2[k][c];
                G[k][c] = 0.f;
            }
        }
    }
}

// The latent update as workgroup `bid` of `nb` 256-thread workgroups (thread `tid`): from
// the update log's rectangles when it describes exactly one train step, else every texel.
__device__ void latent_adam_body(const LatentAdamDesc &d, int bid, int nb, int tid)
{
    constexpr int K = kAdamSpan / 256;
    if (d.log) {
        // NT_LATENT_TOUCHED: every workgroup reads the log's count and rectangles; one
        // thread writes `consumed`, which no other reads.
        const UpdateLog *log = d.log;
        const bool valid = log->magic == kUpdateLogMagic;
        const uint32_t count = valid ? log->count : 0u;
        const bool rects = valid && count == 1u && log->kind == kUpdateLogTexels && (d.C == 16 || d.C == 3);
        if (rects) {
            int32_t rect[NT_MAX_GRIDS][4];
#pragma unroll
            for (int gi = 0; gi < NT_MAX_GRIDS; ++gi)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    rect[gi][k] = __builtin_amdgcn_readfirstlane(log->rect[gi][k]);
            if (d.C == 16)
                latent_adam_rects(d, rect, bid, nb, tid);
            else
                latent_adam_rects3(d, rect, bid, nb, tid);
        }
        if (valid && bid == 0 && tid == 0)
            d.log->consumed = count;
        if (rects)
            return;
    }
    const int64_t total = d.start[d.nseg];
    for (int64_t base = (int64_t)bid * kAdamSpan; base < total; base += (int64_t)nb * kAdamSpan) {
        const int s = adam_segment(d, base);
        const int64_t f = (base - d.start[s] + tid) * 4;
        float4 gv[K];
#pragma unroll
        for (int k = 0; k < K; ++k) {
            const int64_t fk = f + 1024 * k;
            gv[k] = fk + 4 <= d.n[s] ? *(const float4 *)(d.g[s] + fk) : make_float4(1.f, 1.f, 1.f, 1.f);
        }
#pragma unroll
        for (int k = 0; k < K; ++k)
            latent_adam_item(d, s, f + 1024 * k, gv[k]);
    }
}

__global__ __launch_bounds__(256) void latent_adam_kernel(LatentAdamDesc d)
{
    latent_adam_body(d, blockIdx.x, gridDim.x, threadIdx.x);
}

// One launch for both optimizers after a train step (nt_train_iteration): workgroups
// [0, nred) sum the train kernel's MLP-gradient partial rows, 64 parameters each (as
// reduce_rows), and apply the network update to them (as net_adam_kernel: the same sum
// g = grad + partials, then the same lazy update); the others run the latent update. The two
// parts touch disjoint parameters. 256-thread workgroups: the partial rows are summed as
// reduce_rows sums them (kReduceRanges contiguous ranges, each in row order, then the range
// sums in range order), each of the four thread groups taking four consecutive ranges, four
// rows of each per pass with their loads issued together. The latent update shares the
// kernel and so its register count: sixteen loads in flight per thread (74 registers) rather
// than sixty-four (109) leave it six waves per SIMD instead of four (config 4 15.1 ->
// 14.6 us, config 2 9.3 -> 8.5 us).
__device__ void block_adam_body(const LatentAdamDesc &d, int bid, int nb, int tid);

constexpr int kOptCols = 64, kOptGroups = 4, kOptUnroll = 4;
constexpr int kOptRangesPerGroup = kReduceRanges / kOptGroups;
static_assert(kOptRangesPerGroup * kOptGroups == kReduceRanges, "ranges split evenly over the groups");

__global__ __launch_bounds__(kOptCols *kOptGroups) void optimize_step_kernel(OptimizeStepDesc d)
{
    if ((int)blockIdx.x >= d.nred) {
        if (d.lat.rec > 0)
            block_adam_body(d.lat, (int)blockIdx.x - d.nred, (int)gridDim.x - d.nred, threadIdx.x);
        else
            latent_adam_body(d.lat, (int)blockIdx.x - d.nred, (int)gridDim.x - d.nred, threadIdx.x);
        return;
    }
    const ReduceDesc &r = d.red;
    const NetUpdateDesc &n = d.net;
    __shared__ float part[kReduceRanges][kOptCols];
    const int col = threadIdx.x % kOptCols, grp = threadIdx.x / kOptCols;
    const int p0 = blockIdx.x * kOptCols, p = p0 + col;
    // Layers of this workgroup's 64 parameters (at most a few, uniform): the descriptor's
    // per-layer fields are then read with scalar loads, not per lane.
    auto layer_of = [&](int q) {
        int l = 0;
        for (int k = 1; k < r.num_layers; ++k)
            if (q >= r.off[k])
                l = k;
        return l;
    };
    const int lfirst = layer_of(p0), llast = layer_of(min(p0 + kOptCols, r.P) - 1);
    // Group 0 holds the parameters: their gradient, moments and value are loaded before the
    // partial rows are summed (one round trip for both).
    float gsum = 0.f, m1 = 0.f, m2 = 0.f;
    uint16_t wbits = 0;
    float *gp = nullptr, *m1p = nullptr, *m2p = nullptr;
    uint16_t *wp = nullptr;
    bool active = false;
    if (grp == 0 && p < r.P) {
        for (int l = lfirst; l <= llast; ++l) {
            const int local = p - r.off[l];
            const int nw = r.kin[l] * r.kout[l];
            if (local < 0 || local >= nw + r.kout[l])
                continue;
            if (local < nw) {
                // Padded column-major [col][row]: active rows x cols take the update
                // (train.cu:590-623); padding only accumulates.
                const int row = local % r.kin[l], cl = local / r.kin[l];
                gp = r.wgrad[l] + local;
                active = row < n.rows[l] && cl < n.cols[l];
                m1p = n.m1[l] + local;
                m2p = n.m2[l] + local;
                wp = n.w[l] + local;
            } else if (local - nw < r.nbias[l]) {
                const int idx = local - nw;
                gp = r.bgrad[l] + idx;
                active = true;
                m1p = n.bm1[l] + idx;
                m2p = n.bm2[l] + idx;
                wp = n.b[l] + idx;
            }
        }
        if (gp)
            gsum = *gp;
        if (active) {
            m1 = *m1p;
            m2 = *m2p;
            wbits = *wp;
        }
    }
    const int per = (r.rows + kReduceRanges - 1) / kReduceRanges;
    float sum[kOptRangesPerGroup] = {};
    if (p < r.P) {
        const float *c = r.partial + p;
        for (int k0 = 0; k0 < per; k0 += kOptUnroll) {
            float v[kOptRangesPerGroup][kOptUnroll];
#pragma unroll
            for (int q = 0; q < kOptRangesPerGroup; ++q) {
                const int r0 = (grp * kOptRangesPerGroup + q) * per, r1 = min(r0 + per, r.rows);
#pragma unroll
                for (int k = 0; k < kOptUnroll; ++k)
                    v[q][k] = r0 + k0 + k < r1 ? c[(int64_t)(r0 + k0 + k) * r.P] : 0.f;
            }
#pragma unroll
            for (int q = 0; q < kOptRangesPerGroup; ++q)
#pragma unroll
                for (int k = 0; k < kOptUnroll; ++k)
                    sum[q] += v[q][k];
        }
    }
#pragma unroll
    for (int q = 0; q < kOptRangesPerGroup; ++q)
        part[grp * kOptRangesPerGroup + q][col] = sum[q];
    __syncthreads();
    if (grp != 0 || !gp)
        return;
    float s = 0.f;
#pragma unroll
    for (int k = 0; k < kReduceRanges; ++k)
        s += part[k][col];
    const float g = gsum + s;
    if (!active || g == 0.f) {
        // An inactive (padding) parameter only accumulates; a zero gradient skips the lazy
        // update but the buffer still receives the sum, as reduce_rows writes it.
        *gp = g;
        return;
    }
    const float w = adam_update(m1, m2, g, n.a, h2f(wbits));
    *m1p = m1;
    *m2p = m2;
    *wp = h_bits((_Float16)w);
    *gp = 0.f;
}

hipError_t launch_optimize_step(const OptimizeStepDesc &d0, hipStream_t s)
{
    OptimizeStepDesc d = d0;
    d.nred = (d.red.P + kOptCols - 1) / kOptCols;
    const int64_t n = d.lat.start[d.lat.nseg];
    // Block records: 256 records per workgroup pass (block_adam_body); texels: kAdamSpan.
    int64_t lat = d.lat.rec > 0 ? (n + 255) / 256 : (n + kAdamSpan - 1) / kAdamSpan;
    if (d.lat_wg > 0 && d.lat_wg < lat)
        lat = d.lat_wg;
    if (lat > 8192)
        lat = 8192;
    hipLaunchKernelGGL(optimize_step_kernel, dim3((unsigned)(d.nred + lat)), dim3(kOptCols * kOptGroups), 0, s, d);
    return hipGetLastError();
}

// Lazy Adam of one float of a block record, its gradient, moments and value loaded at once
// (in the logged rectangles nearly every gradient is non-zero).
__device__ __forceinline__ void block_adam_float(const LatentAdamDesc &d, float *w, float *g, float *m1, float *m2)
{
    const float gs = *g;
    float a1 = *m1, a2 = *m2;
    const float wv = *w;
    if (gs == 0.f)
        return;
    *w = adam_update(a1, a2, gs, d.a, wv);
    *m1 = a1;
    *m2 = a2;
    *g = 0.f;
}

// BC6 block records (OptimizeFeatureBlock, train.cu:641-679): every float of the
// parameter record except the trailing partition/mode pair. With NT_LATENT_TOUCHED and a
// log of exactly one BC6-phase train step, only the mip-0 blocks of the logged rectangles
// are visited (every other record holds zero gradients, which the lazy rule skips), the
// rectangles' records one after another, each in consecutive floats.
__device__ void block_adam_body(const LatentAdamDesc &d, int bid, int nb, int tid)
{
    if (d.log) {
        const UpdateLog *log = d.log;
        const bool valid = log->magic == kUpdateLogMagic;
        const uint32_t count = valid ? log->count : 0u;
        const bool rects = valid && count == 1u && log->kind == kUpdateLogBlocks;
        if (rects) {
            const int rec = d.rec;
            int64_t start[NT_MAX_GRIDS + 1];
            int r[NT_MAX_GRIDS][4];
            start[0] = 0;
#pragma unroll
            for (int s = 0; s < NT_MAX_GRIDS; ++s) {
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    r[s][k] = __builtin_amdgcn_readfirstlane(log->rect[s][k]);
                const bool on = s < d.nseg;
                start[s + 1] = start[s] + (on ? (int64_t)(r[s][1] - r[s][0] + 1) * (r[s][3] - r[s][2] + 1) * rec : 0);
            }
            const int64_t total = start[NT_MAX_GRIDS];
            for (int64_t i = (int64_t)bid * 256 + tid; i < total; i += (int64_t)nb * 256) {
                int s = 0;
#pragma unroll
                for (int q = 1; q < NT_MAX_GRIDS; ++q)
                    s = i >= start[q] && q < d.nseg ? q : s;
                const int64_t local = i - start[s];
                const int64_t rb = local / rec;
                const int e = (int)(local - rb * rec);
                const int nbx = r[s][1] - r[s][0] + 1;
                const int bx = wrap_coord(r[s][0] + (int)(rb % nbx), d.gw[s]);
                const int by = wrap_coord(r[s][2] + (int)(rb / nbx), d.gh[s]);
                const int64_t blk = (int64_t)by * d.gw[s] + bx;
                block_adam_float(d, d.w[s] + blk * (rec + 2) + e, d.g[s] + blk * rec + e, d.m1[s] + blk * rec + e,
                                 d.m2[s] + blk * rec + e);
            }
        }
        if (valid && bid == 0 && tid == 0)
            d.log->consumed = count;
        if (rects)
            return;
    }
    // A workgroup takes 256 records at a time (segment starts are whole spans, so the
    // records are of one grid) and spreads their rec * 256 floats over its threads, each
    // array read and written in consecutive floats.
    const int64_t total = d.start[d.nseg];
    const int rec = d.rec;
    for (int64_t r0 = (int64_t)bid * 256; r0 < total; r0 += (int64_t)nb * 256) {
        const int s = adam_segment(d, r0);
        const int64_t b0 = r0 - d.start[s];
        const int64_t left = d.n[s] - b0;
        if (left <= 0)
            continue; // padding to the next segment's start
        const int ne = (int)(left < 256 ? left : 256) * rec;
        float *w = d.w[s] + b0 * (rec + 2);
        float *g = d.g[s] + b0 * rec;
        float *m1 = d.m1[s] + b0 * rec;
        float *m2 = d.m2[s] + b0 * rec;
        for (int e = tid; e < ne; e += 256) {
            const float gs = g[e];
            if (gs == 0.f)
                continue;
            const int r = e / rec;
            float *wp = w + r * (rec + 2) + (e - r * rec);
            float a1 = m1[e], a2 = m2[e];
            *wp = adam_update(a1, a2, gs, d.a, *wp);
            m1[e] = a1;
            m2[e] = a2;
            g[e] = 0.f;
        }
    }
}

__global__ __launch_bounds__(256) void block_adam_kernel(LatentAdamDesc d)
{
    block_adam_body(d, blockIdx.x, gridDim.x, threadIdx.x);
}

hipError_t launch_net_adam(const NetAdamDesc &d, hipStream_t s)
{
    const int n = d.wstart[d.num_layers];
    if (n <= 0)
        return hipSuccess;
    hipLaunchKernelGGL(net_adam_kernel, dim3((n + 255) / 256), dim3(256), 0, s, d);
    return hipGetLastError();
}

__global__ void log_dense_step_kernel(UpdateLog *log)
{
    if (log->magic != kUpdateLogMagic) {
        log->magic = kUpdateLogMagic;
        log->consumed = 0u;
    }
    log->count = kUpdateLogDense;
}

hipError_t launch_log_dense_step(UpdateLog *log, hipStream_t s)
{
    hipLaunchKernelGGL(log_dense_step_kernel, dim3(1), dim3(1), 0, s, log);
    return hipGetLastError();
}

hipError_t launch_latent_adam(const LatentAdamDesc &d, hipStream_t s)
{
    const int64_t n = d.start[d.nseg];
    if (n <= 0)
        return hipSuccess;
    int64_t blocks = d.rec > 0 ? (n + 255) / 256 : (n + kAdamSpan - 1) / kAdamSpan;
    if (blocks > 8192)
        blocks = 8192;
    if (d.rec > 0)
        hipLaunchKernelGGL(block_adam_kernel, dim3((unsigned)blocks), dim3(256), 0, s, d);
    else
        hipLaunchKernelGGL(latent_adam_kernel, dim3((unsigned)blocks), dim3(256), 0, s, d);
    return hipGetLastError();
}

} // namespace ntk
