// nt_sort.hip — the sample order of NT_SAMPLES_RANDOM steps. Each sample's texel (the
// placement the train kernel uses: random_texel of its seed) falls in a 64 x 64-texel bin;
// the sample indices are sorted by bin, stably, so that consecutive slots — one chunk of the
// train kernel — lie close together in the image and their target taps, latent corners and
// gradient atomics share cache lines in the L2. The kernel reads the sample of each slot from
// the order and places it exactly as before: the samples and their results are unchanged,
// only the order of the fp32 sums moves. A stable sort by key has one result, so the order is
// the same on every run.
//
// The sort is a counting sort by digits, all integer work. sort_count_kernel: each workgroup
// takes a tile of consecutive samples (4,096, or more so that there are at most 256 tiles),
// computes their bin keys (stored for the later passes) and counts them per first digit in
// LDS (the whole key when it has at most ten bits, config 2's 1,024 bins; else its top eight
// bits). sort_first_pass_kernel: each workgroup derives where its tile's samples of each
// digit start from all tiles' counts (the digits' totals, scanned, plus the digit's counts
// in earlier tiles), then places its samples in order, 256 a round (the keys of 16 rounds
// loaded at once, so that the rounds wait on no memory): a sample's place is its digit's
// running place + the samples before it in the round with the same digit (a wave's lanes by
// ballots on the digit bits, the waves before it by their counts). Keys of more than ten
// bits then go through sort_segment_kernel: one workgroup per first digit sorts that digit's
// segment by the remaining key bits the same way, writing the final order.
#include <hip/hip_runtime.h>

#include "nt_internal.hpp"

namespace ntk {

namespace {

constexpr int kSortThreads = 256, kSortWaves = kSortThreads / 64;
constexpr int kSortRegs = 16;   // items per thread loaded at once in the scatter passes
constexpr int kSortMaxDigits = 1024; // digits of a one-pass sort (keys of at most ten bits)

__device__ __forceinline__ uint32_t bin_key(const RandomOrderDesc &d, uint32_t i)
{
    uint32_t tx, ty;
    random_texel(mix_seed(i, d.step), d.image_w, d.image_h, tx, ty);
    return (ty >> d.bin_shift) * (uint32_t)d.bins_x + (tx >> d.bin_shift);
}

// The lanes of the wave that are active and hold the same digit (`bits` bits) as this lane.
__device__ __forceinline__ uint64_t match_digit(uint32_t digit, int bits, uint64_t active)
{
    uint64_t m = active;
    for (int b = 0; b < bits; ++b) {
        const bool set = (digit >> b) & 1u;
        const uint64_t bal = __ballot(set);
        m &= set ? bal : ~bal;
    }
    return m;
}

// One round of a stable counting-sort pass over 256 items (item t of the round on thread t).
// base[x]: where the next item of digit x goes; wcnt[w][x]: wave w's count of digit x in the
// round, zero outside the round (each wave writes and clears only its own row). The first
// barrier also orders the previous round's additions to base before this round reads it.
// Returns the item's place (valid items only).
template <int ND>
__device__ __forceinline__ uint32_t round_place(uint32_t digit, int bits, bool valid, uint32_t *base,
                                                uint32_t (*wcnt)[ND])
{
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const uint64_t m = match_digit(digit, bits, __ballot(valid));
    const uint64_t before = m & ((1ull << lane) - 1ull);
    const bool leader = valid && before == 0; // the lowest lane of each digit
    const uint32_t cnt = (uint32_t)__popcll(m);
    if (leader)
        wcnt[w][digit] = cnt;
    __syncthreads();
    uint32_t pos = 0;
    if (valid) {
        pos = base[digit] + (uint32_t)__popcll(before);
#pragma unroll
        for (int v = 0; v < kSortWaves - 1; ++v) {
            const uint32_t x = wcnt[v][digit];
            pos += v < w ? x : 0u;
        }
    }
    __syncthreads();
    if (leader) {
        atomicAdd(&base[digit], cnt); // integer adds: the same sum in any order
        wcnt[w][digit] = 0;
    }
    return pos;
}

// Counts per tile and first digit: tile-major rows of max(4, digits) counts.
__global__ __launch_bounds__(kSortThreads) void sort_count_kernel(RandomOrderDesc d)
{
    __shared__ uint32_t hist[kSortMaxDigits];
    const int t = threadIdx.x;
    const int ndig = 1 << d.high_bits, low = d.key_bits - d.high_bits;
    for (int x = t; x < kSortMaxDigits; x += kSortThreads)
        hist[x] = 0;
    __syncthreads();
    const int64_t first = (int64_t)blockIdx.x * d.tile, lim = min(first + d.tile, (int64_t)d.n);
    for (int64_t r = first; r < lim; r += kSortThreads) {
        const int64_t j = r + t;
        if (j < lim) {
            const uint32_t key = bin_key(d, (uint32_t)j);
            d.keys[j] = (uint16_t)key;
            atomicAdd(&hist[key >> low], 1u);
        }
    }
    __syncthreads();
    const int stride = ndig < 4 ? 4 : ndig;
    for (int x = t; x < stride; x += kSortThreads)
        d.counts[(int64_t)blockIdx.x * stride + x] = x < ndig ? hist[x] : 0u;
}

// base[x] (x < max(4, digits)): where this workgroup's first sample of first digit x goes.
// Thread t sums digits 4g .. 4g + 3 (g = t mod G, G = max(4, digits) / 4 groups) over the
// tiles of range t / G (256 / G ranges), 16-byte loads issued 16 at a time; the ranges are
// added in LDS, then the groups' totals scanned.
__device__ __forceinline__ void tile_bases(const RandomOrderDesc &d, uint32_t *base, uint32_t (*red)[kSortThreads][4],
                                           uint32_t *part)
{
    const int t = threadIdx.x, tile = blockIdx.x;
    const int ndig = 1 << d.high_bits, stride = ndig < 4 ? 4 : ndig;
    const int groups = stride / 4, ranges = kSortThreads / groups;
    const int g = t % groups, r = t / groups;
    const int per = (d.tiles + ranges - 1) / ranges, b_lo = min(r * per, d.tiles), b_hi = min(b_lo + per, d.tiles);
    uint32_t tot[4] = {0u, 0u, 0u, 0u}, pre[4] = {0u, 0u, 0u, 0u};
    for (int b0 = b_lo; b0 < b_hi; b0 += 16) {
        uint4 x[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            x[q] = make_uint4(0u, 0u, 0u, 0u);
            if (b0 + q < b_hi)
                x[q] = *(const uint4 *)(d.counts + (int64_t)(b0 + q) * stride + 4 * g);
        }
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const uint32_t e[4] = {x[q].x, x[q].y, x[q].z, x[q].w};
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                tot[c] += e[c];
                pre[c] += b0 + q < tile ? e[c] : 0u;
            }
        }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        red[0][t][c] = tot[c];
        red[1][t][c] = pre[c];
    }
    __syncthreads();
    uint32_t s = 0;
    if (t < groups) {
        for (int q = 1; q < ranges; ++q)
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                tot[c] += red[0][q * groups + t][c];
                pre[c] += red[1][q * groups + t][c];
            }
        s = tot[0] + tot[1] + tot[2] + tot[3];
    }
    part[t] = s;
    __syncthreads();
    for (int off = 1; off < kSortThreads; off <<= 1) {
        const uint32_t x = t >= off ? part[t - off] : 0u;
        __syncthreads();
        part[t] += x;
        __syncthreads();
    }
    if (t < groups) {
        uint32_t run = part[t] - s;
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            base[4 * t + c] = run + pre[c];
            run += tot[c];
        }
    }
    __syncthreads();
}

// The first pass (see the top of the file): the final order for keys of at most ten bits;
// else keys and sample indices into the alternate buffers, grouped by their top eight bits,
// and (workgroup 0) each group's start.
__global__ __launch_bounds__(kSortThreads) void sort_first_pass_kernel(RandomOrderDesc d)
{
    __shared__ uint32_t base[kSortMaxDigits];
    __shared__ uint32_t wcnt[kSortWaves][kSortMaxDigits];
    __shared__ uint32_t red[2][kSortThreads][4];
    __shared__ uint32_t part[kSortThreads];
    const int t = threadIdx.x;
    const int ndig = 1 << d.high_bits, low = d.key_bits - d.high_bits;
    for (int v = 0; v < kSortWaves; ++v)
        for (int x = t; x < kSortMaxDigits; x += kSortThreads)
            wcnt[v][x] = 0;
    tile_bases(d, base, red, part);
    if (low && blockIdx.x == 0) {
        for (int x = t; x < ndig; x += kSortThreads)
            d.seg[x] = base[x];
        if (t == 0)
            d.seg[ndig] = (uint32_t)d.n;
    }
    uint32_t *out = low ? d.vals_alt : d.vals;
    const int64_t first = (int64_t)blockIdx.x * d.tile, lim = min(first + d.tile, (int64_t)d.n);
    for (int64_t c0 = first; c0 < lim; c0 += kSortRegs * kSortThreads) {
        uint32_t key[kSortRegs];
#pragma unroll
        for (int k = 0; k < kSortRegs; ++k) {
            const int64_t j = c0 + k * kSortThreads + t;
            key[k] = j < lim ? d.keys[j] : 0u;
        }
#pragma unroll
        for (int k = 0; k < kSortRegs; ++k) {
            if (c0 + k * kSortThreads >= lim)
                break; // uniform over the workgroup
            const int64_t j = c0 + k * kSortThreads + t;
            const bool valid = j < lim;
            const uint32_t pos = round_place<kSortMaxDigits>(key[k] >> low, d.high_bits, valid, base, wcnt);
            if (valid && pos < (uint32_t)d.n) {
                out[pos] = (uint32_t)j;
                if (low)
                    d.keys_alt[pos] = (uint16_t)key[k];
            }
        }
    }
}

__global__ __launch_bounds__(kSortThreads) void sort_segment_kernel(RandomOrderDesc d)
{
    __shared__ uint32_t base[256];
    __shared__ uint32_t wcnt[kSortWaves][256];
    const int t = threadIdx.x, h = blockIdx.x;
    const int ndig = 1 << d.high_bits, low = d.key_bits - d.high_bits, nlow = 1 << low;
    const uint32_t lmask = (uint32_t)nlow - 1u;
    const uint32_t start = d.seg[h], end = d.seg[h + 1];
    base[t] = 0;
    for (int v = 0; v < kSortWaves; ++v)
        wcnt[v][t] = 0;
    __syncthreads();
    for (uint32_t c0 = start; c0 < end; c0 += kSortRegs * kSortThreads) {
        uint32_t key[kSortRegs];
#pragma unroll
        for (int k = 0; k < kSortRegs; ++k) {
            const uint32_t i = c0 + k * kSortThreads + t;
            key[k] = i < end ? d.keys_alt[i] : 0u;
        }
#pragma unroll
        for (int k = 0; k < kSortRegs; ++k)
            if (c0 + k * kSortThreads + t < end)
                atomicAdd(&base[key[k] & lmask], 1u);
    }
    __syncthreads();
    // Counts -> segment positions (an inclusive scan over the low digits, then shifted).
    const uint32_t own = t < nlow ? base[t] : 0u;
    for (int off = 1; off < nlow; off <<= 1) {
        const uint32_t x = t < nlow && t >= off ? base[t - off] : 0u;
        __syncthreads();
        if (t < nlow)
            base[t] += x;
        __syncthreads();
    }
    if (t < nlow)
        base[t] = start + base[t] - own;
    __syncthreads();
    for (uint32_t c0 = start; c0 < end; c0 += kSortRegs * kSortThreads) {
        uint32_t key[kSortRegs], val[kSortRegs];
#pragma unroll
        for (int k = 0; k < kSortRegs; ++k) {
            const uint32_t i = c0 + k * kSortThreads + t;
            key[k] = i < end ? d.keys_alt[i] : 0u;
            val[k] = i < end ? d.vals_alt[i] : 0u;
        }
#pragma unroll
        for (int k = 0; k < kSortRegs; ++k) {
            if (c0 + k * kSortThreads >= end)
                break; // uniform over the workgroup
            const bool valid = c0 + k * kSortThreads + t < end;
            const uint32_t pos = round_place<256>(key[k] & lmask, low, valid, base, wcnt);
            if (valid && pos < end)
                d.vals[pos] = val[k];
        }
    }
}

} // namespace

void random_order_tiles(int n, int *tile, int *tiles)
{
    // Tiles of 4,096 samples, at most 256 of them (a whole multiple of 256 samples each).
    int64_t t = kRandomSortTile;
    if (((int64_t)n + t - 1) / t > kRandomSortMaxTiles)
        t = (((int64_t)n + kRandomSortMaxTiles - 1) / kRandomSortMaxTiles + kSortThreads - 1) / kSortThreads *
            kSortThreads;
    *tile = (int)t;
    *tiles = (int)(((int64_t)n + t - 1) / t);
}

int random_order_high_bits(int key_bits, int tiles)
{
    // One pass when each workgroup's read of all tiles' counts stays within 64 Ki counts.
    const int64_t stride = key_bits < 2 ? 4 : (int64_t)1 << key_bits;
    if (key_bits <= 10 && stride * tiles <= 65536)
        return key_bits;
    return key_bits < 8 ? key_bits : 8;
}

static size_t random_order_seg_offset(int tiles, int high_bits)
{
    const size_t ndig = (size_t)1 << high_bits;
    return ((ndig < 4 ? 4 : ndig) * (size_t)tiles + 63) / 64 * 64;
}

size_t random_order_count_bytes(int n, int key_bits)
{
    int tile, tiles;
    random_order_tiles(n, &tile, &tiles);
    const int high = random_order_high_bits(key_bits, tiles);
    const size_t ndig = (size_t)1 << high;
    // The counts, then the first digits' segment starts (two-pass keys).
    return random_order_seg_offset(tiles, high) * sizeof(uint32_t) + (ndig + 1) * sizeof(uint32_t);
}

hipError_t launch_random_order(const RandomOrderDesc &d, hipStream_t s, const uint32_t **order)
{
    int tile, tiles;
    random_order_tiles(d.n, &tile, &tiles);
    if (d.n <= 0 || d.key_bits < 1 || d.key_bits > 16 || d.tile != tile || d.tiles != tiles ||
        d.high_bits != random_order_high_bits(d.key_bits, d.tiles))
        return hipErrorInvalidValue;
    RandomOrderDesc e = d;
    e.seg = d.counts + random_order_seg_offset(d.tiles, d.high_bits);
    hipLaunchKernelGGL(sort_count_kernel, dim3((unsigned)e.tiles), dim3(kSortThreads), 0, s, e);
    hipLaunchKernelGGL(sort_first_pass_kernel, dim3((unsigned)e.tiles), dim3(kSortThreads), 0, s, e);
    if (e.key_bits > e.high_bits)
        hipLaunchKernelGGL(sort_segment_kernel, dim3(1u << e.high_bits), dim3(kSortThreads), 0, s, e);
    *order = e.vals;
    return hipGetLastError();
}

} // namespace ntk
