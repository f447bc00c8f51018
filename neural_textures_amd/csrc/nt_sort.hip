// nt_sort.hip — the sample order of NT_SAMPLES_RANDOM steps. Each sample's texel (the
// placement the train kernel uses: random_texel of its seed) falls in a 64 x 64-texel bin;
// the sample indices are sorted by bin, stably, so that consecutive slots — one chunk of the
// train kernel — lie close together in the image and their target taps, latent corners and
// gradient atomics share cache lines in the L2. The kernel reads the sample of each slot from
// the order and places it exactly as before: the samples and their results are unchanged,
// only the order of the fp32 sums moves. A stable sort by key has one result, so the order is
// the same on every run.
//
// Keys of at most ten bits (config 2's 1,024 bins) take two launches: sort_count_kernel
// (below) with its counts tile-major, then sort_one_pass_kernel, where each workgroup
// derives its digits' places from all tiles' counts (the digit totals scanned, plus its
// digit's counts in earlier tiles) and places its tile's samples as in launch 3 below.
// Longer keys: a most-significant-digit counting sort in four launches, all integer work:
//   1. sort_count_kernel: each workgroup takes a tile of consecutive samples (4,096, or
//      more so that there are at most 256 tiles), computes their bin keys (stored for the
//      later passes) and counts the tile's keys per high digit (the top eight key bits) in
//      LDS;
//   2. sort_scan_kernel: one workgroup turns the counts (digit-major: digit h of every tile,
//      then h + 1) into exclusive offsets, so digit h of tile b starts where every smaller
//      digit and digit h of every earlier tile end;
//   3. sort_scatter_kernel: each tile again, in order, 256 samples a round (the keys of 16
//      rounds loaded at once, so that the rounds wait on no memory); a sample's place
//      is its digit's running offset + the samples before it in the round with the same digit
//      (a wave's lanes by ballots on the digit bits, the waves before it by their counts);
//   4. sort_segment_kernel: one workgroup per high digit sorts that digit's segment by the
//      low key bits the same way (its counts in LDS), writing the final order.
#include <hip/hip_runtime.h>

#include "nt_internal.hpp"

namespace ntk {

namespace {

constexpr int kSortThreads = 256, kSortWaves = kSortThreads / 64;
constexpr int kSortRegs = 16;   // items per thread loaded at once in the scatter passes
constexpr int kScanRegs = 64;   // counts per thread of the scan (at most 256 tiles x 256 digits)
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

// Counts per tile and digit: tile-major rows of max(4, digits) counts for one-pass keys,
// digit-major rows of the tiles' counts otherwise.
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
    if (low == 0) {
        const int stride = ndig < 4 ? 4 : ndig;
        for (int x = t; x < stride; x += kSortThreads)
            d.counts[(int64_t)blockIdx.x * stride + x] = x < ndig ? hist[x] : 0u;
    } else if (t < ndig) {
        d.counts[(int64_t)t * d.tiles + blockIdx.x] = hist[t];
    }
}

// Keys of at most ten bits, sorted whole in this pass (see the top of the file).
__global__ __launch_bounds__(kSortThreads) void sort_one_pass_kernel(RandomOrderDesc d)
{
    __shared__ uint32_t base[kSortMaxDigits];
    __shared__ uint32_t wcnt[kSortWaves][kSortMaxDigits];
    __shared__ uint32_t part[kSortThreads];
    const int t = threadIdx.x, tile = blockIdx.x;
    const int ndig = 1 << d.key_bits, stride = ndig < 4 ? 4 : ndig;
    // Digits 4t .. 4t + 3: their totals over all tiles and their counts in earlier tiles.
    uint32_t tot[4] = {0u, 0u, 0u, 0u}, pre[4] = {0u, 0u, 0u, 0u};
    if (4 * t < stride) {
        for (int b0 = 0; b0 < d.tiles; b0 += 16) {
            uint4 x[16];
#pragma unroll
            for (int q = 0; q < 16; ++q) {
                x[q] = make_uint4(0u, 0u, 0u, 0u);
                if (b0 + q < d.tiles)
                    x[q] = *(const uint4 *)(d.counts + (int64_t)(b0 + q) * stride + 4 * t);
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
    }
    const uint32_t s = tot[0] + tot[1] + tot[2] + tot[3];
    part[t] = s;
    __syncthreads();
    for (int off = 1; off < kSortThreads; off <<= 1) {
        const uint32_t x = t >= off ? part[t - off] : 0u;
        __syncthreads();
        part[t] += x;
        __syncthreads();
    }
    uint32_t run = part[t] - s;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        base[4 * t + c] = run + pre[c];
        run += tot[c];
    }
    for (int v = 0; v < kSortWaves; ++v)
        for (int x = t; x < kSortMaxDigits; x += kSortThreads)
            wcnt[v][x] = 0;
    __syncthreads();
    const int64_t first = (int64_t)tile * d.tile, lim = min(first + d.tile, (int64_t)d.n);
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
            const uint32_t pos = round_place<kSortMaxDigits>(key[k], d.key_bits, valid, base, wcnt);
            if (valid && pos < (uint32_t)d.n)
                d.vals[pos] = (uint32_t)j;
        }
    }
}

// Exclusive scan of the digit-major counts, in place: each of the 1,024 threads loads its
// contiguous run of at most 64 counts at once (16-byte loads; the count buffer is padded to
// whole 64-count blocks), the run totals are scanned in LDS, then each run is rewritten.
__global__ __launch_bounds__(1024) void sort_scan_kernel(RandomOrderDesc d)
{
    __shared__ uint32_t part[1024];
    const int t = threadIdx.x;
    const int m = (1 << d.high_bits) * d.tiles;
    const int per = (((m + 1023) / 1024) + 3) & ~3; // <= kScanRegs
    const int lo = t * per;
    uint32_t v[kScanRegs];
    uint32_t s = 0;
#pragma unroll
    for (int q = 0; q < kScanRegs / 4; ++q) {
        const int i = lo + 4 * q;
        uint4 x = {0u, 0u, 0u, 0u};
        if (4 * q < per && i < m)
            x = *(const uint4 *)(d.counts + i);
        v[4 * q] = i < m ? x.x : 0u;
        v[4 * q + 1] = i + 1 < m ? x.y : 0u;
        v[4 * q + 2] = i + 2 < m ? x.z : 0u;
        v[4 * q + 3] = i + 3 < m ? x.w : 0u;
    }
#pragma unroll
    for (int e = 0; e < kScanRegs; ++e)
        s += v[e];
    part[t] = s;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const uint32_t x = t >= off ? part[t - off] : 0u;
        __syncthreads();
        part[t] += x;
        __syncthreads();
    }
    uint32_t run = part[t] - s;
#pragma unroll
    for (int q = 0; q < kScanRegs / 4; ++q) {
        const int i = lo + 4 * q;
        uint4 x;
        x.x = run;
        run += v[4 * q];
        x.y = run;
        run += v[4 * q + 1];
        x.z = run;
        run += v[4 * q + 2];
        x.w = run;
        run += v[4 * q + 3];
        if (4 * q < per && i + 3 < m) {
            *(uint4 *)(d.counts + i) = x;
        } else if (4 * q < per && i < m) {
            d.counts[i] = x.x;
            if (i + 1 < m)
                d.counts[i + 1] = x.y;
            if (i + 2 < m)
                d.counts[i + 2] = x.z;
        }
    }
}

__global__ __launch_bounds__(kSortThreads) void sort_scatter_kernel(RandomOrderDesc d)
{
    __shared__ uint32_t base[256];
    __shared__ uint32_t wcnt[kSortWaves][256];
    const int t = threadIdx.x;
    const int ndig = 1 << d.high_bits, low = d.key_bits - d.high_bits;
    base[t] = t < ndig ? d.counts[(int64_t)t * d.tiles + blockIdx.x] : 0u;
    for (int v = 0; v < kSortWaves; ++v)
        wcnt[v][t] = 0;
    __syncthreads();
    // Keys of more than eight bits go on to the segment pass: this one writes its keys and
    // sample indices to the alternate buffers; shorter keys are sorted after this pass.
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
            const uint32_t pos = round_place<256>(key[k] >> low, d.high_bits, valid, base, wcnt);
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
    const uint32_t start = d.counts[(int64_t)h * d.tiles];
    const uint32_t end = h + 1 < ndig ? d.counts[(int64_t)(h + 1) * d.tiles] : (uint32_t)d.n;
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

size_t random_order_count_bytes(int n, int key_bits)
{
    int tile, tiles;
    random_order_tiles(n, &tile, &tiles);
    const int high = random_order_high_bits(key_bits, tiles);
    const size_t ndig = (size_t)1 << high;
    // Whole blocks of the scan's 1,024 x 64 counts are read: padded to a multiple of 64.
    const size_t m = (ndig < 4 ? 4 : ndig) * (size_t)tiles;
    return (m + 63) / 64 * 64 * sizeof(uint32_t);
}

hipError_t launch_random_order(const RandomOrderDesc &d, hipStream_t s, const uint32_t **order)
{
    int tile, tiles;
    random_order_tiles(d.n, &tile, &tiles);
    if (d.n <= 0 || d.key_bits < 1 || d.key_bits > 16 || d.tile != tile || d.tiles != tiles ||
        d.high_bits != random_order_high_bits(d.key_bits, d.tiles))
        return hipErrorInvalidValue;
    hipLaunchKernelGGL(sort_count_kernel, dim3((unsigned)d.tiles), dim3(kSortThreads), 0, s, d);
    if (d.high_bits == d.key_bits) {
        hipLaunchKernelGGL(sort_one_pass_kernel, dim3((unsigned)d.tiles), dim3(kSortThreads), 0, s, d);
        *order = d.vals;
        return hipGetLastError();
    }
    hipLaunchKernelGGL(sort_scan_kernel, dim3(1), dim3(1024), 0, s, d);
    hipLaunchKernelGGL(sort_scatter_kernel, dim3((unsigned)d.tiles), dim3(kSortThreads), 0, s, d);
    if (d.key_bits > d.high_bits)
        hipLaunchKernelGGL(sort_segment_kernel, dim3(1u << d.high_bits), dim3(kSortThreads), 0, s, d);
    *order = d.vals;
    return hipGetLastError();
}

} // namespace ntk
