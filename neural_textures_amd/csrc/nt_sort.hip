// nt_sort.hip — the sample order of NT_SAMPLES_RANDOM steps. Each sample's texel (the
// placement the train kernel uses: random_texel of its seed) falls in a 64 x 64-texel bin;
// the sample indices are sorted by bin, stably (radix sort, hipCUB), so that consecutive
// slots — one chunk of the train kernel — lie close together in the image and their target
// taps, latent corners and gradient atomics share cache lines in the L2. The kernel reads
// the sample of each slot from the order and places it exactly as before: the samples and
// their results are unchanged, only the order of the fp32 sums (the same for every run:
// the sort is deterministic).
#include <hipcub/hipcub.hpp>

#include "nt_internal.hpp"

namespace ntk {

__global__ __launch_bounds__(256) void random_bin_kernel(RandomOrderDesc d)
{
    const int i = (int)(blockIdx.x * 256 + threadIdx.x);
    if (i >= d.n)
        return;
    uint32_t tx, ty;
    random_texel(mix_seed((uint32_t)i, d.step), d.image_w, d.image_h, tx, ty);
    d.keys[i] = (uint16_t)((ty >> d.bin_shift) * (uint32_t)d.bins_x + (tx >> d.bin_shift));
    d.vals[i] = (uint32_t)i;
}

hipError_t random_order_temp_bytes(int n, int key_bits, size_t *bytes)
{
    hipcub::DoubleBuffer<uint16_t> k(nullptr, nullptr);
    hipcub::DoubleBuffer<uint32_t> v(nullptr, nullptr);
    *bytes = 0;
    const hipError_t e = hipcub::DeviceRadixSort::SortPairs(nullptr, *bytes, k, v, n, 0, key_bits);
    if (e != hipSuccess)
        (void)hipGetLastError();
    return e;
}

hipError_t launch_random_order(const RandomOrderDesc &d, hipStream_t s, const uint32_t **order)
{
    hipLaunchKernelGGL(random_bin_kernel, dim3((unsigned)((d.n + 255) / 256)), dim3(256), 0, s, d);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess)
        return e;
    hipcub::DoubleBuffer<uint16_t> k(d.keys, d.keys_alt);
    hipcub::DoubleBuffer<uint32_t> v(d.vals, d.vals_alt);
    size_t bytes = 0;
    e = hipcub::DeviceRadixSort::SortPairs(nullptr, bytes, k, v, d.n, 0, d.key_bits, s);
    if (e != hipSuccess)
        return e;
    if (bytes > d.temp_bytes)
        return hipErrorInvalidValue; // the planned temporary storage is too small
    bytes = d.temp_bytes;
    e = hipcub::DeviceRadixSort::SortPairs(d.temp, bytes, k, v, d.n, 0, d.key_bits, s);
    *order = v.Current();
    return e;
}

} // namespace ntk
