// nt_train_parts.hpp — device pieces shared by the fused train kernels (nt_train.hip,
// nt_train16.hip): LDS layout constants, the transposed activation stores, the dW phase
// on MFMA and the hidden-layer backward recursion.
#pragma once

#include "nt_internal.hpp"

namespace ntk {

template <class S>
struct TrainLayout {
    static constexpr int frag_bytes = S::all_frags() * kWave * 16;
    static constexpr int bias_bytes = ((S::bias_total() * 4 + 15) / 16) * 16;
    static constexpr int max_in = S::K0 > S::H ? S::K0 : S::H;
    static constexpr int max_out = S::H > S::OUT ? S::H : S::OUT;
    static constexpr int xt_rows = 32 * S::t32(max_in);
    static constexpr int dyt_rows = 32 * S::t32(max_out);
    // LDS: weight fragments | fp32 biases | latent footprint box (runtime size) | a union of
    // the chunk's target tile, the layer transposes and the scatter matrices (runtime size).
    static constexpr int head_bytes = frag_bytes + bias_bytes;
    static constexpr int transpose_bytes = (xt_rows + dyt_rows) * kRowStride * 2;
    static constexpr int slots = (S::dw_total() + 3) / 4;
};

// Wrap for coordinates within one period of the image: training positions are clamped into
// the image (train.cu:838-841), so every bilinear corner lies in [-1, size].
__device__ __forceinline__ int wrap_near(int c, int size)
{
    return c < 0 ? c + size : (c >= size ? c - size : c);
}

// Write fragments transposed into an LDS tile [feature][sample] (fp16).
template <int NQ, bool CHAINED>
__device__ __forceinline__ void store_transposed(_Float16 *buf, const h8 (&v)[NQ], int col, int g)
{
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int row = CHAINED ? chained_feature(q, g, e) : natural_feature(q, g, e);
            buf[row * kRowStride + col] = v[q][e];
        }
}

// dW += X^T dY over one 128-sample chunk for the dW tiles this wave owns, and the
// bias-gradient row sums (mlp.h:101-220).
template <class S, int l>
__device__ __forceinline__ void dw_phase(const _Float16 *xt, const _Float16 *dyt,
                                         f16v (&acc)[TrainLayout<S>::slots], float &db,
                                         int wave, int lane, int tid)
{
    constexpr int kin = S::kin(l), kout = S::kout(l);
    constexpr int KB = S::t32(kin), NA = S::t32(kout);
    constexpr int start = S::dw_start(l), ntiles = NA * KB;
    const int c = lane & 31, g = lane >> 5;
#pragma unroll
    for (int j = 0; j < TrainLayout<S>::slots; ++j) {
        const int t = 4 * j + wave - start;
        if (t >= 0 && t < ntiles) {
            const int a = t / KB, b = t % KB;
            const bool arow = 32 * a + c < kout, brow = 32 * b + c < kin;
            const _Float16 *pa = dyt + (32 * a + c) * kRowStride + 8 * g;
            const _Float16 *pb = xt + (32 * b + c) * kRowStride + 8 * g;
#pragma unroll
            for (int q = 0; q < kChunk / 16; ++q) {
                h8 A = *(const h8 *)(pa + 16 * q);
                h8 B = *(const h8 *)(pb + 16 * q);
                if (!arow)
                    A = (h8)(_Float16)0.f;
                if (!brow)
                    B = (h8)(_Float16)0.f;
                acc[j] = mfma32(A, B, acc[j]);
            }
        }
    }
    if (tid < 4 * kout) {
        const int n = tid >> 2, part = tid & 3;
        const h8 *row = (const h8 *)(dyt + n * kRowStride + 32 * part);
        // fp32 sum of 32 fp16 values, two per v_dot2_f32_f16 (exact products by one).
        const h2 one = {(_Float16)1.f, (_Float16)1.f};
        float s = 0.f;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const h8 r = row[k];
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                const h2 pair = {r[e], r[e + 1]};
                s = __builtin_amdgcn_fdot2(pair, one, s, false);
            }
        }
        s += __shfl_xor(s, 1);
        s += __shfl_xor(s, 2);
        if (part == 0)
            db += s;
    }
}

__device__ __forceinline__ f4v mfma16(h8 a, h8 b, f4v c)
{
    // D(16x16) += A(16x32) B(32x16): lane l holds A[l%16][8(l/16)+i], B[8(l/16)+i][l%16],
    // D[4(l/16)+r][l%16].
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// Backward through hidden layer l (its input is hidden activation l-1), then l-1 ... 1.
template <class S, int l>
__device__ __forceinline__ void backward_hidden(_Float16 *xt, _Float16 *dyt, const h8 *frags,
                                                const h8 (&xh)[S::NH][S::H / 16],
                                                h8 (&dyh)[S::H / 16],
                                                f16v (&dwacc)[TrainLayout<S>::slots],
                                                float (&dbacc)[S::L], int col, int wave, int lane,
                                                int tid)
{
    if constexpr (l >= 1) {
        constexpr int HQ = S::H / 16, HA = S::t32(S::H);
        const int g = lane >> 5;
        store_transposed<HQ, true>(dyt, dyh, col, g);
        store_transposed<HQ, true>(xt, xh[l - 1], col, g);
        f16v acc[HA];
        layer_backward_dx<HQ, HA>(frags + S::bwd_off(l) * kWave, dyh, acc, lane);
        relu_backward<HQ, HA>(acc, xh[l - 1], dyh);
        __syncthreads();
        dw_phase<S, l>(xt, dyt, dwacc, dbacc[l], wave, lane, tid);
        __syncthreads();
        backward_hidden<S, l - 1>(xt, dyt, frags, xh, dyh, dwacc, dbacc, col, wave, lane, tid);
    }
}

} // namespace ntk
