"""Pins the oracle's block codec (the build's own format) and the reference's BC6 emulation.

Codec: order-key bijection and monotonicity over all fp16 patterns, endpoint and index
invariants checked by brute force, round-trip error bounds. BC6 (train.cu:159-202,
373-458): the zeroed-block value 2^-19, the integer-y -> fp16 bit-pattern identity, the
standard partition masks and finite-difference gradients.
"""
import ctypes as C

import numpy as np
import pytest

from neural_textures_amd import abi, params as P
from oracle_lib import load_oracle

O = load_oracle()
WEIGHTS = [0, 4, 9, 13, 17, 21, 26, 30, 34, 38, 43, 47, 51, 55, 60, 64]


def test_order_key_is_a_monotone_bijection():
    bits = np.arange(65536, dtype=np.uint16)
    keys = np.array([O.ntref_codec_key(int(b)) for b in bits], np.uint16)
    assert len(np.unique(keys)) == 65536
    assert all(O.ntref_codec_unkey(int(k)) == int(b) for b, k in zip(bits[::97], keys[::97]))
    vals = bits.view(np.float16).astype(np.float64)
    fin = np.isfinite(vals)
    order = np.argsort(keys[fin], kind="stable")
    assert np.all(np.diff(vals[fin][order]) >= 0)  # sorting by key sorts by value


def test_interp_endpoints_and_monotone():
    rng = np.random.default_rng(20)
    for _ in range(200):
        k0, k1 = sorted(rng.integers(0, 65536, 2))
        seq = [O.ntref_codec_interp(int(k0), int(k1), i) for i in range(16)]
        assert seq[0] == k0 and seq[15] == k1
        assert all(a <= b for a, b in zip(seq, seq[1:]))
        assert seq == [(k0 * (64 - w) + k1 * w + 32) >> 6 for w in WEIGHTS]


def _encode(values, w, h, c):
    blocks = np.zeros(((w + 3) // 4) * ((h + 3) // 4) * 12 * c, np.uint8)
    assert O.ntref_codec_encode(values.ctypes.data, w, h, c, blocks.ctypes.data) == 0
    return blocks


def _decode(blocks, w, h, c):
    out = np.zeros(w * h * c, np.float32)
    assert O.ntref_codec_decode(blocks.ctypes.data, w, h, c, out.ctypes.data) == 0
    return out


def _candidates(k0, k1):
    ks = [O.ntref_codec_interp(k0, k1, i) for i in range(16)]
    return np.array([O.ntref_codec_unkey(k) for k in ks], np.uint16).view(np.float16).astype(np.float32)


@pytest.mark.parametrize("w,h,c", [(8, 8, 4), (6, 5, 8), (4, 4, 16), (3, 2, 12)])
def test_encode_invariants_by_brute_force(w, h, c):
    rng = np.random.default_rng(21 + c)
    vals = rng.normal(0, 0.5, size=w * h * c).astype(np.float32)
    vals[:c] = 0.0
    blocks = _encode(vals, w, h, c)
    img = vals.reshape(h, w, c)
    bw = (w + 3) // 4
    for by in range((h + 3) // 4):
        for bx in range(bw):
            rec = blocks[(by * bw + bx) * 12 * c:(by * bw + bx + 1) * 12 * c]
            ends = rec[:4 * c].view(np.uint16)
            for ch in range(c):
                px = [(y, x) for y in range(4 * by, min(4 * by + 4, h)) for x in range(4 * bx, min(4 * bx + 4, w))]
                keys = [O.ntref_codec_key(int(np.float16(img[y, x, ch]).view(np.uint16))) for y, x in px]
                assert ends[2 * ch] == min(keys) and ends[2 * ch + 1] == max(keys)
                cand = _candidates(int(ends[2 * ch]), int(ends[2 * ch + 1]))
                for y, x in px:
                    p = (y & 3) * 4 + (x & 3)
                    nib = (rec[4 * c + p * (c // 2) + ch // 2] >> (4 * (ch & 1))) & 15
                    err = np.abs(img[y, x, ch] - cand)
                    assert nib == int(np.argmin(err))  # the best index, lowest on ties


def test_round_trip_error_bound_and_constant_blocks():
    rng = np.random.default_rng(22)
    w = h = 16
    c = 16
    vals = rng.normal(0, 0.5, size=w * h * c).astype(np.float32)
    vals.reshape(h, w, c)[:4, :4, :] = 0.3  # a constant block decodes to fp16(0.3)
    out = _decode(_encode(vals, w, h, c), w, h, c)
    img, dec = vals.reshape(h, w, c), out.reshape(h, w, c)
    assert np.all(dec[:4, :4, :] == np.float32(np.float16(0.3)))
    for by in range(4):
        for bx in range(4):
            blk = img[4 * by:4 * by + 4, 4 * bx:4 * bx + 4]
            dblk = dec[4 * by:4 * by + 4, 4 * bx:4 * bx + 4]
            for ch in range(c):
                lo = np.float16(blk[..., ch].min()).view(np.uint16)
                hi = np.float16(blk[..., ch].max()).view(np.uint16)
                cand = _candidates(O.ntref_codec_key(int(lo)), O.ntref_codec_key(int(hi)))
                gap = np.max(np.diff(np.sort(cand))) if len(cand) > 1 else 0
                assert np.max(np.abs(dblk[..., ch] - blk[..., ch])) <= gap / 2 + 1e-3


# ---- BC6 emulation (train.cu:19-35, 159-202) ------------------------------------------

STANDARD_MASK_PIXELS = {  # BC6H/BC7 two-subset partitions 0..3 as per-pixel subset ids
    0: [0, 0, 1, 1, 0, 0, 1, 1, 0, 0, 1, 1, 0, 0, 1, 1],
    1: [0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 0, 1, 0, 0, 0, 1],
    2: [0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 1, 0, 1, 1, 1],
    13: [0, 0, 0, 0, 0, 0, 0, 0, 1, 1, 1, 1, 1, 1, 1, 1],
}


def test_partition_masks():
    sets = C.c_int * 32
    table = list(sets.in_dll(O, "ntref_bc6_partition_sets"))
    for p, pix in STANDARD_MASK_PIXELS.items():
        assert table[p] == sum(b << i for i, b in enumerate(pix))
    assert all((m & 1) == 0 and m != 0 for m in table)  # pixel 0 anchors subset 0
    assert list((C.c_int * 10).in_dll(O, "ntref_bc6_partition_bits")) == [10, 7, 11, 11, 11, 9, 8, 8, 8, 6]


def test_zeroed_block_decodes_to_2_pow_minus_19():
    assert O.ntref_bc6_decompress(0.0, 0.0, 10, 0.0) == 2.0 ** -19


def test_integer_y_is_the_fp16_bit_pattern():
    """e0 = k with b = 10 gives y = 31k + 32 exactly; the decode must equal the fp16 whose
    bit pattern is y (train.cu:169-182)."""
    for k in range(0, 985, 7):
        y = 31 * k + 32
        want = np.array([y], np.uint16).view(np.float16).astype(np.float32)[0]
        assert O.ntref_bc6_decompress(float(k), float(k), 10, 0.0) == want


def test_bc6_backward_matches_finite_differences():
    rng = np.random.default_rng(23)
    g = P.make_grid(8, 8, 1, 3, rng, blocks=True)
    lat = abi.nt_latents()
    lat.num_grids, lat.channels = 1, 3
    lat.grids[0] = g.struct()
    rec = 4 * 3 + 16
    params = g.block_params.reshape(-1, rec + 2)
    params.view(np.int32)[:, rec + 1] = 0  # mode 0: 10 bits
    params[:, :12] = rng.uniform(0.02, 0.2, size=(params.shape[0], 12))
    params[:, 12:rec] = rng.uniform(0.0, 0.1, size=(params.shape[0], 16))
    u, v = 0.4, 0.7
    gvec = np.array([1.0, -0.5, 0.25], np.float16)
    g.block_grads[:] = 0
    O.ntref_scatter_bc6(C.byref(lat), (C.c_float * 3)(u, v, 0.0),
                        gvec.view(np.uint16).ctypes.data_as(C.POINTER(C.c_uint16)))

    def loss():
        out = (C.c_uint16 * 3)()
        O.ntref_sample_latents_bc6(C.byref(lat), (C.c_float * 3)(u, v, 0.0), out)
        # fp16 output rounding is too coarse for FD; evaluate the fp32 decode instead
        tot = 0.0
        for corner, (x, y, w) in enumerate(_corners(u, v)):
            b = (y >> 2) * 2 + (x >> 2)
            pix = ((y & 3) << 2) + (x & 3)
            r = params[b]
            part = (table[int(r.view(np.int32)[rec]) & 31] >> pix) & 1
            for ch in range(3):
                val = O.ntref_bc6_decompress(float(r[2 * part * 3 + ch]), float(r[(2 * part + 1) * 3 + ch]), 10,
                                             float(r[12 + pix]))
                tot += w * val * float(gvec[ch])
        return tot

    table = list((C.c_int * 32).in_dll(O, "ntref_bc6_partition_sets"))
    grads = g.block_grads.reshape(-1, rec)
    touched = np.argwhere(grads != 0)
    assert len(touched) > 0
    for b, k in touched[:12]:
        old = params[b, k]
        eps = 1e-3 * max(abs(old), 1e-2)
        params[b, k] = old + eps
        lp = loss()
        params[b, k] = old - eps
        lm = loss()
        params[b, k] = old
        fd = (lp - lm) / (2 * eps)
        assert abs(grads[b, k] - fd) <= 2e-2 * abs(fd) + 1e-9, (b, k, grads[b, k], fd)


def _corners(u, v, size=8):
    tu, tv = np.float32(u) * size - 0.5, np.float32(v) * size - 0.5
    x0, y0 = int(np.floor(tu)), int(np.floor(tv))
    fx, fy = tu - x0, tv - y0
    out = []
    for c in range(4):
        cx, cy = c & 1, c >> 1
        w = (fx if cx else 1 - fx) * (fy if cy else 1 - fy)
        out.append(((x0 + cx) % size, (y0 + cy) % size, float(w)))
    return out
