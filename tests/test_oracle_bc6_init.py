"""Pins the oracle's BC6 block initialisation (ntref_bc6_init; no reference counterpart:
the reference zero-fills its block records, main.cpp:689-694).

The decode it inverts is the reference's (train.cu:159-181, pinned in
test_oracle_codec_bc6.py). Checks: the value -> y inverse round-trips through the decode
to 2^-10 relative over 12 decades; blocks made by decoding a random two-subset record
(any partition, random endpoints and indices) are recovered to 1e-4 of the block's
largest magnitude per channel, which fails for a swapped subset, a transposed pixel order
or a wrong endpoint mapping; the chosen partition is the least-error one by brute force
over all 32; negative values are fitted as 0 (the decode's range is the unsigned half
range); constant blocks decode to their value; pixels outside a small mip are ignored and
get index 0; the grid walk visits every block of every mip with the right texels.
"""
import ctypes as C

import numpy as np
import pytest

from neural_textures_amd import abi, params as P
from oracle_lib import load_oracle

O = load_oracle()
SETS = [v for v in (0xCCCC, 0x8888, 0xEEEE, 0xECC8, 0xC880, 0xFEEC, 0xFEC8, 0xEC80,
                          0xC800, 0xFFEC, 0xFE80, 0xE800, 0xFFE8, 0xFF00, 0xFFF0, 0xF000,
                          0xF710, 0x008E, 0x7100, 0x08CE, 0x008C, 0x7310, 0x3100, 0x8CCE,
                          0x088C, 0x3110, 0x6666, 0x366C, 0x17E8, 0x0FF0, 0x718E, 0x399C)]


def decode_record(rec, C_):
    """[16][C] values of a block record through the reference decode (mode bits 10)."""
    part = int(rec[4 * C_ + 16:4 * C_ + 17].view(np.int32)[0])
    mask = SETS[part]
    out = np.zeros((16, C_), np.float32)
    for i in range(16):
        s = (mask >> i) & 1
        for c in range(C_):
            out[i, c] = O.ntref_bc6_decompress(float(rec[2 * s * C_ + c]),
                                               float(rec[(2 * s + 1) * C_ + c]), 10,
                                               float(rec[4 * C_ + i]))
    return out


def init_block(v, C_, valid=0xFFFF):
    v = np.ascontiguousarray(v, np.float32).reshape(-1)
    rec = np.zeros(4 * C_ + 18, np.float32)
    O.ntref_bc6_init_block(v.ctypes.data, C_, valid, rec.ctypes.data)
    return rec


def test_value_to_y_inverts_the_decode():
    rng = np.random.default_rng(1)
    vals = np.concatenate([rng.uniform(0, 1, 4000), 10 ** rng.uniform(-7, 4.8, 8000),
                           -rng.uniform(0, 1e-3, 200),
                           [0.0, 2.0 ** -13, 2049 * 2.0 ** -24, 2050 * 2.0 ** -24, 1.0, 65504.0]])
    for v in vals.astype(np.float32):
        y = O.ntref_bc6_value_to_y(float(v))
        # A record whose endpoints unquantize to y exactly: q0 = q1 = y at 10 bits.
        e = (np.float32(y) * np.float32(1024) - np.float32(32768)) / np.float32(31744)
        w = O.ntref_bc6_decompress(float(e), float(e), 10, 0.0)
        # (the endpoint round trip adds ~1e-13 absolute)
        assert abs(w - v) <= 2.0 ** -10 * abs(v) + 1e-12, (v, y, w)
    ys = [O.ntref_bc6_value_to_y(float(v)) for v in np.sort(vals.astype(np.float32))]
    assert all(a <= b for a, b in zip(ys, ys[1:])), "monotone"


@pytest.mark.parametrize("C_", [3, 4, 8, 16])
def test_recovers_blocks_made_by_the_decode(C_):
    rng = np.random.default_rng(10 + C_)
    for trial in range(40):
        part = int(rng.integers(0, 32))
        rec = np.zeros(4 * C_ + 18, np.float32)
        # Unquantized endpoints q (y units), e = (q 2^10 - 32768) / 31744
        # (train.cu:161-166), the segment kept positive: odd trials in the half-float
        # range of y (values ~1e-3 .. 4), even ones in the linear (hy = 0) range.
        lo, hi, up = (9000, 17000, 300) if trial % 2 else (50, 1800, 30)
        q0 = rng.uniform(lo, hi, (2, C_))
        q1 = q0 + rng.uniform(-q0 / 16, up, (2, C_))
        for s in range(2):
            rec[2 * s * C_:(2 * s + 1) * C_] = (q0[s] * 1024 - 32768) / 31744
            rec[(2 * s + 1) * C_:(2 * s + 2) * C_] = (q1[s] * 1024 - 32768) / 31744
        rec[4 * C_:4 * C_ + 16] = rng.uniform(0, 1, 16).astype(np.float32)
        rec[4 * C_ + 16:4 * C_ + 17] = np.array([part], np.int32).view(np.float32)
        v = decode_record(rec, C_)
        got = decode_record(init_block(v, C_), C_)
        scale = np.abs(v).max(axis=0, keepdims=True)
        err = (np.abs(got - v) / scale).max()
        assert err <= 1e-4, (trial, part, err)


@pytest.mark.parametrize("C_", [3, 16])
def test_choice_is_the_least_error_partition(C_):
    rng = np.random.default_rng(30 + C_)
    for trial in range(10):
        v = rng.uniform(0, 1, (16, C_)).astype(np.float32)
        rec = init_block(v, C_)
        part = int(rec[4 * C_ + 16:4 * C_ + 17].view(np.int32)[0])
        mode = int(rec[4 * C_ + 17:4 * C_ + 18].view(np.int32)[0])
        assert 0 <= part < 32 and mode == 0
        assert np.all((rec[4 * C_:4 * C_ + 16] >= 0) & (rec[4 * C_:4 * C_ + 16] <= 1))
        y = np.array([O.ntref_bc6_value_to_y(float(a)) for a in v.reshape(-1)], np.float32)
        tot = []
        for p in range(32):
            s = 0.0
            for sub in (~SETS[p] & 0xFFFF, SETS[p]):
                e0, e1, x = (np.zeros(16, np.float32) for _ in range(3))
                s += O.ntref_bc6_fit_subset(v.ctypes.data, y.ctypes.data, C_, sub, 10,
                                            e0.ctypes.data, e1.ctypes.data, x.ctypes.data)
            tot.append(s)
        assert part == int(np.argmin(tot))
        # The record written decodes with exactly that error (up to summation order).
        err = float(((decode_record(rec, C_).astype(np.float64) - v) ** 2).sum())
        assert abs(err - min(tot)) <= 1e-5 * max(min(tot), 1e-12)


def test_negative_values_clamp_to_zero():
    """The decode cannot reach negative values (unsigned half range): they are fitted as 0,
    and the other texels of the block are unaffected."""
    rng = np.random.default_rng(8)
    v = rng.uniform(0.2, 0.9, (16, 4)).astype(np.float32)
    v[3] = -0.5
    got = decode_record(init_block(v, 4), 4)
    assert np.all(np.abs(got[3]) <= 1e-3)  # near 0 on the scale of the block (~0.5)
    want = np.maximum(v, 0)
    keep = [i for i in range(16) if i != 3]
    assert np.abs(got[keep] - want[keep]).max() <= 0.35  # a two-subset fit of random data
    huge = np.full((16, 4), 1e6, np.float32)
    assert np.allclose(decode_record(init_block(huge, 4), 4), 65504, rtol=2e-3)


def test_constant_block_and_small_mip():
    v = np.full((16, 8), 0.3721, np.float32)
    got = decode_record(init_block(v, 8), 8)
    assert np.abs(got - v).max() <= 2.0 ** -10 * 0.3721
    # A 2x2 mip: only pixels 0, 1, 4, 5 exist.
    rng = np.random.default_rng(4)
    v = rng.uniform(0.1, 1, (16, 4)).astype(np.float32)
    valid = (1 << 0) | (1 << 1) | (1 << 4) | (1 << 5)
    rec = init_block(v, 4, valid)
    x = rec[16:32]
    assert np.all(x[[i for i in range(16) if not (valid >> i) & 1]] == 0)
    got = decode_record(rec, 4)
    for i in (0, 1, 4, 5):
        assert np.abs(got[i] - v[i]).max() <= 0.05 * np.abs(v[i]).max()


def test_grid_init_matches_block_init():
    rng = np.random.default_rng(6)
    C_ = 3
    g = P.make_grid(8, 8, 4, C_, rng, blocks=True)  # mips 8, 4, 2, 1
    lat = abi.nt_latents()
    lat.num_grids, lat.channels = 1, C_
    lat.grids[0] = g.struct()
    assert O.ntref_bc6_init(C.byref(lat)) == 0
    rec_len = 4 * C_ + 18
    blocks = g.block_params.reshape(-1, rec_len)
    for m, boff in enumerate(P.block_chain_layout(8, 8, 4)[0]):
        vm = g.mip(g.values, m)
        h, w, _ = vm.shape
        nbu, nbv = max(w >> 2, 1), max(h >> 2, 1)
        for by in range(nbv):
            for bx in range(nbu):
                v = np.zeros((16, C_), np.float32)
                valid = 0
                for i in range(16):
                    tx, ty = 4 * bx + (i & 3), 4 * by + (i >> 2)
                    if tx < w and ty < h:
                        v[i] = vm[ty, tx]
                        valid |= 1 << i
                want = init_block(v, C_, valid)
                assert np.array_equal(blocks[boff + by * nbu + bx].view(np.uint32), want.view(np.uint32))
