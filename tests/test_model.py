"""The model container on the CPU: nt_model_bytes / nt_model_save / nt_model_load are host
code, so the whole format is exercised here — the byte layout read back independently of
the library (header, description, section table, 256-byte aligned sections), CRC-32C
checksums recomputed in Python (pinned by the algorithm's published check value), round
trips of both contents, and the rejection of damaged, truncated, foreign-version and
misaligned images. The format has no reference counterpart (the reference writes PNG
renders only, main.cpp:855-904); the GPU round trip through nt_decode is in
test_gpu_parity.py."""
import ctypes as C
import struct

import numpy as np
import pytest

import neural_textures_amd as nt
from neural_textures_amd import abi, params as P
from neural_textures_amd import model as M


@pytest.fixture(scope="module")
def lib():
    return nt.load()


def crc32c(data: bytes) -> int:
    """Bit-serial CRC-32C (reflected polynomial 0x82F63B78, init and final xor ~0)."""
    table = []
    for i in range(256):
        c = i
        for _ in range(8):
            c = (c >> 1) ^ (0x82F63B78 if c & 1 else 0)
        table.append(c)
    crc = 0xFFFFFFFF
    for b in data:
        crc = (crc >> 8) ^ table[(crc ^ b) & 0xFF]
    return crc ^ 0xFFFFFFFF


def test_crc32c_check_value():
    # The published check value of CRC-32C (RFC 3720 appendix B.4 / iSCSI).
    assert crc32c(b"123456789") == 0xE3069283
    assert crc32c(b"") == 0
    assert crc32c(bytes(32)) == 0x8A9136AA  # RFC 3720 B.4: 32 bytes of zeros


def make_model(rng, state=True, codec=True, shapes=((20, 12, 3), (9, 9, 2)), channels=8,
               sizes=(16, 32, 12), used=10, step=17, blocks=False):
    net = P.make_network(list(sizes), used_outputs=used, rng=rng)
    for l in range(net.num_layers):
        net.biases[l] = P.f16_bits(rng.normal(size=sizes[l + 1]))
        net.weight_moment1[l] = rng.normal(size=net.weight_moment1[l].size).astype(np.float32)
        net.weight_moment2[l] = rng.random(net.weight_moment2[l].size).astype(np.float32)
        net.bias_moment1[l] = rng.normal(size=sizes[l + 1]).astype(np.float32)
        net.bias_moment2[l] = rng.random(sizes[l + 1]).astype(np.float32)
    m = M.Model(net, channels, [tuple(s) for s in shapes], step=step if state else 0)
    for w, h, mips in shapes:
        if codec:
            n = P.codec_chain_layout(w, h, mips, channels)[1]
            m.codec.append(M.CodecChain(w, h, mips, channels,
                                        rng.integers(0, 256, n, dtype=np.uint8)))
        if state:
            n = P.mip_chain_layout(w, h, mips)[1] * channels
            grid = P.Grid(w, h, mips, channels,
                          values=rng.normal(size=n).astype(np.float32),
                          moment1=rng.normal(size=n).astype(np.float32),
                          moment2=rng.random(n).astype(np.float32))
            if blocks:
                nb = P.block_chain_layout(w, h, mips)[1]
                grid.block_params = rng.normal(size=nb * (4 * channels + 18)).astype(np.float32)
                grid.block_moment1 = rng.normal(size=nb * (4 * channels + 16)).astype(np.float32)
                grid.block_moment2 = rng.random(nb * (4 * channels + 16)).astype(np.float32)
            m.grids.append(grid)
    return m


SECTION_TYPES = {1: "codec", 2: "weights", 3: "biases", 4: "latents", 5: "latent_moment1",
                 6: "latent_moment2", 7: "weight_moment1", 8: "weight_moment2",
                 9: "bias_moment1", 10: "bias_moment2", 11: "block_params",
                 12: "block_moment1", 13: "block_moment2"}


def expected_sections(m: M.Model):
    """(type, index, bytes) in image order, as the header documents the layout."""
    out = []
    for g, c in enumerate(m.codec):
        out.append((1, g, c.blocks.tobytes()))
    for l in range(m.net.num_layers):
        out.append((2, l, np.asarray(m.net.weights[l], np.uint16).tobytes()))
        out.append((3, l, np.asarray(m.net.biases[l], np.uint16).tobytes()))
    if m.grids:
        for g, grid in enumerate(m.grids):
            for t, a in ((4, grid.values), (5, grid.moment1), (6, grid.moment2)):
                out.append((t, g, a.tobytes()))
        for l in range(m.net.num_layers):
            for t, a in ((7, m.net.weight_moment1[l]), (8, m.net.weight_moment2[l]),
                         (9, m.net.bias_moment1[l]), (10, m.net.bias_moment2[l])):
                out.append((t, l, np.asarray(a, np.float32).tobytes()))
    if m.contents & abi.NT_MODEL_BLOCKS:
        for g, grid in enumerate(m.grids):
            for t, a in ((11, grid.block_params), (12, grid.block_moment1), (13, grid.block_moment2)):
                out.append((t, g, a.tobytes()))
    return out


@pytest.mark.parametrize("state,codec,blocks", [(True, True, False), (True, False, False),
                                                (False, True, False), (True, True, True)])
def test_image_layout_read_back_independently(lib, state, codec, blocks):
    rng = np.random.default_rng(3 + 2 * state + codec + 4 * blocks)
    shapes = ((20, 12, 3), (8, 8, 4)) if blocks else ((20, 12, 3), (9, 9, 2))
    m = make_model(rng, state=state, codec=codec, blocks=blocks, shapes=shapes)
    img = M.model_image(m)
    raw = img.tobytes()
    magic, version, hbytes, nsec, contents, total, meta_crc = struct.unpack_from("<8s4IQI", raw, 0)
    assert magic == b"NTMODEL\0" and version == abi.NT_MODEL_VERSION == 1 and hbytes == 64
    assert contents == m.contents and total == len(raw)
    assert raw[36:64] == bytes(28)
    desc = struct.unpack_from("<32i", raw, 64)
    G, L = len(m.shapes), m.net.num_layers
    want_desc = [m.contents, G, m.channels]
    for k in range(3):
        want_desc += [s[k] for s in m.shapes] + [0] * (4 - G)
    want_desc += [L] + list(m.net.sizes) + [0] * (7 - L - 1) + [m.net.used_outputs, m.step]
    assert list(desc) == want_desc + [0] * (32 - len(want_desc))
    sections = expected_sections(m)
    assert nsec == len(sections)
    assert crc32c(raw[64:192 + 32 * nsec]) == meta_crc
    end = 192 + 32 * nsec
    for i, (t, idx, data) in enumerate(sections):
        typ, index, off, nbytes, crc, res = struct.unpack_from("<IIQQII", raw, 192 + 32 * i)
        assert (typ, index, nbytes, res) == (t, idx, len(data), 0), (i, SECTION_TYPES[t])
        assert off % 256 == 0 and off >= end and off - end < 256
        assert raw[end:off] == bytes(off - end)  # zero padding
        assert raw[off:off + nbytes] == data
        assert crc == crc32c(data)
        end = off + nbytes
    assert end == total
    info = M._info(m)
    assert lib.nt_model_bytes(C.byref(info)) == total


def test_round_trip(lib, tmp_path):
    rng = np.random.default_rng(11)
    m = make_model(rng, blocks=True, shapes=((20, 12, 3), (8, 8, 4)))
    path = str(tmp_path / "tex.ntm")
    n = M.save_model(path, m)
    assert n == (tmp_path / "tex.ntm").stat().st_size
    r = M.load_model(path)
    assert (r.channels, r.shapes, r.step, r.contents) == (m.channels, m.shapes, 17, 7)
    assert r.net.sizes == m.net.sizes and r.net.used_outputs == m.net.used_outputs
    for name in ("weights", "biases", "weight_moment1", "weight_moment2", "bias_moment1",
                 "bias_moment2"):
        for a, b in zip(getattr(r.net, name), getattr(m.net, name)):
            assert np.array_equal(np.asarray(a).view(np.uint8), np.asarray(b).view(np.uint8)), name
    for a, b in zip(r.codec, m.codec):
        assert (a.width, a.height, a.num_mips) == (b.width, b.height, b.num_mips)
        assert np.array_equal(a.blocks, b.blocks)
    for a, b in zip(r.grids, m.grids):
        for name in ("values", "moment1", "moment2", "block_params", "block_moment1",
                     "block_moment2"):
            assert np.array_equal(getattr(a, name).view(np.uint32), getattr(b, name).view(np.uint32))
    # An image saved again from what was loaded is the same bytes.
    assert np.array_equal(M.model_image(r), M.read_image(path))


def test_reference_config_sizes(lib):
    """Config 5's decode model (4 grids of 16 channels, 1024^2 x 9 mips down to 128^2 x 6,
    64-64-64-64-12 network): codec chains at 12 bytes per channel per 4x4 block
    (0.75 byte/channel/texel) plus the fp16 network and the section padding."""
    shapes = [(1024, 1024, 9), (512, 512, 8), (256, 256, 7), (128, 128, 6)]
    sizes = [64, 64, 64, 64, 12]
    info = abi.nt_model_info()
    info.contents, info.num_grids, info.channels = abi.NT_MODEL_CODEC, 4, 16
    for g, (w, h, mips) in enumerate(shapes):
        info.width[g], info.height[g], info.num_mips[g] = w, h, mips
    info.num_layers = len(sizes) - 1
    for i, s in enumerate(sizes):
        info.sizes[i] = s
    info.used_outputs = 12
    codec = sum(P.codec_chain_layout(w, h, mips, 16)[1] for w, h, mips in shapes)
    assert codec == 22281984
    net = sum(2 * abi.pad16(a) * abi.pad16(b) + 2 * b for a, b in zip(sizes, sizes[1:]))
    nsec = 4 + 2 * 4
    total = lib.nt_model_bytes(C.byref(info))
    assert codec + net < total <= codec + net + 192 + 32 * nsec + 256 * nsec


def test_rejects_damaged_images(lib):
    rng = np.random.default_rng(5)
    m = make_model(rng)
    img = M.model_image(m)
    info, data = abi.nt_model_info(), abi.nt_model_data()

    def load(buf, nbytes=None):
        return lib.nt_model_load(buf.ctypes.data, buf.nbytes if nbytes is None else nbytes,
                                 C.byref(info), C.byref(data))

    assert load(img) == abi.NT_OK
    raw = img.tobytes()
    nsec = struct.unpack_from("<I", raw, 16)[0]
    # One flipped bit in any section, in the description or in the table is caught.
    offsets = [struct.unpack_from("<IIQQII", raw, 192 + 32 * i)[2] for i in range(nsec)]
    for pos in [70, 100, 192 + 8, 192 + 32 * (nsec - 1) + 24] + [o + 1 for o in offsets]:
        bad = img.copy()
        bad[pos] ^= 0x10
        assert load(bad) == abi.NT_ERR_FORMAT, pos
    bad = img.copy()
    bad[0] = ord("X")
    assert load(bad) == abi.NT_ERR_FORMAT and b"magic" in lib.nt_last_error()
    bad = img.copy()
    bad[8] = 2  # version 2
    assert load(bad) == abi.NT_ERR_FORMAT and b"version 2" in lib.nt_last_error()
    assert load(img, img.nbytes - 1) == abi.NT_ERR_FORMAT
    assert b"truncated" in lib.nt_last_error()
    assert load(img, 40) == abi.NT_ERR_FORMAT
    mis = M.aligned_bytes(img.nbytes + 8)[8:]
    mis[:] = img
    assert load(mis) == abi.NT_ERR_MISALIGNED
    # A section table entry moved (offset + 256, consistent checksums recomputed) is caught
    # by the layout check, not only by checksums.
    bad = bytearray(raw)
    struct.pack_into("<Q", bad, 192 + 8, offsets[0] + 256)
    struct.pack_into("<I", bad, 32, crc32c(bytes(bad[64:192 + 32 * nsec])))
    buf = M.aligned_bytes(len(bad))
    buf[:] = np.frombuffer(bytes(bad), np.uint8)
    assert load(buf) == abi.NT_ERR_FORMAT and b"expected" in lib.nt_last_error()
    # The Python helper raises with the library's message.
    with pytest.raises(nt.NtError, match="checksum"):
        bad = img.copy()
        bad[offsets[-1]] ^= 1
        M.load_model(bad)


def test_rejects_bad_descriptions(lib):
    rng = np.random.default_rng(9)
    m = make_model(rng, channels=8)
    info = M._info(m)
    assert lib.nt_model_bytes(C.byref(info)) > 0
    for field, value in [("contents", 0), ("contents", 4), ("contents", 8), ("num_grids", 0),
                         ("num_grids", 5),
                         ("channels", 0), ("channels", 17), ("num_layers", 0), ("num_layers", 7),
                         ("used_outputs", 13), ("step", -1)]:
        bad = M._info(m)
        setattr(bad, field, value)
        assert lib.nt_model_bytes(C.byref(bad)) == 0, field
    bad = M._info(m)
    bad.channels = 6  # state-only models may have any channel count; the codec may not
    assert lib.nt_model_bytes(C.byref(bad)) == 0
    bad.contents = abi.NT_MODEL_STATE
    assert lib.nt_model_bytes(C.byref(bad)) > 0
    bad = M._info(m)
    bad.contents, bad.step = abi.NT_MODEL_CODEC, 3  # a step without training state
    assert lib.nt_model_bytes(C.byref(bad)) == 0
    bad = M._info(m)
    bad.width[1] = 0
    assert lib.nt_model_bytes(C.byref(bad)) == 0
    bad = M._info(m)  # block records need sizes that are multiples of 4 (9 is not)
    bad.contents |= abi.NT_MODEL_BLOCKS
    assert lib.nt_model_bytes(C.byref(bad)) == 0
    bad = M._info(m)
    bad.sizes[1] = 1025
    assert lib.nt_model_bytes(C.byref(bad)) == 0
    # Save: a missing buffer, a short or misaligned output.
    info = M._info(m)
    n = lib.nt_model_bytes(C.byref(info))
    out = M.aligned_bytes(n + 16)
    d = abi.nt_model_data()
    assert lib.nt_model_save(C.byref(info), C.byref(d), out.ctypes.data, n) == abi.NT_ERR_NULL_POINTER
    assert b"codec[0]" in lib.nt_last_error()
    img = M.model_image(m)
    good = abi.nt_model_data()
    assert lib.nt_model_load(img.ctypes.data, img.nbytes, C.byref(abi.nt_model_info()),
                             C.byref(good)) == abi.NT_OK
    assert lib.nt_model_save(C.byref(info), C.byref(good), out.ctypes.data, n - 1) \
        == abi.NT_ERR_INVALID_ARGUMENT
    assert lib.nt_model_save(C.byref(info), C.byref(good), out.ctypes.data + 8, n) \
        == abi.NT_ERR_MISALIGNED
    assert lib.nt_model_save(C.byref(info), C.byref(good), out.ctypes.data, n) == abi.NT_OK
    assert np.array_equal(out[:n], img)
    assert lib.nt_status_string(abi.NT_ERR_FORMAT) == b"bad model image"
