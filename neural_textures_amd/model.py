"""The model container (nt_model_bytes / nt_model_save / nt_model_load) for numpy buffers.

A model image always carries the fp16 network; with codec chains it is what nt_decode
needs (the compressed latents), with training state (fp32 latents, Adam moments, step) a
run can resume from it. The format is written and checked by libnt_hip.so; this module
only lays host arrays out for it and copies a loaded image back into params.Grid /
params.Network objects.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass, field

import numpy as np

from . import abi, check, load
from .params import Grid, Network, block_chain_layout, codec_chain_layout, mip_chain_layout


def aligned_bytes(nbytes: int, align: int = 256) -> np.ndarray:
    """Zeroed uint8 host buffer whose first byte is `align`-byte aligned."""
    raw = np.zeros(nbytes + align, np.uint8)
    start = (-raw.ctypes.data) % align
    return raw[start:start + nbytes]


@dataclass
class CodecChain:
    """One grid quantized with the codec: its mip chain of block records."""
    width: int
    height: int
    num_mips: int
    channels: int
    blocks: np.ndarray  # uint8, codec_chain_layout bytes

    @property
    def byte_offsets(self):
        return codec_chain_layout(self.width, self.height, self.num_mips, self.channels)[0]


@dataclass
class Model:
    """What a model image holds. `grids` (with values/moment1/moment2, and block_params /
    block_moment1/2 when present) only for training state; `codec` only for images with
    codec chains."""
    net: Network
    channels: int
    shapes: list  # (width, height, num_mips) per grid
    codec: list = field(default_factory=list)
    grids: list = field(default_factory=list)
    step: int = 0

    @property
    def contents(self) -> int:
        blocks = bool(self.grids) and self.grids[0].block_params is not None
        return ((abi.NT_MODEL_CODEC if self.codec else 0) | (abi.NT_MODEL_STATE if self.grids else 0)
                | (abi.NT_MODEL_BLOCKS if blocks else 0))


def _host(a, dtype) -> np.ndarray:
    if a is None:
        return None
    if not isinstance(a, np.ndarray):
        a = a.detach().cpu().numpy()
    return np.ascontiguousarray(a).view(dtype) if a.dtype != dtype else np.ascontiguousarray(a)


def _info(m: Model) -> abi.nt_model_info:
    info = abi.nt_model_info()
    info.contents = m.contents
    info.num_grids = len(m.shapes)
    info.channels = m.channels
    for g, (w, h, mips) in enumerate(m.shapes):
        info.width[g], info.height[g], info.num_mips[g] = w, h, mips
    info.num_layers = m.net.num_layers
    for i, s in enumerate(m.net.sizes):
        info.sizes[i] = s
    info.used_outputs = m.net.used_outputs
    info.step = m.step
    return info


def model_image(m: Model) -> np.ndarray:
    """The file image of a model (uint8, 256-byte aligned)."""
    lib = load()
    info = _info(m)
    n = lib.nt_model_bytes(C.byref(info))
    if n == 0:
        check(abi.NT_ERR_INVALID_ARGUMENT)
    keep = []  # host arrays whose addresses the data struct holds

    def ptr(a, dtype):
        a = _host(a, dtype)
        if a is None:
            return None
        keep.append(a)
        return a.ctypes.data

    d = abi.nt_model_data()
    for g, c in enumerate(m.codec):
        d.codec[g] = ptr(c.blocks, np.uint8)
    net = m.net
    for l in range(net.num_layers):
        d.weights[l] = ptr(net.weights[l], np.uint16)
        d.biases[l] = ptr(net.biases[l], np.uint16)
        if m.grids:
            d.weight_moment1[l] = ptr(net.weight_moment1[l], np.float32)
            d.weight_moment2[l] = ptr(net.weight_moment2[l], np.float32)
            d.bias_moment1[l] = ptr(net.bias_moment1[l], np.float32)
            d.bias_moment2[l] = ptr(net.bias_moment2[l], np.float32)
    for g, grid in enumerate(m.grids):
        d.latents[g] = ptr(grid.values, np.float32)
        d.latent_moment1[g] = ptr(grid.moment1, np.float32)
        d.latent_moment2[g] = ptr(grid.moment2, np.float32)
        if m.contents & abi.NT_MODEL_BLOCKS:
            d.block_params[g] = ptr(grid.block_params, np.float32)
            d.block_moment1[g] = ptr(grid.block_moment1, np.float32)
            d.block_moment2[g] = ptr(grid.block_moment2, np.float32)
    out = aligned_bytes(n)
    check(lib.nt_model_save(C.byref(info), C.byref(d), out.ctypes.data, out.nbytes))
    return out


def save_model(path: str, m: Model) -> int:
    """Writes the image of `m` to `path`; returns its size in bytes."""
    img = model_image(m)
    with open(path, "wb") as f:
        f.write(img.tobytes())
    return img.nbytes


def read_image(path: str) -> np.ndarray:
    """A file's bytes in an aligned host buffer (what nt_model_load checks)."""
    with open(path, "rb") as f:
        f.seek(0, 2)
        n = f.tell()
        f.seek(0)
        buf = aligned_bytes(n)
        f.readinto(memoryview(buf))
    return buf


def load_model(src) -> Model:
    """Checks an image (a path or a uint8 array) with nt_model_load and copies it out."""
    lib = load()
    if isinstance(src, str):
        img = read_image(src)
    else:
        img = np.frombuffer(src, np.uint8) if isinstance(src, (bytes, bytearray)) else src
        if img.ctypes.data % 16:
            buf = aligned_bytes(img.nbytes)
            buf[:] = img
            img = buf
    info, d = abi.nt_model_info(), abi.nt_model_data()
    check(lib.nt_model_load(img.ctypes.data, img.nbytes, C.byref(info), C.byref(d)))
    base = img.ctypes.data

    def arr(addr, dtype, count):
        off = addr - base
        return img[off:off + count * np.dtype(dtype).itemsize].view(dtype).copy()

    G, ch = info.num_grids, info.channels
    shapes = [(info.width[g], info.height[g], info.num_mips[g]) for g in range(G)]
    sizes = [info.sizes[i] for i in range(info.num_layers + 1)]
    net = Network(sizes, info.used_outputs)
    state = bool(info.contents & abi.NT_MODEL_STATE)
    for l in range(info.num_layers):
        nw = abi.pad16(sizes[l]) * abi.pad16(sizes[l + 1])
        net.weights.append(arr(d.weights[l], np.uint16, nw))
        net.biases.append(arr(d.biases[l], np.uint16, sizes[l + 1]))
        if state:
            net.weight_moment1.append(arr(d.weight_moment1[l], np.float32, nw))
            net.weight_moment2.append(arr(d.weight_moment2[l], np.float32, nw))
            net.bias_moment1.append(arr(d.bias_moment1[l], np.float32, sizes[l + 1]))
            net.bias_moment2.append(arr(d.bias_moment2[l], np.float32, sizes[l + 1]))
            net.weight_grads.append(np.zeros(nw, np.float32))
            net.bias_grads.append(np.zeros(sizes[l + 1], np.float32))
    m = Model(net, ch, shapes, step=info.step)
    if info.contents & abi.NT_MODEL_CODEC:
        for g, (w, h, mips) in enumerate(shapes):
            n = codec_chain_layout(w, h, mips, ch)[1]
            m.codec.append(CodecChain(w, h, mips, ch, arr(d.codec[g], np.uint8, n)))
    if state:
        for g, (w, h, mips) in enumerate(shapes):
            n = mip_chain_layout(w, h, mips)[1] * ch
            grid = Grid(w, h, mips, ch,
                        values=arr(d.latents[g], np.float32, n),
                        grads=np.zeros(n, np.float32),
                        moment1=arr(d.latent_moment1[g], np.float32, n),
                        moment2=arr(d.latent_moment2[g], np.float32, n))
            if info.contents & abi.NT_MODEL_BLOCKS:
                nb = block_chain_layout(w, h, mips)[1]
                grid.block_params = arr(d.block_params[g], np.float32, nb * (4 * ch + 18))
                grid.block_grads = np.zeros(nb * (4 * ch + 16), np.float32)
                grid.block_moment1 = arr(d.block_moment1[g], np.float32, nb * (4 * ch + 16))
                grid.block_moment2 = arr(d.block_moment2[g], np.float32, nb * (4 * ch + 16))
            m.grids.append(grid)
    return m


def encode_chain(values, width: int, height: int, num_mips: int, channels: int, stream=None):
    """Codec-quantizes a device latent mip chain (torch fp32, [texel][channels], mips back
    to back) with nt_codec_encode, mip by mip; returns the device uint8 chain."""
    import torch

    from . import stream_handle

    lib = load()
    offs, total = codec_chain_layout(width, height, num_mips, channels)
    texel_offs = mip_chain_layout(width, height, num_mips)[0]
    blob = torch.zeros(total, dtype=torch.uint8, device=values.device)
    s = stream_handle(stream)
    for m in range(num_mips):
        w, h = max(width >> m, 1), max(height >> m, 1)
        src = values.data_ptr() + texel_offs[m] * channels * 4
        check(lib.nt_codec_encode(C.c_void_p(src), w, h, channels,
                                  C.c_void_p(blob.data_ptr() + offs[m]), s))
    return blob
