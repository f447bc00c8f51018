"""Seeded synthetic inputs for the benchmark configurations (no datasets: reference
textures, latents and weights are generated).

Target channel c of a W x H texture:
    clamp(0.5 + 0.25 * value_noise_c(x, y) + 0.25 * sin(2 pi (fx_c x / W + fy_c y / H) + phi_c), 0, 1)
value_noise_c: a lattice of U[-1, 1] values every `cell` pixels with smoothstep interpolation;
fx_c, fy_c in {1..8} and phi_c in [0, 2 pi) are drawn per channel from the seed.
Latents are U[-1, 1]; codec test latents N(0, 0.5). Everything is generated with torch on the
requested device from torch.Generator seeds, so device-side generation needs no host copy.
"""
from __future__ import annotations

import math

import numpy as np

from . import params as P


def _gen(seed: int, device):
    import torch

    g = torch.Generator(device=device)
    g.manual_seed(int(seed))
    return g


def value_noise(height: int, width: int, cell: int, seed: int, device):
    import torch

    g = _gen(seed, device)
    gh, gw = height // cell + 2, width // cell + 2
    lattice = torch.rand(gh, gw, generator=g, device=device) * 2 - 1
    ys = torch.arange(height, device=device, dtype=torch.float32) / cell
    xs = torch.arange(width, device=device, dtype=torch.float32) / cell
    y0, x0 = ys.floor().long(), xs.floor().long()
    fy, fx = ys - y0, xs - x0
    fy, fx = fy * fy * (3 - 2 * fy), fx * fx * (3 - 2 * fx)
    v00 = lattice[y0][:, x0]
    v01 = lattice[y0][:, x0 + 1]
    v10 = lattice[y0 + 1][:, x0]
    v11 = lattice[y0 + 1][:, x0 + 1]
    fx, fy = fx[None, :], fy[:, None]
    return (v00 * (1 - fx) + v01 * fx) * (1 - fy) + (v10 * (1 - fx) + v11 * fx) * fy


def target_channel(height: int, width: int, seed: int, device, cell: int = 32):
    import torch

    rng = np.random.default_rng(seed)
    fx, fy = int(rng.integers(1, 9)), int(rng.integers(1, 9))
    phi = float(rng.uniform(0, 2 * math.pi))
    ys = torch.arange(height, device=device, dtype=torch.float32)[:, None] / height
    xs = torch.arange(width, device=device, dtype=torch.float32)[None, :] / width
    wave = torch.sin(2 * math.pi * (fx * xs + fy * ys) + phi)
    return (0.5 + 0.25 * value_noise(height, width, cell, seed, device) + 0.25 * wave).clamp_(0, 1)


def target_textures(width: int, height: int, channels: int, per_texture: int, seed: int,
                    device) -> list:
    """`channels` target channels packed into textures of `per_texture` (<= 4) channels,
    pitch 4, mip 0 only (the training target of the reference, train.cu:105-157)."""
    import torch

    textures, c = [], 0
    while c < channels:
        n = min(per_texture, channels - c)
        t = torch.zeros(height, width, 4, device=device)
        for k in range(n):
            t[:, :, k] = target_channel(height, width, seed * 1000 + c + k, device)
        textures.append(P.Texture(width, height, n, t.reshape(-1), 1, 4, 1.0))
        c += n
    return textures


def latent_grid(width: int, height: int, num_mips: int, channels: int, seed: int, device,
                low: float = -1.0, high: float = 1.0, adam: bool = True) -> P.Grid:
    import torch

    g = P.Grid(width, height, num_mips, channels)
    n = g.texels * channels
    gen = _gen(seed, device)
    g.values = torch.rand(n, generator=gen, device=device) * (high - low) + low
    if adam:
        g.grads = torch.zeros(n, device=device)
        g.moment1 = torch.zeros(n, device=device)
        g.moment2 = torch.zeros(n, device=device)
    return g


def normal_values(n: int, sigma: float, seed: int, device):
    import torch

    return torch.randn(n, generator=_gen(seed, device), device=device) * sigma
