"""Seeded configurations and runners shared by the parity tests.

States are built on the host (numpy). The oracle runs on one copy; the HIP library runs on
a torch copy of the same arrays; results are compared with the tolerances the tests state.
"""
import ctypes as C

import numpy as np

from neural_textures_amd import abi, params as P

# (MLP sizes, channels per grid, grid resolutions as fractions of the image, mips)
SHAPES = {
    # the reference network: 4 grids x 3 channels, 12 -> 32 -> 32 -> 16 (train.h:9-20)
    "ref": dict(sizes=[12, 32, 32, 16], C=3, grids=[(1.0, 4), (0.5, 4), (0.25, 3), (0.125, 3)],
                tex=[3, 3, 1]),
    # 2 grids x 16 channels, 32 -> 64 -> 64 -> 9
    "c2": dict(sizes=[32, 64, 64, 9], C=16, grids=[(0.25, 3), (0.125, 3)], tex=[3, 3, 3]),
    # BASELINE configs 4/5: 4 grids x 16 channels, 64 -> 64 -> 64 -> 64 -> 12
    "c4": dict(sizes=[64, 64, 64, 64, 12], C=16,
               grids=[(0.25, 4), (0.125, 4), (0.0625, 3), (0.03125, 3)], tex=[4, 4, 4]),
}


def make_state(shape, image=128, region=(64, 32), seed=0, init="xavier", blocks=False,
               offset=(0, 0), step=0):
    cfg = SHAPES[shape]
    rng = np.random.default_rng(seed)
    grids = []
    for frac, mips in cfg["grids"]:
        size = max(int(image * frac), 4)
        grids.append(P.make_grid(size, size, mips, cfg["C"], rng, blocks=blocks))
    nout = sum(1 if c == 1 else min(c, 4) for c in cfg["tex"])
    net = P.make_network(cfg["sizes"], used_outputs=min(nout, cfg["sizes"][-1]), rng=rng, init=init)
    textures = []
    for c in cfg["tex"]:
        data = rng.uniform(0.0, 1.0, size=(image, image, 4)).astype(np.float32)
        textures.append(P.make_texture(image, image, c, data))
    rw, rh = region
    return P.TrainState(grids, net, textures, image, image, rw * rh, region_width=rw,
                        texel_offset_x=offset[0], texel_offset_y=offset[1], step=step,
                        network_adam=(0.9, 0.999, 5e-3, 1e-8), feature_adam=(0.9, 0.999, 1e-2, 1e-8))


def rel_err(a, b):
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a))


def to_np(x):
    return x if isinstance(x, np.ndarray) else x.detach().cpu().numpy()


def gpu_workspace(lib, st, ktype):
    import torch

    p = st.params()
    nbytes = lib.nt_train_workspace_bytes(C.byref(p), ktype)
    assert nbytes > 0, lib.nt_last_error().decode()
    st.workspace = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    return st
