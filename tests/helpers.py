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
    # the reference network with three float4 textures of the image size (the fused kernel's
    # 3-channel variant): grids as main.cpp's BCf-0.5k mode on a 2048^2 image ...
    "ref16": dict(sizes=[12, 32, 32, 16], C=3, grids=[(0.25, 4), (0.125, 4), (0.0625, 3), (0.03125, 3)],
                  tex=[3, 3, 3]),
    # ... and as its default BCf-2k mode on a 2048^2 image, whose finest grid leaves the MFMA
    # reduction (its chunk cell box is too large) and sums its corners in per-tile LDS boxes
    "ref16f": dict(sizes=[12, 32, 32, 16], C=3, grids=[(1.0, 4), (0.5, 4), (0.25, 3), (0.125, 3)],
                   tex=[3, 3, 3]),
    # ... and as BCf-2k++ (main.cpp:76): two grids as fine as the image
    "ref16ff": dict(sizes=[12, 32, 32, 16], C=3, grids=[(1.0, 4), (1.0, 4), (0.25, 3), (0.125, 3)],
                    tex=[3, 3, 3]),
    # ... and a grid finer than the image (1.5x: its box takes per-corner LDS adds or, without
    # room, global atomics) beside one of half the image (its box gathers records)
    "ref16u": dict(sizes=[12, 32, 32, 16], C=3, grids=[(1.5, 4), (0.5, 4), (0.25, 3), (0.125, 3)],
                   tex=[3, 3, 3]),
    # ... and as BCf-1k: only the finest grid leaves the MFMA reduction, the others keep it
    "ref16h": dict(sizes=[12, 32, 32, 16], C=3, grids=[(0.5, 4), (0.25, 4), (0.125, 3), (0.0625, 3)],
                   tex=[3, 3, 3]),
    # BASELINE config 1's network: one grid of 8 channels, 8 -> 64 -> 64 -> 3 (half and full
    # the image's size)
    "c1": dict(sizes=[8, 64, 64, 3], C=8, grids=[(0.5, 3)], tex=[3]),
    "c1f": dict(sizes=[8, 64, 64, 3], C=8, grids=[(1.0, 3)], tex=[3]),
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


def check_loss_curves(curve, tol=0.10, early=400, tail=5):
    """curve: (step, oracle MSE, gpu MSE) checkpoints. Both runs add latent gradients with
    float atomics in no fixed order (the oracle with OpenMP atomics), so the trajectories
    are equal only up to rounding early on and then drift apart as any two runs of either
    implementation do (late checkpoints of one implementation vary by ~10 % from run to
    run). Checked: the oracle's loss falls; every checkpoint up to `early` agrees within
    `tol`; the mean of the last `tail` checkpoints agrees within `tol`."""
    assert curve[-1][1] < 0.25 * curve[0][1], "the oracle's loss must fall"
    for i, c, g in curve:
        if i <= early:
            assert abs(g - c) <= tol * c, f"step {i}: gpu {g} vs oracle {c}"
    mc = float(np.mean([c for _, c, _ in curve[-tail:]]))
    mg = float(np.mean([g for _, _, g in curve[-tail:]]))
    assert abs(mg - mc) <= tol * mc, f"last {tail} checkpoints: gpu mean {mg} vs oracle mean {mc}"


def rel_err(a, b):
    a = np.asarray(a, np.float64).reshape(-1)
    b = np.asarray(b, np.float64).reshape(-1)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / den) if den > 0 else float(np.linalg.norm(a))


def assert_close(got, want, name, alt=None, tol=1e-2, floor=1e-3, outliers=1e-4, loose=1e-2):
    """The MLP-tolerance bar, norm-wise and per element.

    Norm-wise: ||got - want|| <= tol * ||want|| over the whole buffer. Per element:
    |got - want| <= tol * |want| + floor * max|want| + 2 |alt - want| (the strict bound), so
    that a miss confined to a few hundred elements (a wrap column, a tile seam, one fallback
    path) fails even where it moves the norm of a large buffer by little.

    `alt` is the oracle's result for the same step with its MLP sums accumulated in fp32
    instead of float64 (ntref_set_mlp_accum_f32): an element that a one-ulp fp16 rounding
    upstream moves (a pre-activation at zero that flips a ReLU mask, a loss gradient rounded
    the other way) differs between the two, and twice that spread is its own allowance for
    the GPU's third accumulation order. Beyond it, at most max(8, outliers * n) elements may
    leave the strict bound, and none the loose one (loose instead of floor). A failure
    names the worst element by its index in the buffer's own shape (texel, channel)."""
    a = np.asarray(to_np(got), np.float64)
    b = np.asarray(to_np(want), np.float64).reshape(a.shape)
    e = rel_err(a, b)
    assert e <= tol, f"{name}: norm-wise relative error {e:.3e} > {tol}"
    if b.size == 0:
        return
    m = float(np.abs(b).max())
    diff = np.abs(a - b)
    spread = 0.0 if alt is None else 2.0 * np.abs(np.asarray(to_np(alt), np.float64).reshape(a.shape) - b)

    def worst(bound):
        excess = diff - bound
        i = int(np.argmax(excess))
        idx = tuple(int(k) for k in np.unravel_index(i, a.shape))
        return (int(np.count_nonzero(excess > 0)),
                f"worst at index {idx}: got {a.flat[i]:.6e}, ref {b.flat[i]:.6e}, bound {bound.flat[i]:.3e} "
                f"(max|ref| {m:.3e})")

    n_loose, msg = worst(tol * np.abs(b) + loose * m + spread)
    assert n_loose == 0, f"{name}: {n_loose} element(s) outside tol*|ref| + {loose}*max|ref| + spread; {msg}"
    n_strict, msg = worst(tol * np.abs(b) + floor * m + spread)
    allowed = max(8, int(outliers * b.size))
    assert n_strict <= allowed, (f"{name}: {n_strict} element(s) (> {allowed}) outside tol*|ref| + "
                                 f"{floor}*max|ref| + spread; {msg}")


def oracle_step(O, st, ktype, threads=1, accum_f32=False):
    """ntref_train_step on `st`, with the MLP sums in fp32 when accum_f32."""
    O.ntref_set_mlp_accum_f32(1 if accum_f32 else 0)
    try:
        assert O.ntref_train_step(C.byref(st.params()), ktype, threads) == 0
    finally:
        O.ntref_set_mlp_accum_f32(0)


def to_np(x):
    return x if isinstance(x, np.ndarray) else x.detach().cpu().numpy()


def gpu_workspace(lib, st, ktype):
    import torch

    p = st.params()
    nbytes = lib.nt_train_workspace_bytes(C.byref(p), ktype)
    assert nbytes > 0, lib.nt_last_error().decode()
    st.workspace = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    return st
