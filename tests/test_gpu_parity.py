"""Parity of the HIP library (through the C ABI, on cuda:0) with the CPU oracle on the same
seeded inputs.

Bars (written per test): bit-exact for sampled fp16 features, targets-derived integer
work, codec blocks and Adam updates (same IEEE operations in the same order);
<= 1e-2 relative (norm) for fp16-MLP-derived outputs and gradients, whose fp32 MFMA
accumulation order differs from the oracle's float64 sums.
"""
import ctypes as C
import json
import os

import numpy as np
import pytest

import neural_textures_amd as nt
from neural_textures_amd import abi, params as P
from helpers import assert_close, make_state, oracle_step, rel_err, to_np, gpu_workspace
from oracle_lib import load_oracle

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "forward_pass_test.json")
MLP_TOL = 1e-2


@pytest.fixture(scope="module")
def lib():
    import torch
    assert torch.cuda.is_available()
    return nt.load()


@pytest.fixture(scope="module")
def O():
    return load_oracle()


def sync():
    import torch
    torch.cuda.synchronize()


def say(msg):
    print(msg, flush=True)


# ---- MLP forward -----------------------------------------------------------------------

def test_mlp_forward_known_answer(lib, O):
    """tests/forward_pass_test.cu: |out - expected| <= 2e-2 (:236) on the HIP path."""
    import torch
    say("case: mlp_forward forward_pass_test fixture")
    d = json.load(open(GOLDEN))
    net = P.Network([12, 16, 16], 16)
    net.weights = [np.array(d["w0_f16_bits"], np.uint16), np.array(d["w1_f16_bits"], np.uint16)]
    net.biases = [np.array(d["b0_f16_bits"], np.uint16), np.array(d["b1_f16_bits"], np.uint16)]
    inputs = np.array(d["inputs_f16_bits"], np.uint16)
    expected = np.array(d["expected"], np.float32).reshape(32, 16)
    gnet = net.converted(True, "cuda")
    gin = torch.from_numpy(inputs.astype(np.int16)).cuda()
    gout = torch.zeros(32 * 16, dtype=torch.int16, device="cuda")
    m = gnet.struct()
    nt.check(lib.nt_mlp_forward(C.byref(m), gin.data_ptr(), gout.data_ptr(), 32, None))
    sync()
    got = gout.cpu().numpy().view(np.float16).astype(np.float32).reshape(32, 16)
    assert np.max(np.abs(got - expected)) <= d["tolerance_abs"]
    oracle = np.zeros(32 * 16, np.uint16)
    assert O.ntref_mlp_forward(C.byref(net.struct()), inputs.ctypes.data, oracle.ctypes.data, 32) == 0
    assert rel_err(got, oracle.view(np.float16).astype(np.float32).reshape(32, 16)) <= 2e-3


@pytest.mark.parametrize("sizes", [[12, 32, 32, 16], [8, 64, 64, 3], [32, 64, 64, 9],
                                   [64, 64, 64, 64, 12], [12, 16, 16]])
@pytest.mark.parametrize("count", [1, 33, 1000])
def test_mlp_forward_random(lib, O, sizes, count):
    import torch
    say(f"case: mlp_forward sizes={sizes} count={count}")
    rng = np.random.default_rng(len(sizes) * 100 + count)
    net = P.make_network(sizes, rng=rng, init="xavier")
    for l in range(net.num_layers):
        net.biases[l] = P.f16_bits(rng.uniform(-0.1, 0.1, sizes[l + 1]))
    x = P.f16_bits(rng.uniform(-1, 1, size=count * sizes[0]))
    gnet = net.converted(True, "cuda")
    gin = torch.from_numpy(x.astype(np.int16)).cuda()
    gout = torch.zeros(count * sizes[-1], dtype=torch.int16, device="cuda")
    nt.check(lib.nt_mlp_forward(C.byref(gnet.struct()), gin.data_ptr(), gout.data_ptr(), count, None))
    sync()
    got = gout.cpu().numpy().view(np.float16).astype(np.float32)
    want = np.zeros(count * sizes[-1], np.uint16)
    assert O.ntref_mlp_forward(C.byref(net.struct()), x.ctypes.data, want.ctypes.data, count) == 0
    want = want.view(np.float16).astype(np.float32)
    assert_close(got, want, "outputs")
    assert np.max(np.abs(got - want)) <= 2e-2 * max(1.0, np.max(np.abs(want)))


# ---- latent sample + forward (nt_forward) ------------------------------------------------

@pytest.mark.parametrize("shape", ["ref", "c2", "c4"])
@pytest.mark.parametrize("filt", [abi.NT_FILTER_BILINEAR, abi.NT_FILTER_CATMULL_ROM])
def test_forward_features_bit_exact(lib, O, shape, filt):
    import torch
    say(f"case: forward shape={shape} filter={filt}")
    st = make_state(shape, image=64, region=(32, 8), seed=3)
    rng = np.random.default_rng(30)
    n = 777
    uvz = rng.uniform(0, 1, size=(n, 3)).astype(np.float32)
    uvz[:, 2] = rng.uniform(0, 3.5, n) if filt == abi.NT_FILTER_BILINEAR else 0.0
    uvz[:5, :2] = [[0, 0], [1, 1], [0.999, 0.0001], [0.5, 0.5], [1e-7, 0.9999999]]
    F = st.net.sizes[0]
    no = st.net.sizes[-1]
    feats = np.zeros(n * F, np.uint16)
    outs = np.zeros(n * no, np.uint16)
    lat = st.params().latents
    assert O.ntref_forward(C.byref(lat), C.byref(st.net.struct()), filt, uvz.ctypes.data, n,
                           feats.ctypes.data, outs.ctypes.data) == 0
    gs = st.to_torch()
    gl = gs.params().latents
    guvz = torch.from_numpy(uvz).cuda()
    gf = torch.zeros(n * F, dtype=torch.int16, device="cuda")
    go = torch.zeros(n * no, dtype=torch.int16, device="cuda")
    nt.check(lib.nt_forward(C.byref(gl), C.byref(gs.net.struct()), filt, guvz.data_ptr(), n,
                            gf.data_ptr(), go.data_ptr(), None))
    sync()
    assert np.array_equal(gf.cpu().numpy().view(np.uint16), feats)
    got = go.cpu().numpy().view(np.float16).astype(np.float32)
    assert_close(got, outs.view(np.float16).astype(np.float32), "outputs")


# ---- the fused train step -----------------------------------------------------------------

TRAIN_CASES = [
    # shape, image, region (w, h), offset, kernel type
    ("ref", 128, (64, 32), (0, 0), abi.NT_UNCONSTRAINED),
    ("ref", 128, (64, 32), (100, 110), abi.NT_UNCONSTRAINED),  # region wraps past the edge
    ("ref16", 128, (64, 32), (0, 0), abi.NT_UNCONSTRAINED),
    ("ref16", 128, (64, 48), (100, 110), abi.NT_UNCONSTRAINED),
    ("ref16", 64, (50, 21), (3, 5), abi.NT_UNCONSTRAINED),       # ragged region and tail row
    ("ref16f", 128, (64, 32), (7, 13), abi.NT_UNCONSTRAINED),
    ("ref16f", 100, (64, 32), (30, 50), abi.NT_UNCONSTRAINED),
    ("ref16f", 64, (50, 21), (3, 5), abi.NT_UNCONSTRAINED),      # ragged: records of positions past the region
    ("ref16u", 64, (64, 32), (9, 17), abi.NT_UNCONSTRAINED),
    ("ref16ff", 128, (64, 32), (11, 3), abi.NT_UNCONSTRAINED),
    ("ref16ff", 128, (64, 48), (100, 110), abi.NT_UNCONSTRAINED),
    ("ref16h", 128, (64, 32), (40, 9), abi.NT_UNCONSTRAINED),
    ("ref16h", 128, (64, 48), (100, 110), abi.NT_UNCONSTRAINED),
    # BASELINE config 1's network (8 -> 64 -> 64 -> 3, one 8-channel grid) on the general kernel
    ("c1", 128, (64, 32), (16, 40), abi.NT_UNCONSTRAINED),
    ("c1", 64, (50, 21), (3, 5), abi.NT_UNCONSTRAINED),          # ragged region and tail row
    ("c1f", 128, (64, 48), (100, 90), abi.NT_UNCONSTRAINED),     # wraps; a grid as fine as the image
    ("c1", 128, (64, 32), (0, 0), abi.NT_BLOCK_FEATURES),
    ("c2", 128, (64, 32), (16, 40), abi.NT_UNCONSTRAINED),
    ("c2", 64, (50, 21), (3, 5), abi.NT_UNCONSTRAINED),         # ragged region and tail row
    ("c2", 128, (64, 48), (100, 90), abi.NT_UNCONSTRAINED),     # wraps: clamped edge samples
    ("c4", 128, (64, 32), (96, 120), abi.NT_UNCONSTRAINED),
    ("c4", 128, (64, 32), (8, 8), abi.NT_UNCONSTRAINED),
    # image sizes that are not powers of two: positions divide instead of scaling by an exact
    # reciprocal, and footprints come from inexact products
    ("c2", 100, (64, 32), (7, 13), abi.NT_UNCONSTRAINED),
    ("c4", 96, (64, 32), (30, 50), abi.NT_UNCONSTRAINED),
    ("ref", 64, (32, 16), (0, 0), abi.NT_BLOCK_FEATURES),
    ("ref", 64, (32, 16), (5, 7), abi.NT_FINALIZE),
    # the reference network's block phase with float4 textures: block records expanded to
    # texels, the fused kernel, block gradients folded from texel gradients
    ("ref16", 128, (64, 32), (0, 0), abi.NT_BLOCK_FEATURES),
    ("ref16f", 128, (64, 48), (100, 110), abi.NT_BLOCK_FEATURES),  # region wraps past the edge
    ("ref16f", 64, (50, 21), (3, 5), abi.NT_BLOCK_FEATURES),       # ragged region and tail row
    ("ref16ff", 128, (64, 32), (11, 3), abi.NT_BLOCK_FEATURES),
    ("ref16h", 128, (128, 64), (0, 64), abi.NT_BLOCK_FEATURES),    # rectangles as wide as a grid
    ("ref16f", 128, (64, 32), (7, 13), abi.NT_FINALIZE),
    ("c2", 64, (32, 16), (3, 9), abi.NT_BLOCK_FEATURES),
    ("c4", 128, (32, 16), (0, 0), abi.NT_FINALIZE),
]


def run_train_pair(lib, O, shape, image, region, offset, ktype, seed=0, step=0, sample_mode=abi.NT_SAMPLES_REGION):
    """One train step on the GPU and on the oracle from the same state. Returns the oracle's
    state, the GPU's, and the oracle's with fp32 MLP sums (each element's sensitivity to
    the accumulation order, assert_close's `alt`)."""
    def state():
        x = make_state(shape, image=image, region=region, offset=offset, seed=seed, step=step,
                       blocks=ktype != abi.NT_UNCONSTRAINED)
        if region == (50, 21):
            x.num_samples = 50 * 21 - 17  # partial last row
        x.sample_mode = sample_mode
        return x
    st, st32 = state(), state()
    gs = gpu_workspace(lib, st.to_torch(), ktype)
    oracle_step(O, st, ktype)
    oracle_step(O, st32, ktype, accum_f32=True)
    nt.check(lib.nt_train_step(C.byref(gs.params()), ktype, None))
    sync()
    return st, gs, st32


def check_train_grads(st, gs, alt, ktype=abi.NT_UNCONSTRAINED, biases=True, untouched_zero=True):
    """MLP and latent gradients of the GPU (gs) against the oracle (st) at the MLP bar
    (assert_close, with the fp32-sum oracle `alt` as each element's spread)."""
    for l in range(st.net.num_layers):
        assert_close(gs.net.weight_grads[l], st.net.weight_grads[l], f"dW{l}", alt.net.weight_grads[l])
        if biases:
            assert_close(gs.net.bias_grads[l], st.net.bias_grads[l], f"db{l}", alt.net.bias_grads[l])
    for gi, (g, gg, ga) in enumerate(zip(st.grids, gs.grids, alt.grids)):
        if ktype == abi.NT_UNCONSTRAINED:
            got = to_np(gg.grads)
            assert np.count_nonzero(g.grads) > 0
            assert_close(got.reshape(-1, g.channels), g.grads, f"latent grad {gi} [texel, channel]", ga.grads)
            if untouched_zero:
                # texels the oracle leaves untouched stay exactly zero
                assert np.all(got[g.grads == 0] == 0)
        elif ktype == abi.NT_BLOCK_FEATURES:
            assert_close(to_np(gg.block_grads).reshape(-1, 4 * g.channels + 16), g.block_grads,
                         f"block grad {gi} [block, field]", ga.block_grads)
        else:
            assert np.all(to_np(gg.block_grads) == 0)


@pytest.mark.parametrize("case", TRAIN_CASES, ids=lambda c: f"{c[0]}-{c[1]}-{c[2][0]}x{c[2][1]}-{c[4]}")
def test_train_step_gradients(lib, O, case):
    shape, image, region, offset, ktype = case
    say(f"case: train {case}")
    st, gs, alt = run_train_pair(lib, O, shape, image, region, offset, ktype)
    check_train_grads(st, gs, alt, ktype)


@pytest.mark.parametrize("shape", ["ref", "ref16", "ref16f", "ref16ff", "ref16h", "c2", "c4"])
def test_train_step_several_tiles_per_workgroup(lib, O, shape):
    """Fewer workgroups than tiles: each workgroup runs several tiles, flushing its latent
    box per tile and writing one MLP-gradient partial (the path large regions take)."""
    say(f"case: train {shape} 3 workgroups for 4 tiles")
    nt.check(lib.nt_set_test_hooks(3, 0))
    try:
        st, gs, alt = run_train_pair(lib, O, shape, 128, (128, 16 if shape == "c4" else 32), (5, 9),
                                     abi.NT_UNCONSTRAINED)
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))
    check_train_grads(st, gs, alt)


@pytest.mark.parametrize("shape", ["ref", "ref16", "c2", "c4"])
def test_train_step_scatter_out_of_box_paths(lib, O, shape):
    """Without the margin of the chunk cell box, many footprints fall outside it: the
    scatter adds those per sample with atomics (the 16-channel kernel to global memory, the
    general kernel of the 3-channel network into its LDS footprint box), and the one-group
    kernel's gather reads those waves' corners from global memory instead of its LDS copy
    of the cell boxes. Gradients still match the oracle's."""
    say(f"case: train {shape} without box margins")
    nt.check(lib.nt_set_test_hooks(0, abi.NT_HOOK_DROP_MARGINS))
    try:
        st, gs, alt = run_train_pair(lib, O, shape, 128, (64, 32), (11, 21), abi.NT_UNCONSTRAINED)
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))
    check_train_grads(st, gs, alt, biases=False)


@pytest.mark.parametrize("shape,region,max_wg,flags,image", [
    ("ref", (64, 32), 0, 0, 128), ("c1", (64, 32), 0, 0, 128), ("c2", (64, 32), 0, 0, 128),
    ("c4", (64, 32), 0, 0, 128), ("c2", (50, 13), 2, 0, 128), ("c4", (100, 7), 1, 0, 128),
    ("c2", (100, 30), 2, 0, 128),
    # the 16-channel kernel's slots in bin order (a step sorts from 262,144 samples)
    ("c2", (64, 32), 0, abi.NT_HOOK_SORT_RANDOM, 128), ("c4", (100, 7), 1, abi.NT_HOOK_SORT_RANDOM, 128),
    ("c2", (100, 30), 2, abi.NT_HOOK_SORT_RANDOM, 128),
    # images that are no multiple of the 64-texel bins: partial bins on the right and bottom
    ("c2", (64, 32), 0, 0, 168), ("c2", (64, 32), 0, abi.NT_HOOK_SORT_RANDOM, 168),
    ("c4", (100, 7), 1, abi.NT_HOOK_SORT_RANDOM, 200),
    # several tiles of the one-pass sort; keys of 11 bits (33 x 33 bins): the two-pass sort
    ("c2", (128, 100), 0, abi.NT_HOOK_SORT_RANDOM, 128), ("c2", (100, 100), 0, abi.NT_HOOK_SORT_RANDOM, 2112),
], ids=["ref", "c1", "c2", "c4", "c2-ragged-2wg", "c4-ragged-1wg", "c2-3tiles-2wg", "c2-sorted",
        "c4-ragged-1wg-sorted", "c2-3tiles-2wg-sorted", "c2-image168", "c2-image168-sorted",
        "c4-image200-1wg-sorted", "c2-4tiles-sorted", "c2-image2112-two-pass-sorted"])
def test_train_step_random_texels(lib, O, shape, region, max_wg, flags, image):
    """NT_SAMPLES_RANDOM: samples anywhere in the image (the 16-channel kernel with taps
    from global memory and per-sample corner atomics; the general kernel for the reference
    network); gradients match the oracle's at the MLP tolerance. Ragged regions leave
    partial tiles; one or two workgroups walk every tile (config 2 runs two groups of 512
    samples per tile: 3,000 samples are three tiles, two of them on one workgroup). With the
    samples sorted by bin the kernel's slots hold other samples, placed as before: the same
    gradients."""
    say(f"case: train {shape} random texels image {image} region {region} max workgroups {max_wg} flags {flags}")
    nt.check(lib.nt_set_test_hooks(max_wg, flags))
    try:
        st, gs, alt = run_train_pair(lib, O, shape, image, region, (0, 0), abi.NT_UNCONSTRAINED, seed=17,
                                     sample_mode=abi.NT_SAMPLES_RANDOM)
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))
    check_train_grads(st, gs, alt)


def test_random_texel_sorted_step_is_deterministic(lib):
    """The bin sort of NT_SAMPLES_RANDOM is stable, so a step's slots hold the same samples
    on every run and the network gradient (summed per workgroup in slot order, then in a
    fixed order) is bit-identical across runs; the latent gradients (float atomics) match
    to rounding."""
    import torch
    say("case: random texels sorted, two runs")
    st = make_state("c2", image=256, region=(128, 64), seed=23)
    st.sample_mode = abi.NT_SAMPLES_RANDOM
    nt.check(lib.nt_set_test_hooks(0, abi.NT_HOOK_SORT_RANDOM))
    try:
        runs = []
        for _ in range(2):
            g = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
            nt.check(lib.nt_train_step(C.byref(g.params()), abi.NT_UNCONSTRAINED, None))
            sync()
            runs.append(g)
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))
    a, b = runs
    for x, y in zip((*a.net.weight_grads, *a.net.bias_grads), (*b.net.weight_grads, *b.net.bias_grads)):
        assert torch.equal(x.view(torch.int32), y.view(torch.int32))
    assert torch.count_nonzero(a.net.weight_grads[0]) > 0
    for ga, gb in zip(a.grids, b.grids):
        assert_close(to_np(gb.grads), to_np(ga.grads), "latent grads of two runs", tol=1e-5, floor=1e-6)


@pytest.mark.parametrize("image,region", [(128, (128, 100)), (2112, (100, 100)), (168, (64, 32)),
                                          (2048, (512, 512)), (4096, (1024, 1024))],
                         ids=["one-pass-4tiles", "two-pass", "partial-bins", "config2-full-size",
                              "config4-size-two-pass"])
def test_random_sample_order_is_the_stable_bin_sort(lib, O, image, region):
    """The order a sorted NT_SAMPLES_RANDOM step reads its samples in, exactly (integer
    work): the sample indices sorted stably by the 64 x 64-texel bin, row-major, of each
    sample's texel, the texel from the oracle's seed and hash (the placement the oracle's
    own position test pins against ntref_sample_uvz)."""
    import torch
    say(f"case: random sample order image {image} region {region}")
    st = make_state("c2", image=image, region=region, seed=29, step=7)
    st.sample_mode = abi.NT_SAMPLES_RANDOM
    nt.check(lib.nt_set_test_hooks(0, abi.NT_HOOK_SORT_RANDOM))
    try:
        g = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
        n = st.num_samples
        order = torch.full((n,), -1, dtype=torch.int32, device="cuda")
        nt.check(lib.nt_random_sample_order(C.byref(g.params()), C.c_void_p(order.data_ptr()), None))
        sync()
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))
    W = H = image
    # config 2's full size: 262,144 samples, 1,024 bins, 64 tiles, one pass; config 4's
    # sample count and image: 1,048,576 samples, 4,096 bins, 256 tiles, two passes
    key = np.empty(n, np.int64)
    for i in range(n):
        h1 = O.ntref_fmix32(O.ntref_sample_seed(i, 7))
        h2 = O.ntref_fmix32(h1)
        u0 = np.float32(h1 & 0xFFFFFF) * np.float32(2.0 ** -24)
        u1 = np.float32(h2 & 0xFFFFFF) * np.float32(2.0 ** -24)
        x, y = min(int(np.float32(u0) * np.float32(W)), W - 1), min(int(np.float32(u1) * np.float32(H)), H - 1)
        key[i] = (y >> 6) * ((W + 63) // 64) + (x >> 6)
    expected = np.argsort(key, kind="stable")
    got = order.cpu().numpy().astype(np.int64)
    assert np.array_equal(got, expected)
    assert len(np.unique(key)) > 1


def test_train_step_accumulates(lib, O):
    """Two passes without an optimizer step add up (the zero-gradient contract)."""
    say("case: train accumulate")
    st = make_state("c2", image=64, region=(32, 16), seed=4)
    gs = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    for _ in range(2):
        assert O.ntref_train_step(C.byref(st.params()), 0, 1) == 0
        nt.check(lib.nt_train_step(C.byref(gs.params()), 0, None))
    sync()
    assert_close(gs.net.weight_grads[1], st.net.weight_grads[1], "dW1")
    assert_close(to_np(gs.grids[0].grads).reshape(-1, 16), st.grids[0].grads, "latent grad 0 [texel, channel]")


# ---- Adam ------------------------------------------------------------------------------------

def test_optimize_network_and_latents_bit_exact(lib, O):
    say("case: adam network + latents")
    rng = np.random.default_rng(40)
    st = make_state("c2", image=64, region=(32, 16), seed=5, step=3)
    for l in range(st.net.num_layers):
        g = st.net.weight_grads[l]
        g[:] = np.where(rng.uniform(size=g.size) < 0.7, rng.normal(0, 1e-3, g.size), 0)
        st.net.weight_moment1[l][:] = rng.normal(0, 1e-4, g.size)
        st.net.weight_moment2[l][:] = rng.uniform(0, 1e-6, g.size)
        st.net.bias_grads[l][:] = rng.normal(0, 1e-3, st.net.bias_grads[l].size)
    for g in st.grids:
        g.grads[:] = np.where(rng.uniform(size=g.grads.size) < 0.3, rng.normal(0, 1e-2, g.grads.size), 0)
        g.moment1[:] = rng.normal(0, 1e-3, g.grads.size)
        g.moment2[:] = rng.uniform(0, 1e-4, g.grads.size)
    gs = st.to_torch()
    assert O.ntref_optimize_network(C.byref(st.params())) == 0
    assert O.ntref_optimize_latents(C.byref(st.params()), 0) == 0
    nt.check(lib.nt_optimize_network(C.byref(gs.params()), None))
    nt.check(lib.nt_optimize_latents(C.byref(gs.params()), 0, None))
    sync()
    for l in range(st.net.num_layers):
        for name in ("weights", "weight_grads", "weight_moment1", "weight_moment2", "biases",
                     "bias_grads", "bias_moment1", "bias_moment2"):
            a, b = to_np(getattr(gs.net, name)[l]), getattr(st.net, name)[l]
            assert np.array_equal(a.view(np.uint16) if a.dtype == np.int16 else a, b), (name, l)
    for g, gg in zip(st.grids, gs.grids):
        for name in ("values", "grads", "moment1", "moment2"):
            assert np.array_equal(to_np(getattr(gg, name)), getattr(g, name)), name


def test_optimize_block_latents(lib, O):
    say("case: adam blocks")
    rng = np.random.default_rng(41)
    st = make_state("ref", image=64, region=(32, 16), seed=6, step=2, blocks=True)
    for g in st.grids:
        g.block_grads[:] = np.where(rng.uniform(size=g.block_grads.size) < 0.5,
                                    rng.normal(0, 1e-2, g.block_grads.size), 0)
    gs = st.to_torch()
    assert O.ntref_optimize_latents(C.byref(st.params()), abi.NT_BLOCK_FEATURES) == 0
    nt.check(lib.nt_optimize_latents(C.byref(gs.params()), abi.NT_BLOCK_FEATURES, None))
    sync()
    for g, gg in zip(st.grids, gs.grids):
        assert np.array_equal(to_np(gg.block_params), g.block_params)
        assert np.array_equal(to_np(gg.block_grads), g.block_grads)


@pytest.mark.parametrize("C_,sizes", [(3, [(32, 6), (16, 5)]), (16, [(64, 7), (16, 3)]),
                                      (8, [(8, 4)]), (4, [(4, 3), (12, 2)])])
def test_bc6_init_bit_exact(lib, O, C_, sizes):
    """nt_bc6_init == the oracle's block records, bit for bit, on every mip down to 1x1."""
    import torch
    say(f"case: bc6 init C={C_} grids={sizes}")
    rng = np.random.default_rng(60 + C_)
    grids = []
    for size, mips in sizes:
        g = P.make_grid(size, size, mips, C_, rng, blocks=True)
        # Unconstrained latents as training leaves them: mostly positive, a few small
        # negative texels and a run of equal texels.
        g.values[:] = np.abs(rng.normal(0.3, 0.4, g.values.size)).astype(np.float32)
        g.values[: 4 * C_] *= -1e-3
        g.values[16 * C_: 32 * C_] = 0.125
        g.block_params[:] = 0
        grids.append(g)
    lat = abi.nt_latents()
    lat.num_grids, lat.channels = len(grids), C_
    for i, g in enumerate(grids):
        lat.grids[i] = g.struct()
    assert O.ntref_bc6_init(C.byref(lat)) == 0
    ggrids = [g.converted(True, "cuda") for g in grids]
    for gg in ggrids:
        gg.block_params.fill_(float("nan"))  # every record must be written
    glat = abi.nt_latents()
    glat.num_grids, glat.channels = len(ggrids), C_
    for i, g in enumerate(ggrids):
        glat.grids[i] = g.struct()
    nt.check(lib.nt_bc6_init(C.byref(glat), None))
    sync()
    for g, gg in zip(grids, ggrids):
        got = to_np(gg.block_params)
        assert np.array_equal(got.view(np.uint32), g.block_params.view(np.uint32))


# ---- inference (train.cu:917-961) --------------------------------------------------------------

@pytest.mark.parametrize("shape", ["ref", "c2"])
def test_inference(lib, O, shape):
    import torch
    say(f"case: inference {shape}")
    st = make_state(shape, image=48, region=(16, 16), seed=7)
    no = st.net.sizes[-1]
    st.inference_output = np.zeros(48 * 48 * no, np.float32)
    st.inference_mse_accum = np.zeros(1, np.float32)
    gs = st.to_torch()
    assert O.ntref_inference(C.byref(st.params())) == 0
    nt.check(lib.nt_inference(C.byref(gs.params()), None))
    sync()
    assert_close(gs.inference_output, st.inference_output, "inference output")
    assert abs(float(to_np(gs.inference_mse_accum)[0]) - float(st.inference_mse_accum[0])) <= \
        1e-2 * abs(float(st.inference_mse_accum[0]))


def test_inference_sse_fixed_order(lib, O):
    """With a workspace the SSE is summed in a fixed order: the same bits on every run, and
    within rounding of the atomic path and of the oracle's float64 sum."""
    import torch
    say("case: inference c2 256^2 fixed-order SSE")
    image = 256
    st = make_state("c2", image=image, region=(16, 16), seed=9)
    no = st.net.sizes[-1]
    st.inference_output = np.zeros(image * image * no, np.float32)
    st.inference_mse_accum = np.zeros(1, np.float32)
    assert O.ntref_inference(C.byref(st.params())) == 0
    gs = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    need = lib.nt_inference_workspace_bytes(C.byref(gs.params()))
    assert need == (image * image // 32 // 4) * 4 * 4
    assert gs.workspace.numel() >= need

    def run(s):
        s.inference_mse_accum.zero_()
        nt.check(lib.nt_inference(C.byref(s.params()), None))
        sync()
        return to_np(s.inference_mse_accum).copy()

    fixed = [run(gs) for _ in range(3)]
    assert all(np.array_equal(f.view(np.uint32), fixed[0].view(np.uint32)) for f in fixed)
    want = float(st.inference_mse_accum[0])
    assert abs(float(fixed[0][0]) - want) <= 1e-2 * want
    ws = gs.workspace
    gs.workspace = None
    atomic = run(gs)
    gs.workspace = ws
    assert abs(float(atomic[0]) - float(fixed[0][0])) <= 1e-5 * float(fixed[0][0])


# ---- codec ----------------------------------------------------------------------------------------

@pytest.mark.parametrize("w,h,c", [(64, 64, 16), (37, 22, 16), (16, 8, 8), (9, 13, 4), (20, 12, 12)])
def test_codec_bit_exact(lib, O, w, h, c):
    import torch
    say(f"case: codec {w}x{h}x{c}")
    rng = np.random.default_rng(w * h + c)
    vals = rng.normal(0, 0.5, size=w * h * c).astype(np.float32)
    vals[:10] = [0.0, -0.0, 1e-8, -1e-8, 7e4, -7e4, 65504.0, np.nan, np.inf, -np.inf]
    nb = ((w + 3) // 4) * ((h + 3) // 4) * 12 * c
    want = np.zeros(nb, np.uint8)
    assert O.ntref_codec_encode(vals.ctypes.data, w, h, c, want.ctypes.data) == 0
    gv = torch.from_numpy(vals).cuda()
    gb = torch.zeros(nb, dtype=torch.uint8, device="cuda")
    nt.check(lib.nt_codec_encode(gv.data_ptr(), w, h, c, gb.data_ptr(), None))
    sync()
    assert np.array_equal(gb.cpu().numpy(), want)
    dec = np.zeros(w * h * c, np.float32)
    assert O.ntref_codec_decode(want.ctypes.data, w, h, c, dec.ctypes.data) == 0
    gd = torch.zeros(w * h * c, dtype=torch.float32, device="cuda")
    nt.check(lib.nt_codec_decode(gb.data_ptr(), w, h, c, gd.data_ptr(), None))
    sync()
    assert np.array_equal(gd.cpu().numpy().view(np.uint32), dec.view(np.uint32))


# ---- decode from quantized latents ------------------------------------------------------------------

@pytest.mark.parametrize("shape,W,H,jitter,mip_min,mip_max", [
    ("c4", 96, 96, 1.0, 0.0, 3.0),
    ("c4", 100, 37, -1.5, 0.5, 6.0),   # ragged blocks, negative jitter, mips past the last one
    ("c4", 70, 20, 3.0, -1.0, 1.0),    # negative mip coordinates clamp to mip 0
    ("c2", 100, 37, 1.0, 0.0, 3.0),    # the 2-grid network (32->64->64->9)
    ("c2", 128, 64, 1.0, 0.0, 3.0),    # power-of-two sizes: positions scaled by exact reciprocals
    ("c4", 256, 128, 0.5, 0.0, 2.0),
], ids=["96x96", "100x37", "70x20", "c2-100x37", "c2-128x64", "256x128"])
def test_decode_from_codec_latents(lib, O, shape, W, H, jitter, mip_min, mip_max):
    import torch
    say(f"case: decode {shape} {W}x{H} jitter {jitter} z [{mip_min}, {mip_max})")
    rng = np.random.default_rng(50)
    C16 = 16
    sizes = [(64, 5), (32, 5), (16, 4), (8, 3)] if shape == "c4" else [(64, 5), (32, 5)]
    net_sizes = [64, 64, 64, 64, 12] if shape == "c4" else [32, 64, 64, 9]
    nout = net_sizes[-1]
    blobs, grids_np = [], []
    for size, mips in sizes:
        offs, total = P.codec_chain_layout(size, size, mips, C16)
        blob = np.zeros(total, np.uint8)
        for m in range(mips):
            s = P.mip_dim(size, m)
            vals = rng.normal(0, 0.5, size=s * s * C16).astype(np.float32)
            blk = np.zeros(((s + 3) // 4) ** 2 * 12 * C16, np.uint8)
            assert O.ntref_codec_encode(vals.ctypes.data, s, s, C16, blk.ctypes.data) == 0
            blob[offs[m]:offs[m] + blk.size] = blk
        blobs.append((size, mips, offs, blob))
    net = P.make_network(net_sizes, rng=rng, init="xavier")

    def dparams(blob_ptrs, netv, out_ptr):
        d = abi.nt_decode_params()
        d.num_grids, d.channels = len(sizes), C16
        for i, (size, mips, offs, _) in enumerate(blobs):
            d.grids[i].width = d.grids[i].height = size
            d.grids[i].num_mips = mips
            for m, o in enumerate(offs):
                d.grids[i].byte_offset[m] = o
            d.grids[i].blocks = blob_ptrs[i]
        d.mlp = netv.struct()
        d.out_width, d.out_height = W, H
        d.seed, d.jitter, d.mip_min, d.mip_max = 1234, jitter, mip_min, mip_max
        d.output = C.cast(out_ptr, abi.u16p)
        return d

    want = np.zeros(W * H * nout, np.uint16)
    dp = dparams([b[3].ctypes.data for b in blobs], net, want.ctypes.data)
    assert O.ntref_decode(C.byref(dp), 1) == 0
    gblobs = [torch.from_numpy(b[3]).cuda() for b in blobs]
    gnet = net.converted(True, "cuda")
    gout = torch.zeros(W * H * nout, dtype=torch.int16, device="cuda")
    gp = dparams([g.data_ptr() for g in gblobs], gnet, gout.data_ptr())
    nt.check(lib.nt_decode(C.byref(gp), None))
    sync()
    got = gout.cpu().numpy().view(np.float16).astype(np.float32)
    assert_close(got, want.view(np.float16).astype(np.float32), "decoded pixels")
    # The two-pass decode (blocks expanded to fp16 texels first, then sampled from per-block
    # LDS boxes) gives the same bits.
    say(f"case: decode {shape} two-pass")
    nbytes = lib.nt_decode_workspace_bytes(C.byref(gp))
    assert nbytes > 0
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    gout2 = torch.zeros_like(gout)
    gp2 = dparams([g.data_ptr() for g in gblobs], gnet, gout2.data_ptr())
    gp2.workspace, gp2.workspace_bytes = ws.data_ptr(), nbytes
    nt.check(lib.nt_decode(C.byref(gp2), None))
    sync()
    assert torch.equal(gout2, gout)
    gp2.workspace_bytes = nbytes - 16
    assert lib.nt_decode(C.byref(gp2), None) == abi.NT_ERR_WORKSPACE


# ---- lazy latent Adam over touched runs --------------------------------------------------------------

@pytest.mark.parametrize("shape,mode,margins", [("c2", abi.NT_SAMPLES_REGION, 0), ("c4", abi.NT_SAMPLES_REGION, 0),
                                                ("c2", abi.NT_SAMPLES_REGION, 1), ("c2", abi.NT_SAMPLES_RANDOM, 0),
                                                ("ref", abi.NT_SAMPLES_REGION, 0), ("ref16", abi.NT_SAMPLES_REGION, 0),
                                                ("ref16f", abi.NT_SAMPLES_REGION, 0)],
                         ids=["c2", "c4", "c2-out-of-box", "c2-random", "ref", "ref16", "ref16f"])
def test_latent_touched_update_equals_dense(lib, shape, mode, margins):
    """NT_LATENT_TOUCHED: after one logged train step the optimizer updates only the logged
    footprint rectangles (every texel after other kernels). Fed the same gradients, it must
    leave latents, moments and gradients bit-identical to the dense scan (train.cu:764-803):
    over several steps with moving regions, starting from a workspace of random bytes, and
    with two train steps accumulated before one optimizer call."""
    import torch
    say(f"case: touched latent Adam {shape} mode {mode} margins-dropped {margins}")
    st = make_state(shape, image=256, region=(64, 32), seed=8, offset=(0, 0), step=1)
    st.sample_mode = mode
    st.latent_update = abi.NT_LATENT_TOUCHED
    a = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    a.latent_update = abi.NT_LATENT_TOUCHED
    a.workspace.random_(0, 256)  # a fresh workspace: no valid log
    b = st.to_torch()
    b.latent_update = abi.NT_LATENT_DENSE
    offs = np.random.default_rng(3).integers(0, 256 - 64, size=(4, 2))
    nt.check(lib.nt_set_test_hooks(0, margins))
    try:
        for i in range(4):
            for s in (a, b):
                s.texel_offset_x, s.texel_offset_y = int(offs[i, 0]), int(offs[i, 1])
                s.step = 1 + i
            nt.check(lib.nt_train_step(C.byref(a.params()), abi.NT_UNCONSTRAINED, None))
            if i == 2:  # two steps accumulate before this optimizer call
                a.texel_offset_x, a.texel_offset_y = int(offs[i, 1]), int(offs[i, 0])
                nt.check(lib.nt_train_step(C.byref(a.params()), abi.NT_UNCONSTRAINED, None))
            sync()
            for ga, gb in zip(a.grids, b.grids):
                gb.grads.copy_(ga.grads)
            nt.check(lib.nt_optimize_latents(C.byref(a.params()), abi.NT_UNCONSTRAINED, None))
            nt.check(lib.nt_optimize_latents(C.byref(b.params()), abi.NT_UNCONSTRAINED, None))
            sync()
            for gi, (ga, gb) in enumerate(zip(a.grids, b.grids)):
                for name in ("values", "moment1", "moment2", "grads"):
                    x, y = getattr(ga, name), getattr(gb, name)
                    assert torch.equal(x.view(torch.int32), y.view(torch.int32)), f"step {i} grid {gi} {name}"
                assert torch.count_nonzero(ga.moment1) > 0
            for s in (a, b):  # the network gradients are not under test: clear them
                for arr in (*s.net.weight_grads, *s.net.bias_grads):
                    arr.zero_()
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))


@pytest.mark.parametrize("shape", ["ref16", "ref16f"])
def test_block_touched_update_equals_dense(lib, shape):
    """NT_LATENT_TOUCHED with BC6 block records: the BC6 phase's fold logs the mip-0 block
    rectangle of each grid, and nt_optimize_latents then visits only those records. Fed the
    same block gradients, it must leave every record, moment and gradient bit-identical to
    the dense scan of every record of every mip (train.cu:641-679, 805-816): over several
    steps with moving regions (one wrapping past the image edge), from a workspace of random
    bytes, and with two train steps accumulated before one optimizer call."""
    import torch
    say(f"case: touched block Adam {shape}")
    st = make_state(shape, image=128, region=(64, 32), seed=8, offset=(0, 0), step=1, blocks=True)
    st.latent_update = abi.NT_LATENT_TOUCHED
    a = gpu_workspace(lib, st.to_torch(), abi.NT_BLOCK_FEATURES)
    a.latent_update = abi.NT_LATENT_TOUCHED
    a.workspace.random_(0, 256)  # a fresh workspace: no valid log
    b = st.to_torch()
    b.latent_update = abi.NT_LATENT_DENSE
    offs = [(3, 5), (100, 110), (40, 17), (64, 96)]
    for i in range(4):
        for s in (a, b):
            s.texel_offset_x, s.texel_offset_y = offs[i]
            s.step = 1 + i
        nt.check(lib.nt_train_step(C.byref(a.params()), abi.NT_BLOCK_FEATURES, None))
        if i == 2:  # two steps accumulate before this optimizer call
            a.texel_offset_x, a.texel_offset_y = offs[i][1], offs[i][0]
            nt.check(lib.nt_train_step(C.byref(a.params()), abi.NT_BLOCK_FEATURES, None))
        sync()
        for ga, gb in zip(a.grids, b.grids):
            gb.block_grads.copy_(ga.block_grads)
        assert any(torch.count_nonzero(g.block_grads) > 0 for g in a.grids)
        nt.check(lib.nt_optimize_latents(C.byref(a.params()), abi.NT_BLOCK_FEATURES, None))
        nt.check(lib.nt_optimize_latents(C.byref(b.params()), abi.NT_BLOCK_FEATURES, None))
        sync()
        for gi, (ga, gb) in enumerate(zip(a.grids, b.grids)):
            for name in ("block_params", "block_moment1", "block_moment2", "block_grads"):
                x, y = getattr(ga, name), getattr(gb, name)
                assert torch.equal(x.view(torch.int32), y.view(torch.int32)), f"step {i} grid {gi} {name}"
            assert torch.count_nonzero(ga.block_moment1) > 0
        for s in (a, b):  # the network gradients are not under test: clear them
            for arr in (*s.net.weight_grads, *s.net.bias_grads):
                arr.zero_()


# ---- the reference-target pipeline: packing, loss weights, target mips ------------------------------

def _texture_chain(image, nch, rng, mips, weight=1.0):
    """A reference texture with `mips` levels, each the 2 x 2 box average of the one above
    (a software mip chain in the layout of nt_texture; main.cpp:360-434 reads such chains
    from tiled EXRs), pitch 1 for one channel, else 4."""
    pitch = 1 if nch == 1 else 4
    levels = [rng.uniform(0, 1, size=(image, image, pitch)).astype(np.float32)]
    for _ in range(1, mips):
        a = levels[-1]
        h, w = max(a.shape[0] // 2, 1), max(a.shape[1] // 2, 1)
        levels.append(a[:2 * h, :2 * w].reshape(h, 2, w, 2, pitch).mean(axis=(1, 3)).astype(np.float32))
    if pitch == 4 and nch < 4:
        for lv in levels:
            lv[:, :, nch:] = 0
    return P.Texture(image, image, nch, np.concatenate([lv.reshape(-1) for lv in levels]), mips, pitch, weight)


TARGET_CASES = [
    # (shape, per-texture channels, loss weights): the 16-channel kernel takes up to four
    # float4 textures; five or more, or one-channel textures (pitch 1), take the general one
    ("c2", [2, 4, 3], [4.0, 1.0, 0.5]),
    ("c4", [4, 4, 4], [1.0, 4.0, 1.0]),
    ("c2", [1, 2, 1, 3, 2], [1.0, 4.0, 1.0, 0.5, 2.0]),
    ("c4", [1] * 12, [0.25 * (k + 1) for k in range(12)]),
    ("ref", [3, 2, 4, 1, 3, 2, 1], [4.0, 1.0, 1.0, 2.0, 0.5, 1.0, 3.0]),
    ("ref", [1] * 16, [1.0 + (k % 3) for k in range(16)]),
]


@pytest.mark.parametrize("case", TARGET_CASES, ids=lambda c: f"{c[0]}-{len(c[1])}tex-{sum(min(n, 4) for n in c[1])}ch")
def test_train_step_target_packing_and_loss_weights(lib, O, case):
    """train.cu:105-157: a 1-channel texture feeds one output, others min(channels, 4), up to
    16 outputs, each output weighted by its texture's loss weight (train.cu:138-153)."""
    shape, chans, weights = case
    say(f"case: targets {case}")
    st = make_state(shape, image=128, region=(64, 32), offset=(7, 19), seed=12)
    rng = np.random.default_rng(13)
    st.textures = [_texture_chain(128, n, rng, 1, w) for n, w in zip(chans, weights)]
    nout = min(16, sum(1 if n == 1 else min(n, 4) for n in chans))
    assert nout <= abi.pad16(st.net.sizes[-1])
    gs = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    assert O.ntref_train_step(C.byref(st.params()), abi.NT_UNCONSTRAINED, 1) == 0
    nt.check(lib.nt_train_step(C.byref(gs.params()), abi.NT_UNCONSTRAINED, None))
    sync()
    for l in range(st.net.num_layers):
        assert_close(gs.net.weight_grads[l], st.net.weight_grads[l], f"dW{l}")
        assert_close(gs.net.bias_grads[l], st.net.bias_grads[l], f"db{l}")
    for gi, (g, gg) in enumerate(zip(st.grids, gs.grids)):
        assert_close(to_np(gg.grads).reshape(-1, g.channels), g.grads, f"latent grad {gi} [texel, channel]")
    # the loss weights matter: the oracle's gradient with unit weights differs
    st1 = make_state(shape, image=128, region=(64, 32), offset=(7, 19), seed=12)
    rng = np.random.default_rng(13)
    st1.textures = [_texture_chain(128, n, rng, 1, 1.0) for n in chans]
    assert O.ntref_train_step(C.byref(st1.params()), abi.NT_UNCONSTRAINED, 1) == 0
    assert rel_err(st1.net.weight_grads[-1], st.net.weight_grads[-1]) > 0.05


@pytest.mark.parametrize("shape", ["ref", "c2", "c4"])
@pytest.mark.parametrize("z", [0.5, 1.0, 2.25, 9.0])
def test_train_step_at_mip_coordinate(lib, O, shape, z):
    """nt_params.sample_mip = z > 0: latents sampled trilinearly across mips floor(z) and
    floor(z) + 1 (train.cu:263-314), gradients scattered into both (train.cu:460-509), targets
    by trilinear Catmull-Rom across their own mip chains (train.cu:78-103); z past the last
    mip clamps to it."""
    say(f"case: train {shape} at mip coordinate {z}")
    st = make_state(shape, image=128, region=(64, 32), offset=(30, 61), seed=14)
    rng = np.random.default_rng(15)
    st.textures = [_texture_chain(128, n, rng, 5, 1.0 + 0.5 * k) for k, n in enumerate(SHAPES_TEX[shape])]
    st.sample_mip = z
    gs = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    assert O.ntref_train_step(C.byref(st.params()), abi.NT_UNCONSTRAINED, 1) == 0
    nt.check(lib.nt_train_step(C.byref(gs.params()), abi.NT_UNCONSTRAINED, None))
    sync()
    for l in range(st.net.num_layers):
        assert_close(gs.net.weight_grads[l], st.net.weight_grads[l], f"dW{l}")
        assert_close(gs.net.bias_grads[l], st.net.bias_grads[l], f"db{l}")
    for gi, (g, gg) in enumerate(zip(st.grids, gs.grids)):
        got = to_np(gg.grads)
        assert np.count_nonzero(g.grads[g.mip_offsets[0] * g.channels:g.mip_offsets[1] * g.channels]) == 0 or z < 1
        assert_close(got.reshape(-1, g.channels), g.grads, f"latent grad {gi} [texel, channel]")
        assert np.all(got[g.grads == 0] == 0)


SHAPES_TEX = {"ref": [3, 3, 1], "c1": [3], "c2": [3, 3, 3], "c4": [4, 4, 4]}


@pytest.mark.parametrize("shape", ["ref", "c1", "c2", "c4"])
@pytest.mark.parametrize("z", [0.5, 1.0, 2.25, 9.0])
def test_block_train_step_at_mip_coordinate(lib, O, shape, z):
    """BC6 block records sampled at a mip coordinate z > 0: the reference's block sampler and
    its backward blend mips floor(z) and floor(z) + 1 (train.cu:316-371, 373-458; z past the
    last mip clamps to it, and mips narrower than a block hold one partial block). Both
    levels are expanded, trained as unconstrained texels and folded back; MLP and block
    gradients match the oracle's at the MLP bar."""
    say(f"case: BC6 blocks {shape} at mip coordinate {z}")

    def state():
        x = make_state(shape, image=128, region=(64, 32), offset=(30, 61), seed=14, blocks=True)
        rng = np.random.default_rng(15)
        x.textures = [_texture_chain(128, n, rng, 5, 1.0 + 0.5 * k) for k, n in enumerate(SHAPES_TEX[shape])]
        x.sample_mip = z
        return x
    st, alt = state(), state()
    gs = gpu_workspace(lib, st.to_torch(), abi.NT_BLOCK_FEATURES)
    oracle_step(O, st, abi.NT_BLOCK_FEATURES)
    oracle_step(O, alt, abi.NT_BLOCK_FEATURES, accum_f32=True)
    nt.check(lib.nt_train_step(C.byref(gs.params()), abi.NT_BLOCK_FEATURES, None))
    sync()
    check_train_grads(st, gs, alt, abi.NT_BLOCK_FEATURES)
    for g in st.grids:  # some record beyond mip 0 is reached (z >= 1: none at mip 0)
        rec = 4 * g.channels + 16
        nb0 = (max(g.width >> 2, 1) * max(g.height >> 2, 1)) * rec
        assert np.count_nonzero(g.block_grads[nb0:]) > 0
        assert z < 1 or np.count_nonzero(g.block_grads[:nb0]) == 0


# ---- one training-loop iteration in one call ---------------------------------------------------

def _all_buffers(s):
    for gi, g in enumerate(s.grids):
        for name in ("values", "grads", "moment1", "moment2", "block_params", "block_grads", "block_moment1",
                     "block_moment2"):
            a = getattr(g, name)
            if a is not None:
                yield f"grid {gi} {name}", a
    for name in ("weights", "biases", "weight_grads", "weight_moment1", "weight_moment2", "bias_grads",
                 "bias_moment1", "bias_moment2"):
        for l, a in enumerate(getattr(s.net, name)):
            yield f"{name}[{l}]", a


def _run_iterations(lib, a, b, ktype, offs):
    for i in range(len(offs)):
        for s in (a, b):
            s.texel_offset_x, s.texel_offset_y = int(offs[i][0]), int(offs[i][1])
            s.step = 1 + i
            s.feature_adam = (0.9, 0.999, 1e-2 * 0.9999 ** i, 1e-8)
        nt.check(lib.nt_train_iteration(C.byref(a.params()), ktype, None))
        pb = b.params()
        nt.check(lib.nt_train_step(C.byref(pb), ktype, None))
        nt.check(lib.nt_optimize_network(C.byref(pb), None))
        nt.check(lib.nt_optimize_latents(C.byref(pb), ktype, None))
        sync()
        yield i


@pytest.mark.parametrize("shape,mode,update,ktype,blocks,image,region,flags", [
    ("c2", abi.NT_SAMPLES_REGION, abi.NT_LATENT_TOUCHED, abi.NT_UNCONSTRAINED, False, 128, (64, 32), 0),
    ("c4", abi.NT_SAMPLES_REGION, abi.NT_LATENT_DENSE, abi.NT_UNCONSTRAINED, False, 128, (64, 32), 0),
    ("c2", abi.NT_SAMPLES_RANDOM, abi.NT_LATENT_TOUCHED, abi.NT_UNCONSTRAINED, False, 128, (64, 32), 0),
    ("ref", abi.NT_SAMPLES_REGION, abi.NT_LATENT_DENSE, abi.NT_UNCONSTRAINED, False, 128, (64, 32), 0),
    ("ref", abi.NT_SAMPLES_REGION, abi.NT_LATENT_DENSE, abi.NT_BLOCK_FEATURES, True, 128, (64, 32), 0),
    ("ref16", abi.NT_SAMPLES_REGION, abi.NT_LATENT_TOUCHED, abi.NT_UNCONSTRAINED, False, 128, (64, 32), 0),
    ("ref16f", abi.NT_SAMPLES_REGION, abi.NT_LATENT_DENSE, abi.NT_UNCONSTRAINED, False, 128, (64, 32), 0),
    # more partial rows than reduction ranges (one row per train workgroup: 128 for c2,
    # one per CU for c4), so a different split of the rows would change the sums' bits
    ("c2", abi.NT_SAMPLES_REGION, abi.NT_LATENT_TOUCHED, abi.NT_UNCONSTRAINED, False, 512, (512, 256), 0),
    ("c4", abi.NT_SAMPLES_REGION, abi.NT_LATENT_TOUCHED, abi.NT_UNCONSTRAINED, False, 512, (512, 256), 0),
    # random texels in bin order (a step sorts from 262,144 samples): the same sort on both
    # paths, so the same slots
    ("c2", abi.NT_SAMPLES_RANDOM, abi.NT_LATENT_TOUCHED, abi.NT_UNCONSTRAINED, False, 128, (64, 32),
     abi.NT_HOOK_SORT_RANDOM),
], ids=["c2-touched", "c4-dense", "c2-random-touched", "ref", "ref-blocks", "ref16-touched", "ref16f-dense",
        "c2-many-rows", "c4-many-rows", "c2-random-sorted"])
def test_train_iteration_equals_three_calls(lib, shape, mode, update, ktype, blocks, image, region, flags):
    """nt_train_iteration (the train step with the MLP-gradient reduction and both
    optimizers in one launch) against nt_train_step + nt_optimize_network +
    nt_optimize_latents, over four iterations with moving regions and a decaying feature
    learning rate (main.cpp:1043-1077). The network's weights, moments and gradients are
    bit-identical (its gradient is summed in a fixed order on both paths). The latent
    gradients are sums of float atomics whose order varies from run to run (as the
    reference's atomicAdd does), so latent state is compared at the 1e-5 Adam tolerance and
    every latent gradient must be consumed (zero) on both paths; the second path's latents
    then take the first path's values, so that every iteration starts both paths from the
    same inputs (a last-bit latent difference can flip an fp16 feature rounding and with it
    the next step's network gradient)."""
    import torch
    say(f"case: train iteration {shape} mode {mode} update {update} type {ktype} image {image} region {region} "
        f"flags {flags}")
    nt.check(lib.nt_set_test_hooks(0, flags))  # before the workspaces are sized
    try:
        st = make_state(shape, image=image, region=region, seed=9, blocks=blocks)
        st.sample_mode = mode
        st.latent_update = update
        a = gpu_workspace(lib, st.to_torch(), ktype)
        b = gpu_workspace(lib, st.to_torch(), ktype)
        # Past the first iteration the latents of the two paths differ by the order of their
        # float atomics, which at 131,072 samples flips fp16 feature roundings and with them
        # every later gradient; the large cases therefore check the one iteration whose inputs
        # are identical on both paths.
        n_iter = 4 if image <= 128 else 1
        offs = np.random.default_rng(5).integers(0, max(image - region[0], 1), size=(n_iter, 2))
        for i in _run_iterations(lib, a, b, ktype, offs):
            bb = dict(_all_buffers(b))
            for name, x in _all_buffers(a):
                y = bb[name]
                if name.startswith("grid"):
                    xf, yf = x.float(), y.float()
                    scale = max(float(yf.abs().max()), 1e-30)
                    assert float((xf - yf).abs().max()) <= 1e-5 * scale, f"iteration {i}: {name}"
                    if "grads" in name:
                        assert torch.count_nonzero(x) == 0 and torch.count_nonzero(y) == 0, f"iteration {i}: {name}"
                else:
                    assert torch.equal(x.view(torch.uint8), y.view(torch.uint8)), f"iteration {i}: {name}"
            for name, x in _all_buffers(a):
                if name.startswith("grid"):
                    bb[name].copy_(x)
            sync()
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))
    assert torch.count_nonzero(a.net.weight_moment1[0]) > 0


@pytest.mark.parametrize("update", [abi.NT_LATENT_TOUCHED, abi.NT_LATENT_DENSE], ids=["touched", "dense"])
def test_train_iteration_bit_identical_single_chunk(lib, update):
    """With one chunk of samples (a 16 x 8 region, one workgroup) every latent texel takes at
    most one atomic add per step, so both paths see identical gradients and every buffer,
    latent and network, must agree bit for bit."""
    import torch
    say(f"case: train iteration single chunk update {update}")
    st = make_state("c2", image=64, region=(16, 8), seed=11)
    st.latent_update = update
    a = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    b = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    nt.check(lib.nt_set_test_hooks(1, 0))
    try:
        for i in _run_iterations(lib, a, b, abi.NT_UNCONSTRAINED, [(3, 5), (40, 17), (9, 30)]):
            bb = dict(_all_buffers(b))
            for name, x in _all_buffers(a):
                assert torch.equal(x.view(torch.uint8), bb[name].view(torch.uint8)), f"iteration {i}: {name}"
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))
    assert torch.count_nonzero(a.grids[0].moment1) > 0


def test_train_iteration_checks_every_argument_first(lib):
    """An argument error of any of the three parts returns before anything is enqueued."""
    import torch
    st = make_state("c2", image=64, region=(32, 16), seed=3)
    a = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    before = a.net.weight_moment1[0].clone(), a.grids[0].values.clone()
    p = a.params()
    p.mlp.weight_moment1[0] = None  # the network optimizer's argument
    assert lib.nt_train_iteration(C.byref(p), abi.NT_UNCONSTRAINED, None) == abi.NT_ERR_NULL_POINTER
    p = a.params()
    p.latents.grids[1].moment2 = None  # the latent optimizer's argument
    assert lib.nt_train_iteration(C.byref(p), abi.NT_UNCONSTRAINED, None) == abi.NT_ERR_NULL_POINTER
    sync()
    assert torch.equal(a.net.weight_moment1[0], before[0]) and torch.equal(a.grids[0].values, before[1])
    assert all(torch.count_nonzero(g.grads) == 0 for g in a.grids)
