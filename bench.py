#!/usr/bin/env python3
"""Benchmark of the MI355X neural-texture hot path (one GPU).

Headline (`value`): train texels/s on BASELINE config 4, the largest single-GPU
configuration — one full training iteration of the reference (InvokeTraining ->
InvokeOptimizeNetwork -> InvokeOptimizeFeatures, main.cpp:1071-1076) per step: fused
sample / Catmull-Rom target / MLP fwd+bwd / latent scatter over a 1024 x 1024 jittered
region (1,048,576 samples) of a synthetic 4096^2 x 12-channel target, latents 4 grids x 16
channels at 1024^2 .. 128^2, MLP 64->64->64->64->12 fp16, lazy Adam (lr 1e-2 latents, 5e-3
network). Inputs are resident in HBM before timing; every step moves the region (seeded)
and advances the step counter, as the reference loop does.

Extras on the same JSON line: config 2 (region and uniform-random texels), config 5 decode
(8192^2 from codec latents), config 3 codec, config 1 Catmull-Rom forward; the roofline of
the dominant kernel from live HIP events; CPU baselines (the scalar C oracle, one thread
and OpenMP over the host's cores) for every configuration, on bounded samples.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--only c4,c2,...] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import platform
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "train texels/s + decode texels/s at 1 GPU; % MFMA / HBM roofline"
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
FLOP_PER_TRAIN_SAMPLE = {0: 10176,   # 3 x 2 x (12*32 + 32*32 + 32*9)
                         10: 10176,  # the same network
                         2: 40320,   # 3 x 2 x (32*64 + 64*64 + 64*9)
                         4: 78336}   # 3 x 2 x (64*64*3 + 64*12)
FLOP_PER_DECODE_PIXEL = 26112        # 2 x (64*64*3 + 64*12)
FLOP_PER_FORWARD_C1 = 9600           # 2 x (8*64 + 64*64 + 64*3)
# HBM bytes per train-kernel launch: rocprofv3 FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000 (KiB),
# the factors being what the two counters read for a 256 MiB device copy (--copy-probe).
# Counters cannot be read live; re-measured whenever the kernel changes.
TRAIN_HBM_BYTES_PER_LAUNCH = {0: (7102.0 * 2.0 + 4181.4) * 1024,
                              2: (7669.1 * 2.0 + 11470.0) * 1024,
                              4: (29020.1 * 2.0 + 37302.6) * 1024,
                              10: (9164.4 * 2.0 + 8478.5) * 1024}
# Random-texel steps: algorithmic bytes per sample = corner gathers (grids x 4 x 64 B) +
# gradient read-modify-write (2 x that) + the targets' channels at 16 taps x 4 B.
RANDOM_BYTES_PER_SAMPLE = {2: 2 * 4 * 64 * 3 + 16 * 9 * 4,    # 2,112
                           4: 4 * 4 * 64 * 3 + 16 * 12 * 4}   # 3,840
TRAIN_HBM_BYTES_RANDOM = {2: (201679.5 * 2.0 + 138384.0) * 1024,    # same counters, config 2 random texels
                          4: (885876.8 * 2.0 + 1183510.6) * 1024}   # and config 4 random texels (both bin-sorted)
# The BC6 block phase's train kernel (the reference network on texels expanded from its
# BCf-2k block records), same counters.
TRAIN_HBM_BYTES_BC6 = (9164.0 * 2.0 + 8478.2) * 1024
WORKLOADS = ("c4", "c2", "c2r", "c4r", "c5", "c3", "c1", "cref", "cref2k", "crefbc6")


def log(msg):
    print(msg, file=sys.stderr, flush=True)


class HipEvents:
    """hipEvent_t pairs through the HIP runtime torch already loaded."""

    def __init__(self):
        self.hip = C.CDLL("libamdhip64.so.7")
        self.hip.hipEventCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [C.POINTER(C.c_float), C.c_void_p, C.c_void_p]
        self.hip.hipEventDestroy.argtypes = [C.c_void_p]
        self.hip.hipEventRecord.argtypes = [C.c_void_p, C.c_void_p]

    def record(self, e, stream):
        assert self.hip.hipEventRecord(e, stream) == 0

    def create(self):
        e = C.c_void_p()
        assert self.hip.hipEventCreate(C.byref(e)) == 0
        return e

    def ms(self, a, b):
        out = C.c_float()
        assert self.hip.hipEventElapsedTime(C.byref(out), a, b) == 0
        return out.value

    def destroy(self, e):
        self.hip.hipEventDestroy(e)


# Train configurations: image size, target channels (packed per texture), latent grids
# (size, mips), MLP sizes, training region side (batch = region^2).
TRAIN_CONFIGS = {
    # The reference's own network (train.h:9-20, main.cpp:72-77 mode 0): 4 grids of 3
    # channels, 12 -> 32 -> 32 -> 16 with 9 outputs in use, 262,144 samples of a 512^2 region.
    0: dict(image=2048, channels=9, per_texture=3, grids=[(512, 8), (256, 7), (128, 6), (64, 5)],
            mlp=[12, 32, 32, 16], used=9, latent_channels=3, region=512),
    # The same network with the grids of main.cpp's default mode (BCf-2k, main.cpp:56, 75):
    # the two finest grids are as fine as the 2048^2 target and half as fine.
    10: dict(image=2048, channels=9, per_texture=3, grids=[(2048, 10), (1024, 9), (512, 8), (256, 7)],
             mlp=[12, 32, 32, 16], used=9, latent_channels=3, region=512),
    # main.cpp's other grid modes (main.cpp:73-76), used by the full-size tests only:
    # BCf-1k and BCf-2k++ (two grids as fine as the target).
    11: dict(image=2048, channels=9, per_texture=3, grids=[(1024, 9), (512, 8), (256, 7), (128, 6)],
             mlp=[12, 32, 32, 16], used=9, latent_channels=3, region=512),
    12: dict(image=2048, channels=9, per_texture=3, grids=[(2048, 10), (2048, 10), (512, 8), (256, 7)],
             mlp=[12, 32, 32, 16], used=9, latent_channels=3, region=512),
    2: dict(image=2048, channels=9, per_texture=3, grids=[(512, 8), (256, 7)],
            mlp=[32, 64, 64, 9], region=512),
    4: dict(image=4096, channels=12, per_texture=4, grids=[(1024, 9), (512, 8), (256, 7), (128, 6)],
            mlp=[64, 64, 64, 64, 12], region=1024),
}


def build_config(device, cfg=2, seed=1337):
    """A BASELINE train configuration on the device (synthetic target, U[-1,1] latents)."""
    from neural_textures_amd import params as P, synthetic as S

    c = TRAIN_CONFIGS[cfg]
    n = c["image"]
    textures = S.target_textures(n, n, c["channels"], c["per_texture"], seed, device)
    grids = [S.latent_grid(size, size, mips, c.get("latent_channels", 16), seed + 1 + i, device)
             for i, (size, mips) in enumerate(c["grids"])]
    net = P.make_network(c["mlp"], used_outputs=c.get("used", c["mlp"][-1]), rng=np.random.default_rng(seed),
                         init="xavier").converted(True, device)
    r = c["region"]
    return P.TrainState(grids, net, textures, n, n, r * r, region_width=r,
                        network_adam=(0.9, 0.999, 5e-3, 1e-8),
                        feature_adam=(0.9, 0.999, 1e-2, 1e-8))


def build_config2(device, seed=1337):
    """BASELINE config 2 on the device."""
    return build_config(device, 2, seed)


def bench_train(lib, nt, ev, cfg, steps, warmup, sample_mode=0, blocks=False):
    """K timed steps (after W warm-up steps), each one nt_train_iteration (train step, network
    and latent optimizers, the same results as the three separate calls); then K timed steps
    made of the three separate calls (nt_train_step, nt_optimize_network,
    nt_optimize_latents); then K more with the train kernel bracketed by HIP events on its
    stream. With `blocks` the latents are BC6 block records (NT_BLOCK_FEATURES, the
    reference's block phase, main.cpp:1052-1060), initialised from the synthetic latents by
    nt_bc6_init before the warm-up."""
    import torch

    from neural_textures_amd import abi

    device = "cuda:0"
    st = build_config(device, cfg)
    st.sample_mode = sample_mode
    # The optimizer visits the texel (or block-record) rectangles the train step logged
    # (same results as the reference's dense scan, which the tests check).
    st.latent_update = abi.NT_LATENT_TOUCHED
    ktype = abi.NT_BLOCK_FEATURES if blocks else abi.NT_UNCONSTRAINED
    if blocks:
        for g in st.grids:
            rec = 4 * g.channels + 16
            g.block_params = torch.zeros(g.blocks * (rec + 2), device=device)
            g.block_grads, g.block_moment1, g.block_moment2 = (
                torch.zeros(g.blocks * rec, device=device) for _ in range(3))
        p = st.params()
        nt.check(lib.nt_bc6_init(C.byref(p.latents), None))
    image, region = st.image_width, st.region_width
    p = st.params()
    ws_bytes = lib.nt_train_workspace_bytes(C.byref(p), ktype)
    assert ws_bytes > 0, lib.nt_last_error().decode()
    st.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    p = st.params()
    stream = torch.cuda.current_stream()
    sh = C.c_void_p(stream.cuda_stream)
    total = warmup + steps
    rng = np.random.default_rng(20260411)  # region offsets, like main.cpp:1033-1044
    offs = rng.integers(0, image - region + 1, size=(total + 2 * steps, 2))
    base_lr = 1e-2
    torch.cuda.synchronize()

    def step(i, prof=None, separate=False):
        p.texel_offset_x, p.texel_offset_y = int(offs[i % len(offs), 0]), int(offs[i % len(offs), 1])
        p.step = i
        p.feature_adam.learning_rate = base_lr * 0.9995 ** i  # main.cpp:1068-1069
        if prof is not None:
            lib.nt_profile_next_launch(prof[0], prof[1])
        if separate:
            nt.check(lib.nt_train_step(C.byref(p), ktype, sh))
            nt.check(lib.nt_optimize_network(C.byref(p), sh))
            nt.check(lib.nt_optimize_latents(C.byref(p), ktype, sh))
        else:
            nt.check(lib.nt_train_iteration(C.byref(p), ktype, sh))

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup, total):
        step(i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / steps
    t0 = time.perf_counter()
    for i in range(total, total + steps):
        step(i, separate=True)
    torch.cuda.synchronize()
    ms_separate = (time.perf_counter() - t0) * 1e3 / steps

    pairs = [(ev.create(), ev.create()) for _ in range(steps)]
    for k in range(steps):
        step(total + steps + k, pairs[k])
    torch.cuda.synchronize()
    kms = [ev.ms(a, b) for a, b in pairs]
    for a, b in pairs:
        ev.destroy(a)
        ev.destroy(b)
    assert np.isfinite(st.grids[0].values.float().sum().item())
    if blocks:
        assert np.isfinite(st.grids[0].block_params.sum().item())
    return st, ms_per_step, ms_separate, float(np.mean(kms)), float(np.median(kms))


def train_entry(lib, nt, ev, cfg, steps, warmup, sample_mode=0, blocks=False):
    st, ms, ms_sep, kmean, kmed = bench_train(lib, nt, ev, cfg, steps, warmup, sample_mode, blocks)
    n = st.num_samples
    flops = FLOP_PER_TRAIN_SAMPLE[cfg] * n
    achieved = flops / (kmean / 1e3) / 1e12
    kernel = {0: "train16_kernel<Shape<16,32,2>,3,2,false,false>", 10: "train16_kernel<Shape<16,32,2>,3,2,false,false>",
              2: "train16_kernel<Shape<32,64,2>,16,2,false,false>",
              4: "train16_kernel<Shape<64,64,3>,16,1,false,false>"}[cfg]
    if blocks:
        # The block phase: records expanded to texels, this kernel, gradients folded back.
        kernel = "train16_kernel<Shape<16,32,2>,3,2,false,false> (BC6 block phase on expanded texels)"
    if sample_mode:
        kernel = ("train16_kernel<Shape<32,64,2>,16,2,true,true>" if cfg == 2
                  else "train16_kernel<Shape<64,64,3>,16,2,true,true>")
    if sample_mode:
        # Random texels: bound by scattered memory traffic, priced at the algorithmic bytes
        # per sample (corner gathers, gradient read-modify-write, the taps' target channels).
        nbytes = RANDOM_BYTES_PER_SAMPLE[cfg] * n
        gbs = nbytes / (kmean / 1e3) / 1e9
        roof = {"kernel": kernel, "bound": "hbm", "achieved": gbs, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": gbs / PEAK_HBM_GBS, "traffic": TRAIN_HBM_BYTES_RANDOM.get(cfg),
                "bytes_per_launch": nbytes, "mfma_tflops": achieved, "mfma_frac": achieved / PEAK_FP16_TFLOPS}
    else:
        roof = {"kernel": kernel, "bound": "mfma", "achieved": achieved, "peak": PEAK_FP16_TFLOPS,
                "unit": "TFLOP/s", "frac": achieved / PEAK_FP16_TFLOPS,
                "traffic": TRAIN_HBM_BYTES_BC6 if blocks else TRAIN_HBM_BYTES_PER_LAUNCH.get(cfg),
                "flop_per_launch": flops}
    roof.update({"launch_ms_mean": kmean, "launch_ms_median": kmed})
    return st, {"value": n / (ms / 1e3), "unit": "texels/s", "ms_per_step": ms, "steps": steps, "batch": n,
                "ms_per_step_separate_calls": ms_sep, "roofline": roof}


def bench_decode(lib, nt, ev, reps=3):
    """8192^2 decode from codec-quantized 4-grid 16-channel latents."""
    import torch

    from neural_textures_amd import abi, params as P, synthetic as S

    device = "cuda:0"
    C16 = 16
    shapes = [(1024, 9), (512, 8), (256, 7), (128, 6)]  # BCf-1k (main.cpp:72-77)
    blobs = []
    for gi, (size, mips) in enumerate(shapes):
        offs, total = P.codec_chain_layout(size, size, mips, C16)
        blob = torch.zeros(total, dtype=torch.uint8, device=device)
        for m in range(mips):
            s = P.mip_dim(size, m)
            vals = S.normal_values(s * s * C16, 0.5, 7000 + 10 * gi + m, device)
            nt.check(lib.nt_codec_encode(vals.data_ptr(), s, s, C16, blob.data_ptr() + offs[m], None))
        blobs.append((size, mips, offs, blob))
    net = P.make_network([64, 64, 64, 64, 12], rng=np.random.default_rng(1337),
                         init="xavier").converted(True, device)
    W = H = 8192
    out = torch.empty(W * H * 12, dtype=torch.int16, device=device)
    d = abi.nt_decode_params()
    d.num_grids, d.channels = 4, C16
    for i, (size, mips, offs, blob) in enumerate(blobs):
        g = d.grids[i]
        g.width = g.height = size
        g.num_mips = mips
        for m, o in enumerate(offs):
            g.byte_offset[m] = o
        g.blocks = blob.data_ptr()
    d.mlp = net.struct()
    d.out_width, d.out_height = W, H
    d.seed, d.jitter, d.mip_min, d.mip_max = 5, 1.0, 0.0, 3.0
    d.output = C.cast(out.data_ptr(), abi.u16p)
    # Two-pass decode: blocks -> fp16 texels once, then every pixel samples those. The timed
    # call includes both passes.
    nbytes = lib.nt_decode_workspace_bytes(C.byref(d))
    assert nbytes > 0, lib.nt_last_error().decode()
    ws = torch.empty(nbytes, dtype=torch.uint8, device=device)
    d.workspace, d.workspace_bytes = ws.data_ptr(), nbytes
    sh = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    nt.check(lib.nt_decode(C.byref(d), sh))
    torch.cuda.synchronize()
    a, b, k0, k1 = ev.create(), ev.create(), ev.create(), ev.create()
    times, ktimes = [], []
    for _ in range(reps):
        ev.record(a, sh)
        lib.nt_profile_next_launch(k0, k1)
        nt.check(lib.nt_decode(C.byref(d), sh))
        ev.record(b, sh)
        torch.cuda.synchronize()
        times.append(ev.ms(a, b))
        ktimes.append(ev.ms(k0, k1))
    for e in (a, b, k0, k1):
        ev.destroy(e)
    ms = float(np.mean(times))
    assert torch.isfinite(out[:1 << 20].view(torch.float16).float()).all()
    kms = float(np.mean(ktimes))
    dach = FLOP_PER_DECODE_PIXEL * W * H / (kms / 1e3) / 1e12
    return {"value": W * H / (ms / 1e3), "unit": "decode texels/s", "ms": ms,
            "workload": "BASELINE config 5: 8192^2 fp16 x12 from codec latents (4 grids 16ch "
                        "1024..128, mips 9..6), jitter + z~U[0,3]; two passes (block expand to fp16 "
                        "texels + sample/MLP)",
            "workspace_bytes": nbytes,
            "roofline": {"kernel": "decode_box_kernel<Shape<64,64,3>>", "bound": "mfma",
                         "achieved": dach, "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                         "frac": dach / PEAK_FP16_TFLOPS, "launch_ms_mean": kms}}


def bench_codec(lib, nt, ev, reps=3):
    """4096^2 x 16 fp32 latents N(0, 0.5) -> blocks -> fp32."""
    import torch

    from neural_textures_amd import synthetic as S

    device = "cuda:0"
    W = H = 4096
    C16 = 16
    vals = S.normal_values(W * H * C16, 0.5, 4242, device)
    blocks = torch.empty((W // 4) * (H // 4) * 12 * C16, dtype=torch.uint8, device=device)
    dec = torch.empty_like(vals)
    sh = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    nt.check(lib.nt_codec_encode(vals.data_ptr(), W, H, C16, blocks.data_ptr(), sh))
    nt.check(lib.nt_codec_decode(blocks.data_ptr(), W, H, C16, dec.data_ptr(), sh))
    torch.cuda.synchronize()
    a, b = ev.create(), ev.create()

    def timed(fn):
        lib.nt_profile_next_launch(a, b)
        fn()
        torch.cuda.synchronize()
        return ev.ms(a, b)

    def encode():
        nt.check(lib.nt_codec_encode(vals.data_ptr(), W, H, C16, blocks.data_ptr(), sh))

    def decode():
        nt.check(lib.nt_codec_decode(blocks.data_ptr(), W, H, C16, dec.data_ptr(), sh))

    # Each launch timed alone (HIP events on its stream, a synchronisation after it): the
    # encodes in a row, then the decodes in a row; then alternating pairs, where each decode
    # runs right after an encode has streamed 1.27 GB through the memory system.
    enc_ms = [timed(encode) for _ in range(reps)]
    dec_ms = [timed(decode) for _ in range(reps)]
    pair_ms = [(timed(encode), timed(decode)) for _ in range(reps)]
    ev.destroy(a)
    ev.destroy(b)
    diff = (dec - vals).double()
    err = diff.abs().max().item()
    rmse = diff.pow(2).mean().sqrt().item()
    peak = vals.abs().max().item()
    ntex = W * H
    ems, cms = float(np.mean(enc_ms)), float(np.mean(dec_ms))
    enc_bytes = ntex * C16 * 4 + ntex * 12  # fp32 in + 12 B per block-channel / 16 texels
    return {"encode_ms": ems, "decode_ms": cms,
            "encode_texels_per_s": ntex / (ems / 1e3), "decode_texels_per_s": ntex / (cms / 1e3),
            "encode_GBps": enc_bytes / (ems / 1e3) / 1e9, "decode_GBps": enc_bytes / (cms / 1e3) / 1e9,
            "roofline": {"kernel": "codec_encode_kernel<16>", "bound": "hbm",
                         "achieved": enc_bytes / (ems / 1e3) / 1e9, "peak": PEAK_HBM_GBS, "unit": "GB/s",
                         "frac": enc_bytes / (ems / 1e3) / 1e9 / PEAK_HBM_GBS},
            "decode_ms_after_encode": float(np.mean([p[1] for p in pair_ms])),
            "encode_ms_after_decode": float(np.mean([p[0] for p in pair_ms])),
            "decode_write_GBps": ntex * C16 * 4 / (cms / 1e3) / 1e9,
            "max_abs_roundtrip_error": err, "roundtrip_rmse": rmse,
            "roundtrip_psnr_db": 20 * np.log10(peak / rmse) if rmse > 0 else None,
            "workload": "BASELINE config 3: 4096^2 x 16 fp32 N(0,0.5) encode + decode"}


def bench_forward_c1(lib, nt, ev, reps=5):
    """BASELINE config 1 on the GPU: Catmull-Rom latent sample + MLP 8->64->64->3 at 65,536
    uniform-random UVs of a 256^2 x 8 grid."""
    import torch

    from neural_textures_amd import abi, params as P

    rng = np.random.default_rng(1337)
    grid = P.make_grid(256, 256, 1, 8, rng, with_adam=False).converted(True, "cuda:0")
    net = P.make_network([8, 64, 64, 3], used_outputs=3, rng=rng, init="xavier").converted(True, "cuda:0")
    n = 65536
    uvz = np.zeros((n, 3), np.float32)
    uvz[:, :2] = np.random.default_rng(1338).uniform(0, 1, size=(n, 2))
    guvz = torch.from_numpy(uvz).cuda()
    out = torch.empty(n * 3, dtype=torch.int16, device="cuda:0")
    lat = abi.nt_latents()
    lat.num_grids, lat.channels = 1, 8
    lat.grids[0] = grid.struct()
    sh = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    nt.check(lib.nt_forward(C.byref(lat), C.byref(net.struct()), abi.NT_FILTER_CATMULL_ROM, guvz.data_ptr(),
                            n, None, out.data_ptr(), sh))
    torch.cuda.synchronize()
    a, b = ev.create(), ev.create()
    times = []
    for _ in range(reps):
        lib.nt_profile_next_launch(a, b)
        nt.check(lib.nt_forward(C.byref(lat), C.byref(net.struct()), abi.NT_FILTER_CATMULL_ROM,
                                guvz.data_ptr(), n, None, out.data_ptr(), sh))
        torch.cuda.synchronize()
        times.append(ev.ms(a, b))
    ev.destroy(a)
    ev.destroy(b)
    ms = float(np.mean(times))
    return {"value": n / (ms / 1e3), "unit": "samples/s", "ms": ms,
            "workload": "BASELINE config 1: Catmull-Rom sample of a 256^2x8 grid + MLP 8-64-64-3 "
                        "at 65,536 UVs (cache-resident; a correctness configuration)"}


# ---- CPU baselines (the scalar C oracle) -----------------------------------------------

def host_cpu():
    model = platform.processor() or "unknown"
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    try:
        usable = len(os.sched_getaffinity(0))
    except AttributeError:
        usable = os.cpu_count() or 1
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or usable
    return model, os.cpu_count() or 1, usable, max(1, min(threads, usable))


def _oracle():
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_lib import load_oracle

    return load_oracle()


def cpu_train(O, st_gpu, n, threads):
    """The oracle's train step (sample, target, MLP fwd+bwd, scatter) over the first n
    samples of the configuration's region, plus one dense lazy-Adam pass over every latent
    and network parameter; per-sample rate of the train part, the Adam time per step."""
    host = st_gpu.to_numpy()
    host.workspace = None
    for g in host.grids:
        g.grads[:] = 0
    for lst in (host.net.weight_grads, host.net.bias_grads):
        for a in lst:
            a[:] = 0
    host.texel_offset_x = host.texel_offset_y = 0
    host.step = 1
    host.num_samples = n
    p = host.params()
    t = time.perf_counter()
    assert O.ntref_train_step(C.byref(p), 0, threads) == 0
    t_train = time.perf_counter() - t
    t = time.perf_counter()
    O.ntref_optimize_network(C.byref(p))
    O.ntref_optimize_latents(C.byref(p), 0)
    t_adam = time.perf_counter() - t
    return t_train, t_adam


def cpu_baselines(results, states, threads):
    """Per-configuration CPU rates on bounded samples: train steps single-thread and OpenMP,
    codec and decode tiles, the config-1 forward at full size."""
    from neural_textures_amd import abi, params as P

    O = _oracle()
    out = {}
    for cfg, key, n1, nmt in ((4, "c4", 4096, 65536), (2, "c2", 4096, 65536)):
        st = states.get(cfg)
        if st is None:
            continue
        full = st.num_samples
        t1, adam = cpu_train(O, st, n1, 1)
        tm, _ = cpu_train(O, st, nmt, threads)
        per1 = t1 / n1 * full + adam
        perm = tm / nmt * full + adam
        out[key] = {"single_thread": full / per1, "openmp": full / perm, "threads": threads,
                    "unit": "train texels/s",
                    "sample": f"{n1} (1 thread) and {nmt} ({threads} threads) of the {full:,} samples "
                              f"of one step, + one dense lazy-Adam pass ({adam:.2f} s), extrapolated "
                              "to a full step"}
    # config 3: one 1024^2 x 16 tile, encode + decode, one thread and OpenMP
    rng = np.random.default_rng(4242)
    vals = rng.normal(0, 0.5, size=1024 * 1024 * 16).astype(np.float32)
    blocks = np.zeros(256 * 256 * 12 * 16, np.uint8)
    dec = np.zeros_like(vals)
    c3 = {}
    for th in (1, threads):
        O.ntref_set_threads(th)
        t = time.perf_counter()
        O.ntref_codec_encode(vals.ctypes.data, 1024, 1024, 16, blocks.ctypes.data)
        te = time.perf_counter() - t
        t = time.perf_counter()
        O.ntref_codec_decode(blocks.ctypes.data, 1024, 1024, 16, dec.ctypes.data)
        td = time.perf_counter() - t
        key = "single_thread" if th == 1 else "openmp"
        c3[f"encode_{key}"] = 1024 * 1024 / te
        c3[f"decode_{key}"] = 1024 * 1024 / td
    O.ntref_set_threads(threads)
    out["c3"] = {**c3, "threads": threads, "unit": "texels/s",
                 "sample": "one 1024^2 x 16 tile of the 4096^2 configuration"}
    # config 5: decode of a crop of the 8192^2 output, per pixel
    d5 = results.get("_c5_cpu")
    if d5 is not None:
        out["c5"] = d5
    # config 1: the full 65,536-UV forward, one thread
    rng = np.random.default_rng(1337)
    grid = P.make_grid(256, 256, 1, 8, rng, with_adam=False)
    net = P.make_network([8, 64, 64, 3], used_outputs=3, rng=rng, init="xavier")
    n = 65536
    uvz = np.zeros((n, 3), np.float32)
    uvz[:, :2] = np.random.default_rng(1338).uniform(0, 1, size=(n, 2))
    lat = abi.nt_latents()
    lat.num_grids, lat.channels = 1, 8
    lat.grids[0] = grid.struct()
    outs = np.zeros(n * 3, np.uint16)
    t = time.perf_counter()
    O.ntref_forward(C.byref(lat), C.byref(net.struct()), abi.NT_FILTER_CATMULL_ROM, uvz.ctypes.data, n,
                    None, outs.ctypes.data)
    out["c1"] = {"single_thread": n / (time.perf_counter() - t), "unit": "samples/s",
                 "sample": "the full 65,536 UVs"}
    return out


def cpu_decode_crop(threads):
    """The oracle's decode (config 5 network and latent pyramid shapes, codec latents) on a
    256 x 256 crop with OpenMP and a 64 x 64 crop on one thread; pixels/s."""
    from neural_textures_amd import abi, params as P

    O = _oracle()
    C16 = 16
    rng = np.random.default_rng(7000)
    d = abi.nt_decode_params()
    d.num_grids, d.channels = 4, C16
    keep = []
    for gi, (size, mips) in enumerate([(1024, 9), (512, 8), (256, 7), (128, 6)]):
        offs, total = P.codec_chain_layout(size, size, mips, C16)
        blob = np.zeros(total, np.uint8)
        for m in range(mips):
            s = P.mip_dim(size, m)
            vals = rng.normal(0, 0.5, size=s * s * C16).astype(np.float32)
            O.ntref_codec_encode(vals.ctypes.data, s, s, C16, blob[offs[m]:].ctypes.data)
        keep.append(blob)
        g = d.grids[gi]
        g.width = g.height = size
        g.num_mips = mips
        for m, o in enumerate(offs):
            g.byte_offset[m] = o
        g.blocks = blob.ctypes.data
    net = P.make_network([64, 64, 64, 64, 12], rng=np.random.default_rng(1337), init="xavier")
    d.mlp = net.struct()
    d.seed, d.jitter, d.mip_min, d.mip_max = 5, 1.0, 0.0, 3.0
    rates = {}
    for side, th in ((64, 1), (256, threads)):
        out = np.zeros(side * side * 12, np.uint16)
        d.out_width = d.out_height = side
        d.output = out.ctypes.data_as(abi.u16p)
        t = time.perf_counter()
        O.ntref_decode(C.byref(d), th)
        rates[th] = side * side / (time.perf_counter() - t)
    return {"single_thread": rates[1], "openmp": rates[threads], "threads": threads, "unit": "decode texels/s",
            "sample": "a 64^2 crop (1 thread) and a 256^2 crop (OpenMP) of the 8192^2 decode"}


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=30)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--only", default=",".join(WORKLOADS),
                    help="comma-separated subset of " + ",".join(WORKLOADS) + " (the first is the headline)")
    ap.add_argument("--no-extras", action="store_true", help="the headline only")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baselines")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="first run one device-to-device copy of BYTES (a known-size kernel for "
                         "calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the path "
              "would shard by training region, one process per GPU, with one all-reduce of the "
              "MLP gradient per step; only the one-GPU share is built", file=sys.stderr)
        sys.exit(2)
    only = [w for w in args.only.split(",") if w]
    if args.no_extras:
        only = only[:1]
    assert only and all(w in WORKLOADS for w in only), f"--only takes {WORKLOADS}"

    import torch

    import neural_textures_amd as nt

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    lib = nt.load()
    ev = HipEvents()
    if args.copy_probe:
        src = torch.ones(args.copy_probe // 4, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        torch.cuda.synchronize()
        dst.copy_(src)
        torch.cuda.synchronize()
        log(f"bench: copy probe of {args.copy_probe} bytes done")
        del src, dst

    entries, states = {}, {}
    for w in only:
        log(f"bench: {w}")
        if w in ("c4", "c2"):
            cfg = int(w[1])
            steps = args.steps if w == only[0] else max(10, args.steps // 2)
            st, e = train_entry(lib, nt, ev, cfg, steps, args.warmup)
            e["workload"] = {
                4: "BASELINE config 4 train step: 1,048,576 jittered samples of a 1024^2 region of a "
                   "4096^2x12 target; latents 16ch@1024^2..128^2 (4 grids); MLP 64-64-64-64-12 fp16; "
                   "L2 loss; lazy Adam on network and latents (touched runs)",
                2: "BASELINE config 2 train step: 262,144 jittered samples of a 512^2 region of a "
                   "2048^2x9 target; latents 16ch@512^2+16ch@256^2; MLP 32-64-64-9 fp16; L2 loss; "
                   "lazy Adam on network and latents (touched runs)"}[cfg]
            states[cfg] = st.to_numpy() if not args.no_cpu else None
            del st
        elif w == "cref":
            st, e = train_entry(lib, nt, ev, 0, 20, 5)
            e["workload"] = ("the reference's own network (not a BASELINE config): 262,144 jittered samples "
                             "of a 512^2 region of a 2048^2x9 target; latents 3ch@512^2..64^2 (4 grids); "
                             "MLP 12-32-32-16 (9 outputs used) fp16; lazy Adam on network and latents (touched runs)")
            del st
        elif w == "cref2k":
            st, e = train_entry(lib, nt, ev, 10, 20, 5)
            e["workload"] = ("the reference's own network with the grids of its default mode BCf-2k (not a "
                             "BASELINE config): 262,144 jittered samples of a 512^2 region of a 2048^2x9 "
                             "target; latents 3ch@2048^2..256^2 (4 grids); MLP 12-32-32-16 fp16; lazy Adam")
            del st
        elif w == "crefbc6":
            st, e = train_entry(lib, nt, ev, 10, 20, 5, blocks=True)
            e["workload"] = ("the reference's own network in its BC6 block phase (NT_BLOCK_FEATURES, "
                             "main.cpp:1052-1060; not a BASELINE config): BCf-2k grids 3ch@2048^2..256^2 "
                             "as BC6 block records initialised by nt_bc6_init; 262,144 jittered samples of "
                             "a 512^2 region of a 2048^2x9 target; MLP 12-32-32-16 fp16; lazy Adam on the "
                             "network and on the block records (touched rectangles)")
            del st
        elif w == "c2r":
            st, e = train_entry(lib, nt, ev, 2, 20, 5, sample_mode=1)
            e["workload"] = ("config 2 with NT_SAMPLES_RANDOM (BASELINE's 'random texels'): 262,144 "
                             "samples at uniformly random texels of the whole 2048^2 image")
            del st
        elif w == "c4r":
            st, e = train_entry(lib, nt, ev, 4, 10, 3, sample_mode=1)
            e["workload"] = ("config 4 with NT_SAMPLES_RANDOM (BASELINE's 'random texels'): 1,048,576 "
                             "samples at uniformly random texels of the whole 4096^2 image")
            del st
        elif w == "c5":
            e = bench_decode(lib, nt, ev)
        elif w == "c3":
            e = bench_codec(lib, nt, ev)
        else:
            e = bench_forward_c1(lib, nt, ev)
        entries[w] = e
        torch.cuda.empty_cache()

    head = entries[only[0]]
    names = {"c4": "train_config4", "c2": "train_config2", "c2r": "train_config2_random_texels",
             "c4r": "train_config4_random_texels",
             "c5": "decode", "c3": "codec", "c1": "forward_config1", "cref": "train_reference_network",
             "cref2k": "train_reference_network_bcf2k", "crefbc6": "train_reference_network_bc6_blocks"}
    ms_head = head.get("ms_per_step", head.get("ms", head.get("encode_ms")))
    result = {
        "metric": METRIC,
        "value": head.get("value", head.get("encode_texels_per_s")),
        "unit": head.get("unit", "texels/s"),
        "n_gpus": 1,
        "steps": head.get("steps", args.steps),
        "warmup": args.warmup,
        "ms_per_step": ms_head,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded value-noise + sinusoid target, U[-1,1] latents, Xavier fp16 MLP)",
        "config": {"workload": head.get("workload"), "batch": head.get("batch"),
                   "step": "nt_train_iteration (nt_train_step + nt_optimize_network + nt_optimize_latents, "
                           "the reduction and both optimizers in one launch)"
                   if only[0] in ("c4", "c2", "c2r", "c4r") else None},
        "roofline": head.get("roofline"),
    }
    if "ms_per_step_separate_calls" in head:
        result["ms_per_step_separate_calls"] = head["ms_per_step_separate_calls"]
    for w in only[1:]:
        result[names[w]] = entries[w]
    if not args.no_cpu:
        log("bench: CPU baselines (oracle)")
        model, ncpu, usable, threads = host_cpu()
        extra = {}
        if "c5" in only:
            extra["_c5_cpu"] = cpu_decode_crop(threads)
        per = cpu_baselines(extra, {k: v for k, v in states.items() if v is not None}, threads)
        hk = only[0] if only[0] in per else None
        if hk is not None:
            b = per[hk]
            # The codec's figures are per direction; its headline is the encode.
            par = b.get("openmp", b.get("encode_openmp", b.get("single_thread")))
            one = b.get("single_thread", b.get("encode_single_thread"))
            result["cpu_baseline"] = {
                "value": par if par is not None else one, "unit": b["unit"],
                "cores": b.get("threads", 1) if par is not None else 1, "kind": "port",
                "single_thread": one,
                "sample": b["sample"] + f"; scalar C oracle (-O2, no fast-math); host CPU {model}, "
                                        f"nproc {ncpu}, {usable} usable",
            }
        result["cpu_baselines"] = {"cpu_model": model, "nproc": ncpu, "usable_cores": usable,
                                   "kind": "port", **per}
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
