#!/usr/bin/env python3
"""Benchmark of the MI355X neural-texture hot path (one GPU).

Headline (`value`): train texels/s on BASELINE config 2 — a full training iteration of the
reference (InvokeTraining -> InvokeOptimizeNetwork -> InvokeOptimizeFeatures,
main.cpp:1071-1076) per step: fused sample/target/MLP fwd+bwd/scatter over a 512 x 512
jittered region (262,144 samples) of a synthetic 2048^2 x 9-channel target, latents
16 ch @ 512^2 + 16 ch @ 256^2, MLP 32->64->64->9 fp16, lazy Adam (lr 1e-2 latents,
5e-3 network). Inputs are resident in HBM before timing; every step changes the region
offset (seeded) and the step counter, as the reference's loop does.

Also reported: decode texels/s (config 5, 8192^2 from codec-quantized 4-grid latents),
codec encode+decode rate (config 3), the dominant kernel's roofline fraction from live HIP
events, and a CPU baseline (the scalar C oracle on a bounded sample, this box's host).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-extras] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "train texels/s + decode texels/s at 1 GPU; % MFMA / HBM roofline"
PEAK_FP16_TFLOPS = 2500.0  # MI355X dense fp16 MFMA
PEAK_HBM_GBS = 8000.0      # MI355X HBM3E
FLOP_PER_TRAIN_SAMPLE_C2 = 40320   # 3 x 2 x (32*64 + 64*64 + 64*9)
FLOP_PER_DECODE_PIXEL = 26112      # 2 x (64*64*3 + 64*12)
FLOP_PER_TRAIN_SAMPLE_C4 = 78336   # 3 x 2 x (64*64*3 + 64*12)
# HBM bytes per config-2 train-kernel launch: rocprofv3 FETCH_SIZE x 2.000 + WRITE_SIZE x 1.000,
# the factors being what the two counters read for a 256 MiB device copy (--copy-probe).
# Counters cannot be read live; re-measure whenever the train kernel changes.
TRAIN_HBM_BYTES_PER_LAUNCH = (7640.7 * 2.0 + 11408.1) * 1024


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
    grids = [S.latent_grid(size, size, mips, 16, seed + 1 + i, device)
             for i, (size, mips) in enumerate(c["grids"])]
    net = P.make_network(c["mlp"], used_outputs=c["mlp"][-1], rng=np.random.default_rng(seed),
                         init="xavier").converted(True, device)
    r = c["region"]
    return P.TrainState(grids, net, textures, n, n, r * r, region_width=r,
                        network_adam=(0.9, 0.999, 5e-3, 1e-8),
                        feature_adam=(0.9, 0.999, 1e-2, 1e-8))


def build_config2(device, seed=1337):
    """BASELINE config 2 on the device."""
    return build_config(device, 2, seed)


def bench_train(lib, nt, args, ev, cfg=2, steps=None, warmup=None, sample_mode=0):
    import torch

    from neural_textures_amd import abi

    device = "cuda:0"
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    st = build_config(device, cfg)
    st.sample_mode = sample_mode
    image, region = st.image_width, st.region_width
    p = st.params()
    ws_bytes = lib.nt_train_workspace_bytes(C.byref(p), abi.NT_UNCONSTRAINED)
    assert ws_bytes > 0, lib.nt_last_error().decode()
    st.workspace = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    p = st.params()
    stream = torch.cuda.current_stream()
    sh = C.c_void_p(stream.cuda_stream)
    total = warmup + steps
    rng = np.random.default_rng(20260411)  # region offsets, like main.cpp:1033-1044
    offs = rng.integers(0, image - region + 1, size=(total + steps, 2))
    base_lr = 1e-2
    torch.cuda.synchronize()

    def step(i, prof=None):
        p.texel_offset_x, p.texel_offset_y = int(offs[i, 0]), int(offs[i, 1])
        p.step = i
        p.feature_adam.learning_rate = base_lr * 0.9995 ** i  # main.cpp:1068-1069
        if prof is not None:
            lib.nt_profile_next_launch(prof[0], prof[1])
        nt.check(lib.nt_train_step(C.byref(p), abi.NT_UNCONSTRAINED, sh))
        nt.check(lib.nt_optimize_network(C.byref(p), sh))
        nt.check(lib.nt_optimize_latents(C.byref(p), abi.NT_UNCONSTRAINED, sh))

    for i in range(warmup):
        step(i)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(warmup, total):
        step(i)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    ms_per_step = (t1 - t0) * 1e3 / steps

    # Dominant kernel (the fused train kernel) timed with events on its own stream.
    pairs = [(ev.create(), ev.create()) for _ in range(steps)]
    for k in range(steps):
        step(total + k, pairs[k])
    torch.cuda.synchronize()
    kms = [ev.ms(a, b) for a, b in pairs]
    for a, b in pairs:
        ev.destroy(a)
        ev.destroy(b)
    kernel_ms = float(np.mean(kms))
    assert np.isfinite(st.grids[0].values.float().sum().item())
    return st, ms_per_step, kernel_ms, float(np.median(kms))


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
    return ms, float(np.mean(ktimes)), W * H, nbytes


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
    enc_ms, dec_ms = [], []
    a, b = ev.create(), ev.create()
    for _ in range(reps):
        lib.nt_profile_next_launch(a, b)
        nt.check(lib.nt_codec_encode(vals.data_ptr(), W, H, C16, blocks.data_ptr(), sh))
        torch.cuda.synchronize()
        enc_ms.append(ev.ms(a, b))
        lib.nt_profile_next_launch(a, b)
        nt.check(lib.nt_codec_decode(blocks.data_ptr(), W, H, C16, dec.data_ptr(), sh))
        torch.cuda.synchronize()
        dec_ms.append(ev.ms(a, b))
    ev.destroy(a)
    ev.destroy(b)
    err = (dec - vals).abs().max().item()
    return float(np.mean(enc_ms)), float(np.mean(dec_ms)), W * H, err


def cpu_baseline(st_gpu, budget_s=12.0):
    """The scalar C oracle (one host thread) on a bounded sample of config 2: the first rows
    of the same 512-wide region with the same latents, network and target, plus one dense
    lazy-Adam pass over all parameters; extrapolated to a full 262,144-sample step."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_lib import load_oracle

    O = load_oracle()
    host = st_gpu.to_numpy()
    host.workspace = None
    for g in host.grids:
        g.grads[:] = 0
    for lst in (host.net.weight_grads, host.net.bias_grads):
        for a in lst:
            a[:] = 0
    host.texel_offset_x = host.texel_offset_y = 0
    host.step = 1

    def run(n):
        host.num_samples = n
        p = host.params()
        t = time.perf_counter()
        assert O.ntref_train_step(C.byref(p), 0, 1) == 0
        return time.perf_counter() - t

    t_cal = run(1024)
    n = int(min(262144, max(1024, budget_s / max(t_cal / 1024, 1e-9))))
    n = max(512, (n // 512) * 512)
    t_train = run(n)
    p = host.params()
    t = time.perf_counter()
    O.ntref_optimize_network(C.byref(p))
    O.ntref_optimize_latents(C.byref(p), 0)
    t_adam = time.perf_counter() - t
    per_step = t_train / n * 262144 + t_adam
    nlat = sum(g.texels * g.channels for g in host.grids)
    return {
        "value": 262144 / per_step,
        "unit": "train texels/s",
        "cores": 1,
        "kind": "port",
        "sample": f"{n} of 262,144 samples of one config-2 step (train {t_train:.2f} s) + one "
                  f"dense lazy-Adam pass over all {nlat / 1e6:.1f}M latent and 7K network parameters "
                  f"({t_adam:.2f} s), extrapolated to a full step; scalar C oracle, -O2, "
                  f"one thread, host {os.uname().nodename}",
    }


def main():
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-extras", action="store_true", help="skip decode and codec")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="BYTES",
                    help="first run one device-to-device copy of BYTES (a known-size kernel for "
                         "calibrating rocprofv3 FETCH_SIZE / WRITE_SIZE counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (got --gpus {args.gpus}); the path "
              "would shard by training region, one process per GPU, with one all-reduce of the "
              "MLP gradient per step; only the one-GPU share is built", file=sys.stderr)
        sys.exit(2)

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

    log("bench: config 2 train steps")
    st, ms_per_step, kernel_ms, kernel_med = bench_train(lib, nt, args, ev)
    value = 262144 / (ms_per_step / 1e3)
    kflops = FLOP_PER_TRAIN_SAMPLE_C2 * 262144
    achieved = kflops / (kernel_ms / 1e3) / 1e12
    result = {
        "metric": METRIC,
        "value": value,
        "unit": "texels/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded value-noise + sinusoid target, U[-1,1] latents, Xavier fp16 MLP)",
        "config": {
            "workload": "BASELINE config 2 train step: 262,144 jittered samples of a 512^2 region "
                        "of a 2048^2x9 target; latents 16ch@512^2+16ch@256^2; MLP 32-64-64-9 fp16; "
                        "L2 loss; lazy Adam on network and latents",
            "batch": 262144,
            "step": "nt_train_step + nt_optimize_network + nt_optimize_latents",
        },
        "roofline": {
            "kernel": "train16_kernel<Shape<32,64,2>,2> (fused sample/target/MLP fwd+bwd/scatter)",
            "bound": "mfma",
            "achieved": achieved,
            "peak": PEAK_FP16_TFLOPS,
            "unit": "TFLOP/s",
            "frac": achieved / PEAK_FP16_TFLOPS,
            "traffic": TRAIN_HBM_BYTES_PER_LAUNCH,
            "traffic_unit": "bytes/launch (rocprofv3 FETCH_SIZE+WRITE_SIZE, copy-calibrated)",
            "launch_ms_mean": kernel_ms,
            "launch_ms_median": kernel_med,
            "flop_per_launch": kflops,
        },
    }
    if not args.no_extras:
        log("bench: config 4 train steps")
        st4, ms4, k4, _ = bench_train(lib, nt, args, ev, cfg=4, steps=10, warmup=3)
        n4 = st4.num_samples
        ach4 = FLOP_PER_TRAIN_SAMPLE_C4 * n4 / (k4 / 1e3) / 1e12
        result["train_config4"] = {
            "value": n4 / (ms4 / 1e3), "unit": "texels/s", "ms_per_step": ms4, "steps": 10,
            "workload": "BASELINE config 4 train step: 1,048,576 jittered samples of a 1024^2 region "
                        "of a 4096^2x12 target; latents 16ch@1024^2..128^2 (4 grids); MLP "
                        "64-64-64-64-12 fp16; lazy Adam",
            "roofline": {"kernel": "train16_kernel<Shape<64,64,3>,1>", "bound": "mfma",
                         "achieved": ach4, "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                         "frac": ach4 / PEAK_FP16_TFLOPS, "launch_ms_mean": k4}}
        del st4
        log("bench: config 2 train steps, uniform-random texels")
        str_, msr, kr, _ = bench_train(lib, nt, args, ev, cfg=2, steps=20, warmup=5, sample_mode=1)
        achr = FLOP_PER_TRAIN_SAMPLE_C2 * 262144 / (kr / 1e3) / 1e12
        result["train_config2_random_texels"] = {
            "value": 262144 / (msr / 1e3), "unit": "texels/s", "ms_per_step": msr, "steps": 20,
            "workload": "config 2 with NT_SAMPLES_RANDOM: 262,144 samples at uniformly random "
                        "texels of the whole 2048^2 image (no region locality: gathers, target "
                        "taps and latent-gradient atomics all go to L2/HBM)",
            "roofline": {"kernel": "train_kernel<Shape<32,64,2>,16,UNCONSTRAINED>", "bound": "mfma",
                         "achieved": achr, "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                         "frac": achr / PEAK_FP16_TFLOPS, "launch_ms_mean": kr}}
        del str_
        log("bench: config 5 decode")
        dms, kms, npx, wsb = bench_decode(lib, nt, ev)
        dach = FLOP_PER_DECODE_PIXEL * npx / (kms / 1e3) / 1e12
        result["decode"] = {"value": npx / (dms / 1e3), "unit": "decode texels/s", "ms": dms,
                            "workload": "BASELINE config 5: 8192^2 fp16 x12 from codec latents "
                                        "(4 grids 16ch 1024..128, mips 9..6), jitter + z~U[0,3]; "
                                        "two passes (block expand to fp16 texels + sample/MLP)",
                            "workspace_bytes": wsb,
                            "roofline": {"kernel": "decode_box_kernel<Shape<64,64,3>>",
                                         "bound": "mfma", "achieved": dach, "peak": PEAK_FP16_TFLOPS,
                                         "unit": "TFLOP/s", "frac": dach / PEAK_FP16_TFLOPS,
                                         "launch_ms_mean": kms}}
        log("bench: config 3 codec")
        ems, cms, ntex, err = bench_codec(lib, nt, ev)
        enc_bytes = ntex * 16 * 4 + ntex * 12  # fp32 in + 0.75 B/texel/channel out
        result["codec"] = {"encode_ms": ems, "decode_ms": cms,
                           "encode_texels_per_s": ntex / (ems / 1e3),
                           "decode_texels_per_s": ntex / (cms / 1e3),
                           "encode_GBps": enc_bytes / (ems / 1e3) / 1e9,
                           "decode_GBps": enc_bytes / (cms / 1e3) / 1e9,
                           "max_abs_roundtrip_error": err,
                           "workload": "BASELINE config 3: 4096^2 x 16 fp32 N(0,0.5)"}
    if not args.no_cpu:
        log("bench: CPU baseline (oracle)")
        result["cpu_baseline"] = cpu_baseline(st)
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
