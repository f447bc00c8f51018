"""The C-ABI library on the CPU: it loads, exports every function include/nt/nt.h declares,
its struct layouts match the ctypes mirror, and its host-only helpers and argument checks
work (no kernel is launched: every call here fails validation before touching HIP)."""
import ctypes as C
import os
import re
import subprocess
import tempfile

import numpy as np
import pytest

import neural_textures_amd as nt
from neural_textures_amd import abi, params as P

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nt", "nt.h")


def declared_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(nt_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(nt.LIBRARY_PATH):
        pytest.fail("libnt_hip.so is not built (run __graft_entry__.build())")
    return nt.load()


def test_exports_every_declared_function(lib):
    names = declared_functions()
    assert len(names) >= 17
    out = subprocess.run(["nm", "-D", "--defined-only", nt.LIBRARY_PATH], capture_output=True,
                         text=True, check=True).stdout
    exported = set(re.findall(r" T (nt_\w+)", out))
    assert set(names) <= exported, set(names) - exported
    assert set(names) == set(abi.SIGNATURES), "abi.py and nt.h disagree"


def test_struct_layout_matches_c():
    structs = {"nt_adam": abi.nt_adam, "nt_grid": abi.nt_grid, "nt_latents": abi.nt_latents,
               "nt_mlp": abi.nt_mlp, "nt_texture": abi.nt_texture, "nt_params": abi.nt_params,
               "nt_codec_grid": abi.nt_codec_grid, "nt_decode_params": abi.nt_decode_params,
               "nt_model_info": abi.nt_model_info, "nt_model_data": abi.nt_model_data}
    lines = ['#include <stdio.h>', '#include <stddef.h>', f'#include "{HEADER}"', "int main(void){"]
    for name, cls in structs.items():
        lines.append(f'printf("{name} %zu\\n", sizeof({name}));')
        for fname, _ in cls._fields_:
            lines.append(f'printf("{name}.{fname} %zu\\n", offsetof({name}, {fname}));')
    lines.append("return 0;}")
    with tempfile.TemporaryDirectory() as d:
        src, exe = os.path.join(d, "l.c"), os.path.join(d, "l")
        open(src, "w").write("\n".join(lines))
        subprocess.run(["gcc", "-o", exe, src], check=True)
        out = subprocess.run([exe], capture_output=True, text=True, check=True).stdout
    got = dict(line.rsplit(" ", 1) for line in out.strip().splitlines())
    for name, cls in structs.items():
        assert int(got[name]) == C.sizeof(cls), name
        for fname, _ in cls._fields_:
            assert int(got[f"{name}.{fname}"]) == getattr(cls, fname).offset, f"{name}.{fname}"


def test_layout_helpers(lib):
    offs = (C.c_int64 * 16)()
    for w, h, m in [(512, 512, 8), (1024, 256, 11), (3, 5, 3), (1, 1, 1)]:
        total = lib.nt_mip_chain_layout(w, h, m, offs)
        want, wt = P.mip_chain_layout(w, h, m)
        assert total == wt and list(offs)[:m] == want
        total = lib.nt_block_chain_layout(w, h, m, offs)
        want, wt = P.block_chain_layout(w, h, m)
        assert total == wt and list(offs)[:m] == want
        for c in (4, 8, 16):
            total = lib.nt_codec_mip_chain_layout(w, h, m, c, offs)
            want, wt = P.codec_chain_layout(w, h, m, c)
            assert total == wt and list(offs)[:m] == want
    assert lib.nt_mip_chain_layout(0, 4, 1, offs) == -1
    assert lib.nt_codec_block_bytes(16) == 192 and lib.nt_codec_block_bytes(3) == 0
    assert lib.nt_abi_version() == abi.NT_ABI_VERSION
    assert lib.nt_status_string(abi.NT_ERR_WORKSPACE) == b"workspace too small"


def _state():
    from helpers import make_state
    return make_state("c2", image=64, region=(32, 16))


def test_argument_errors_enqueue_nothing(lib):
    st = _state()
    p = st.params()
    assert lib.nt_train_step(None, 0, None) == abi.NT_ERR_NULL_POINTER
    assert lib.nt_train_step(C.byref(p), 7, None) == abi.NT_ERR_INVALID_ARGUMENT
    bad = st.params()
    bad.mlp.sizes[1] = 48
    assert lib.nt_train_step(C.byref(bad), 0, None) == abi.NT_ERR_UNSUPPORTED
    assert b"no kernel is built" in lib.nt_last_error()
    bad = st.params()
    bad.latents.channels = 8
    assert lib.nt_train_step(C.byref(bad), 0, None) == abi.NT_ERR_UNSUPPORTED
    bad = st.params()
    bad.latents.grids[0].values = None
    assert lib.nt_train_step(C.byref(bad), 0, None) == abi.NT_ERR_NULL_POINTER
    bad = st.params()
    bad.num_samples = 0
    assert lib.nt_train_step(C.byref(bad), 0, None) == abi.NT_ERR_INVALID_ARGUMENT
    need = lib.nt_train_workspace_bytes(C.byref(p), 0)
    assert need > 0
    assert lib.nt_train_step(C.byref(p), 0, None) == abi.NT_ERR_WORKSPACE
    ws = np.zeros(need // 4 + 8, np.float32)
    small = st.params()
    small.workspace, small.workspace_bytes = C.c_void_p(ws.ctypes.data), need - 4
    assert lib.nt_train_step(C.byref(small), 0, None) == abi.NT_ERR_WORKSPACE
    misaligned = st.params()
    misaligned.latents.grids[0].values = C.cast(st.grids[0].values.ctypes.data + 4, abi.f32p)
    assert lib.nt_train_step(C.byref(misaligned), 0, None) == abi.NT_ERR_MISALIGNED
    assert lib.nt_optimize_latents(C.byref(p), 9, None) == abi.NT_ERR_INVALID_ARGUMENT
    bad = st.params()
    bad.mlp.weight_moment1[0] = None
    assert lib.nt_optimize_network(C.byref(bad), None) == abi.NT_ERR_NULL_POINTER
    assert lib.nt_inference(C.byref(p), None) == abi.NT_ERR_NULL_POINTER  # no output buffers
    assert lib.nt_codec_encode(None, 4, 4, 16, None, None) == abi.NT_ERR_NULL_POINTER
    buf = np.zeros(64, np.float32)
    assert lib.nt_codec_encode(buf.ctypes.data, 4, 4, 3, buf.ctypes.data, None) == abi.NT_ERR_INVALID_ARGUMENT
    assert lib.nt_mlp_forward(None, None, None, 1, None) == abi.NT_ERR_NULL_POINTER
    assert lib.nt_bc6_init(None, None) == abi.NT_ERR_NULL_POINTER
    lat = st.params().latents  # no block_params
    assert lib.nt_bc6_init(C.byref(lat), None) == abi.NT_ERR_NULL_POINTER
    lat.channels = 5
    assert lib.nt_bc6_init(C.byref(lat), None) == abi.NT_ERR_UNSUPPORTED
    lat = st.params().latents
    lat.grids[0].width = 6
    assert lib.nt_bc6_init(C.byref(lat), None) == abi.NT_ERR_INVALID_ARGUMENT
    with pytest.raises(nt.NtError) as e:
        nt.check(lib.nt_decode(None, None))
    assert e.value.status == abi.NT_ERR_NULL_POINTER


@pytest.mark.parametrize("margins", [None, "0"])
@pytest.mark.parametrize("shape,ng", [("c2", 2), ("c4", 1)])
def test_config_shapes_plan_the_16_channel_kernel(lib, shape, ng, margins):
    """The BASELINE config 2 / 4 shapes (grid-to-image ratios, textures, MLP) must be planned
    on the 16-channel train kernel: its LDS layout has to fit. That plan's workspace is
    exactly one gradient partial row per 64 x 8*groups tile (no prepared weight image), which
    tells it apart from the generic kernel's."""
    from helpers import make_state
    assert lib.nt_set_test_hooks(0, 1 if margins else 0) == 0
    try:
        st = make_state(shape, image=256, region=(64, 64))
        p = st.params()
        sizes = list(st.net.sizes)
        pads = [abi.pad16(s) for s in sizes]
        P_total = sum(pads[l + 1] * pads[l] + pads[l + 1] for l in range(len(sizes) - 1))
        tiles = (64 // 64) * (64 // (8 * ng))
        assert lib.nt_train_workspace_bytes(C.byref(p), 0) == tiles * P_total * 4
    finally:
        assert lib.nt_set_test_hooks(0, 0) == 0


def test_random_sample_order_refusals(lib):
    """nt_random_sample_order refuses, before touching a device, parameters that train in
    slot order (random texels below the sort's sample count without the hook, region
    samples) and a null order buffer."""
    from helpers import make_state
    st = make_state("c2", image=256, region=(64, 64))
    st.sample_mode = abi.NT_SAMPLES_RANDOM
    p = st.params()
    order = np.zeros(64 * 64, np.uint32)
    assert lib.nt_random_sample_order(C.byref(p), C.c_void_p(order.ctypes.data), None) == abi.NT_ERR_UNSUPPORTED
    assert b"slot order" in lib.nt_last_error()
    region = make_state("c2", image=256, region=(64, 64)).params()
    assert lib.nt_set_test_hooks(0, abi.NT_HOOK_SORT_RANDOM) == 0
    try:
        assert lib.nt_random_sample_order(C.byref(region), C.c_void_p(order.ctypes.data), None) == abi.NT_ERR_UNSUPPORTED
        assert lib.nt_random_sample_order(C.byref(p), None, None) == abi.NT_ERR_NULL_POINTER
        assert lib.nt_random_sample_order(C.byref(p), C.c_void_p(order.ctypes.data), None) == abi.NT_ERR_WORKSPACE
    finally:
        assert lib.nt_set_test_hooks(0, 0) == 0
