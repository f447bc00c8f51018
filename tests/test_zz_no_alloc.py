"""nt_train_step_static: the train step with its scratch in the library's static device array
instead of a caller workspace. Two calls in a row (the second on a smaller region) must give
what nt_train_step gives with a workspace: the MLP gradients bit for bit (both reduce the
per-workgroup partial rows in the same fixed order), the latent gradients within 1e-5
relative (float atomics add in arrival order). A step whose scratch would exceed the array is
refused before anything is enqueued.
"""
import ctypes as C

import numpy as np
import pytest

import neural_textures_amd as nt
from neural_textures_amd import abi
from helpers import make_state, rel_err, to_np, gpu_workspace

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    import torch
    assert torch.cuda.is_available()
    return nt.load()


def say(msg):
    print(msg, flush=True)


def _grads(s):
    return ([to_np(a).copy() for a in s.net.weight_grads], [to_np(a).copy() for a in s.net.bias_grads],
            [to_np(g.grads).copy() for g in s.grids])


def _zero(s):
    for a in (*s.net.weight_grads, *s.net.bias_grads, *(g.grads for g in s.grids)):
        a.zero_()


@pytest.mark.parametrize("shape", ["c4", "c2", "ref", "ref16f", "c2-random-sorted"])
def test_static_scratch_matches_workspace_step(lib, shape):
    """c2-random-sorted: random texels in bin order (the sort's buffers in the static array
    too): both entry points read the samples in the same order."""
    import torch
    assert lib.nt_train_static_scratch_bytes() == 32 << 20
    sorted_random = shape.endswith("-random-sorted")
    st = make_state(shape.split("-")[0], image=256, region=(128, 64), seed=3, offset=(40, 17), step=5)
    if sorted_random:
        st.sample_mode = abi.NT_SAMPLES_RANDOM
    nt.check(lib.nt_set_test_hooks(0, abi.NT_HOOK_SORT_RANDOM if sorted_random else 0))
    try:
        _static_matches_workspace(lib, shape, st)
    finally:
        nt.check(lib.nt_set_test_hooks(0, 0))


def _static_matches_workspace(lib, shape, st):
    import torch
    with_ws = gpu_workspace(lib, st.to_torch(), abi.NT_UNCONSTRAINED)
    static = st.to_torch()  # no workspace
    for region, offset in (((128, 64), (40, 17)), ((64, 16), (9, 201))):  # the second is smaller
        say(f"case: {shape} static scratch, region {region} at {offset}")
        for s in (with_ws, static):
            s.region_width, s.num_samples = region[0], region[0] * region[1]
            s.texel_offset_x, s.texel_offset_y = offset
            _zero(s)
        nt.check(lib.nt_train_step(C.byref(with_ws.params()), abi.NT_UNCONSTRAINED, None))
        nt.check(lib.nt_train_step_static(C.byref(static.params()), abi.NT_UNCONSTRAINED, None))
        torch.cuda.synchronize()
        (wa, ba, la), (wb, bb, lb) = _grads(with_ws), _grads(static)
        for l in range(len(wa)):
            assert np.array_equal(wa[l].view(np.uint32), wb[l].view(np.uint32)), f"dW{l}"
            assert np.array_equal(ba[l].view(np.uint32), bb[l].view(np.uint32)), f"db{l}"
            assert np.any(wa[l] != 0)
        for gi in range(len(la)):
            assert rel_err(lb[gi], la[gi]) <= 1e-5, f"latent grad {gi}"
            assert np.array_equal(la[gi] == 0, lb[gi] == 0)


def test_static_scratch_refuses_oversized_steps(lib):
    """The reference network on the general kernel writes one gradient row per 64 x 8 tile:
    about two million samples need more than the 32 MiB array."""
    st = make_state("ref", image=256, region=(64, 32))
    st.region_width, st.num_samples = 512, 512 * 4096
    p = st.params()
    need = lib.nt_train_workspace_bytes(C.byref(p), abi.NT_UNCONSTRAINED)
    assert need > lib.nt_train_static_scratch_bytes()
    assert lib.nt_train_step_static(C.byref(p), abi.NT_UNCONSTRAINED, None) == abi.NT_ERR_WORKSPACE
    assert b"static scratch" in lib.nt_last_error()
