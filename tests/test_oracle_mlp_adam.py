"""Pins the oracle's MLP forward/backward, loss gradient and lazy Adam.

Forward: the reference's own known-answer test (tests/forward_pass_test.cu, committed as
tests/golden/forward_pass_test.json) and a float64 GEMM. Backward: float64 finite
differences of a scalar loss. Adam: the closed form at t = 1 and the lazy-update rules.
"""
import ctypes as C
import json
import os

import numpy as np

from neural_textures_amd import abi, params as P
from oracle_lib import load_oracle

O = load_oracle()
GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "forward_pass_test.json")


def fixture_network():
    d = json.load(open(GOLDEN))
    net = P.Network([12, 16, 16], 16)
    net.weights = [np.array(d["w0_f16_bits"], np.uint16), np.array(d["w1_f16_bits"], np.uint16)]
    net.biases = [np.array(d["b0_f16_bits"], np.uint16), np.array(d["b1_f16_bits"], np.uint16)]
    inputs = np.array(d["inputs_f16_bits"], np.uint16)
    expected = np.array(d["expected"], np.float32).reshape(32, 16)
    return net, inputs, expected, d["tolerance_abs"]


def oracle_mlp_forward(net, inputs, count):
    out = np.zeros(count * net.sizes[-1], np.uint16)
    m = net.struct()
    assert O.ntref_mlp_forward(C.byref(m), inputs.ctypes.data, out.ctypes.data, count) == 0
    return out.view(np.float16).astype(np.float32).reshape(count, net.sizes[-1])


def test_forward_pass_known_answer():
    """tests/forward_pass_test.cu:236: |out - expected| <= 2e-2 for all 32 x 16 outputs."""
    net, inputs, expected, tol = fixture_network()
    got = oracle_mlp_forward(net, inputs, 32)
    assert np.max(np.abs(got - expected)) <= tol
    assert np.max(np.abs(got - expected)) <= 2e-3  # fp16 hidden + output rounding only


def _forward64(net, x):
    """float64 GEMM chain with the oracle's rounding points (fp16 layer outputs)."""
    h = x.astype(np.float64)
    L = net.num_layers
    for l in range(L):
        pin, pout = net.padded(l)
        W = net.weight_matrix(l).astype(np.float64)  # [pout, pin]
        b = np.zeros(pout)
        b[:net.sizes[l + 1]] = net.biases[l].view(np.float16).astype(np.float64)
        hp = np.zeros((h.shape[0], pin))
        hp[:, :h.shape[1]] = h
        y = hp @ W.T + b
        if l < L - 1:
            y = np.maximum(y, 0)
        h = y.astype(np.float32).astype(np.float16).astype(np.float64)
    return h


def test_forward_matches_float64_gemm():
    rng = np.random.default_rng(10)
    for sizes in ([12, 32, 32, 16], [32, 64, 64, 9], [64, 64, 64, 64, 12], [8, 64, 64, 3]):
        net = P.make_network(sizes, rng=rng, init="xavier")
        for l in range(net.num_layers):
            net.biases[l] = P.f16_bits(rng.uniform(-0.1, 0.1, sizes[l + 1]))
        x = rng.uniform(-1, 1, size=(64, sizes[0])).astype(np.float16)
        got = oracle_mlp_forward(net, x.view(np.uint16).copy(), 64)
        want = _forward64(net, x)[:, :sizes[-1]]
        # same rounding points; only the summation order can flip an fp16 rounding
        assert np.max(np.abs(got - want) / (np.abs(want) + 1e-3)) < 2e-3


def _backward_oracle(net, x16, dy16):
    """One-sample backward through the oracle; returns dW list, db list, dinput."""
    L = net.num_layers
    m = net.struct()
    acts = np.zeros(abi.NT_MAX_LAYERS * 64, np.uint16)
    out = np.zeros(16, np.uint16)
    O.ntref_mlp_forward_one(C.byref(m), x16.ctypes.data_as(C.POINTER(C.c_uint16)),
                            acts.ctypes.data_as(C.POINTER(C.c_uint16)),
                            out.ctypes.data_as(C.POINTER(C.c_uint16)))
    dws = [np.zeros(net.padded(l)[0] * net.padded(l)[1]) for l in range(L)]
    dbs = [np.zeros(net.padded(l)[1]) for l in range(L)]
    dwp = (C.POINTER(C.c_double) * L)(*[a.ctypes.data_as(C.POINTER(C.c_double)) for a in dws])
    dbp = (C.POINTER(C.c_double) * L)(*[a.ctypes.data_as(C.POINTER(C.c_double)) for a in dbs])
    din = np.zeros(64, np.uint16)
    dyp = np.zeros(16, np.uint16)
    dyp[:len(dy16)] = dy16
    O.ntref_mlp_backward_one(C.byref(m), acts.ctypes.data_as(C.POINTER(C.c_uint16)),
                             dyp.ctypes.data_as(C.POINTER(C.c_uint16)), dwp, dbp,
                             din.ctypes.data_as(C.POINTER(C.c_uint16)))
    return dws, dbs, din[:net.sizes[0]].view(np.float16).astype(np.float64)


def test_backward_matches_finite_differences():
    """Gradients of L = <dy, f(x)> in float64 (no fp16 rounding) vs the oracle's backward,
    which rounds activations and gradients to fp16 as the reference does (mlp.h:222-362)."""
    rng = np.random.default_rng(11)
    sizes = [12, 32, 32, 16]
    net = P.make_network(sizes, rng=rng, init="xavier")
    for l in range(net.num_layers):
        net.biases[l] = P.f16_bits(rng.uniform(0.05, 0.2, sizes[l + 1]))
    x = rng.uniform(-1, 1, sizes[0]).astype(np.float16)
    dy = rng.uniform(-1, 1, 16).astype(np.float16)
    dws, dbs, din = _backward_oracle(net, x.view(np.uint16).copy(), dy.view(np.uint16))

    Ws = [net.weight_matrix(l).astype(np.float64) for l in range(net.num_layers)]
    bs = []
    for l in range(net.num_layers):
        b = np.zeros(net.padded(l)[1])
        b[:sizes[l + 1]] = net.biases[l].view(np.float16).astype(np.float64)
        bs.append(b)

    def loss(Ws, bs, xin):
        h = np.zeros(16)
        h[:12] = xin
        for l in range(net.num_layers):
            y = Ws[l] @ h + bs[l]
            h = np.maximum(y, 0) if l < net.num_layers - 1 else y
        return float(np.dot(h[:16], dy.astype(np.float64)))

    eps = 1e-6
    # input gradient
    fd = np.array([(loss(Ws, bs, x.astype(np.float64) + eps * np.eye(12)[i]) -
                    loss(Ws, bs, x.astype(np.float64) - eps * np.eye(12)[i])) / (2 * eps) for i in range(12)])
    assert np.linalg.norm(din - fd) <= 1e-2 * np.linalg.norm(fd)
    # weight and bias gradients of every layer
    for l in range(net.num_layers):
        pin, pout = net.padded(l)
        g = np.zeros((pout, pin))
        for n in range(pout):
            for k in range(min(pin, sizes[l])):
                Wp = [w.copy() for w in Ws]
                Wm = [w.copy() for w in Ws]
                Wp[l][n, k] += eps
                Wm[l][n, k] -= eps
                g[n, k] = (loss(Wp, bs, x.astype(np.float64)) - loss(Wm, bs, x.astype(np.float64))) / (2 * eps)
        got = dws[l].reshape(pout, pin)
        assert np.linalg.norm(got - g) <= 1e-2 * np.linalg.norm(g), l
        gb = np.zeros(pout)
        for n in range(sizes[l + 1]):
            bp = [b.copy() for b in bs]
            bm = [b.copy() for b in bs]
            bp[l][n] += eps
            bm[l][n] -= eps
            gb[n] = (loss(Ws, bp, x.astype(np.float64)) - loss(Ws, bm, x.astype(np.float64))) / (2 * eps)
        assert np.linalg.norm(dbs[l] - gb) <= 1e-2 * np.linalg.norm(gb), l


def test_weight_gradient_is_outer_product_and_padding_stays_zero():
    rng = np.random.default_rng(12)
    net = P.make_network([12, 32, 32, 16], rng=rng, init="xavier")
    x = rng.uniform(-1, 1, 12).astype(np.float16)
    dy = rng.uniform(-1, 1, 16).astype(np.float16)
    dws, dbs, _ = _backward_oracle(net, x.view(np.uint16).copy(), dy.view(np.uint16))
    dw0 = dws[-1].reshape(16, 32)  # last layer: dW = dy x h^T
    assert np.allclose(dbs[-1], dy.astype(np.float64))
    # rows of the input-padding columns of layer 0 (inputs 12..15 are zero) stay zero
    assert np.all(dws[0].reshape(32, 16)[:, 12:] == 0)
    assert np.all(np.isfinite(dw0))


def _one_layer_state(num_samples, seed):
    import sys
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    from helpers import make_state
    st = make_state("c2", image=64, region=(16, (num_samples + 15) // 16), offset=(9, 21), seed=seed)
    st.num_samples = num_samples
    # one layer 32 -> 9: its input is the sampled features, so the weight gradient is the
    # outer product of quantities ntref_train_intermediates returns
    st.net = P.make_network([32, 9], used_outputs=9, rng=np.random.default_rng(seed), init="xavier")
    return st


def _dw_from_intermediates(st, fp16_partials):
    """Sum over samples of f (x) dy (fp16 features and loss gradients from the oracle), in
    sample order in float64; with fp16_partials, each run of 32 consecutive samples is summed
    alone and rounded to fp16 (numpy's binary16, nearest-even) before it is added."""
    n = st.num_samples
    f = np.zeros(n * 32, np.uint16)
    dy = np.zeros(n * 16, np.uint16)
    assert O.ntref_train_intermediates(C.byref(st.params()), 0, f.ctypes.data, dy.ctypes.data, None) == 0
    f = f.view(np.float16).astype(np.float64).reshape(n, 32)
    dy = dy.view(np.float16).astype(np.float64).reshape(n, 16)
    total = np.zeros((16, 32))
    for w0 in range(0, n, 32):
        part = np.zeros((16, 32))
        for s in range(w0, min(w0 + 32, n)):
            part += np.outer(dy[s], f[s])
        total += part.astype(np.float16).astype(np.float64) if fp16_partials else part
    return total.astype(np.float32).reshape(-1)


def test_dw_partials_rounded_to_fp16_per_warp():
    """ntref_set_dw_partial_fp16: each 32-sample warp's weight-gradient partial is rounded to
    fp16 before the sum (the reference's __half2 outer-product registers, mlp.h:166-173).
    Pinned on a one-layer network, whose weight gradient is the outer product of the
    features and loss gradients ntref_train_intermediates returns, over 2.5 warps (a ragged
    last warp): bit-exact against the sum restated in numpy in both modes, and the two modes
    differ. Rounding per sample, rounding the total, or another warp size fails it."""
    for fp16 in (0, 1):
        st = _one_layer_state(80, seed=31)
        O.ntref_set_dw_partial_fp16(fp16)
        try:
            assert O.ntref_train_step(C.byref(st.params()), 0, 1) == 0
        finally:
            O.ntref_set_dw_partial_fp16(0)
        want = _dw_from_intermediates(st, bool(fp16))
        assert np.array_equal(st.net.weight_grads[0], want), fp16
        if fp16:
            assert not np.array_equal(want, _dw_from_intermediates(st, False))
        # the bias gradient is the fp32 sum of fp16 dy either way
        assert np.count_nonzero(st.net.bias_grads[0]) > 0


def _forward_f32_sequential(net, x16):
    """The forward of a batch [n, in] with each output's sum accumulated in float32 in input
    order from the bias (fp16 products are exact in float32), ReLU on hidden layers, fp16
    rounding per layer."""
    cur = x16.astype(np.float32)
    L = len(net.sizes) - 1
    for l in range(L):
        pin, pout = abi.pad16(net.sizes[l]), abi.pad16(net.sizes[l + 1])
        W = net.weights[l].view(np.float16).astype(np.float32).reshape(pout, pin)
        b = np.zeros(pout, np.float32)
        b[:net.sizes[l + 1]] = net.biases[l].view(np.float16).astype(np.float32)
        x = np.zeros((cur.shape[0], pin), np.float32)
        x[:, :min(cur.shape[1], pin)] = cur[:, :pin]
        a = np.broadcast_to(b, (cur.shape[0], pout)).astype(np.float32)
        for k in range(pin):  # sequential in k, each step rounded to float32
            a = (a + x[:, k:k + 1] * W[None, :, k]).astype(np.float32)
        if l < L - 1:
            a = np.where(a > 0, a, np.float32(0))
        cur = a.astype(np.float16).astype(np.float32)
    return cur


def test_mlp_accum_f32_switch_is_float32_in_index_order():
    """ntref_set_mlp_accum_f32(1): the forward sums accumulate in float32 in index order
    (bit-exact against a numpy float32 restatement); off, the forward is the float64 one
    (float64 GEMM, rounded once); on this batch the two orders differ on some outputs."""
    rng = np.random.default_rng(21)
    net = P.make_network([64, 64, 64, 64, 16], rng=rng, init="xavier")
    count = 4096
    x = rng.uniform(-1, 1, size=(count, 64)).astype(np.float16)
    O.ntref_set_mlp_accum_f32(1)
    try:
        got = oracle_mlp_forward(net, x.view(np.uint16).copy(), count)
    finally:
        O.ntref_set_mlp_accum_f32(0)
    assert np.array_equal(got, _forward_f32_sequential(net, x)[:, :16])
    off = oracle_mlp_forward(net, x.view(np.uint16).copy(), count)
    assert np.array_equal(off, _forward64(net, x).astype(np.float32)[:, :16])
    assert not np.array_equal(off, got)


# ---- lazy Adam (train.cu:521-816) -----------------------------------------------------

def _adam_state(step, grads_w0):
    rng = np.random.default_rng(13)
    net = P.make_network([12, 32, 32, 16], used_outputs=9, rng=rng, init="xavier")
    g = P.make_grid(8, 8, 2, 3, rng)
    st = P.TrainState([g], net, [], 8, 8, 1, step=step, network_adam=(0.9, 0.999, 1e-2, 1e-8),
                      feature_adam=(0.9, 0.999, 5e-2, 1e-8))
    net.weight_grads[0][:] = grads_w0
    return st


def test_adam_first_step_closed_form_and_lazy_rules():
    rng = np.random.default_rng(14)
    grads = np.zeros(32 * 16, np.float32)
    active = rng.choice(32 * 12, 100, replace=False)
    rows = active % 12
    cols = active // 12
    idx = cols * 16 + rows
    grads[idx] = rng.uniform(-1, 1, 100).astype(np.float32)
    grads[5 * 16 + 13] = 0.7  # a padded row: never updated
    for step in (0, 1):  # t = max(step, 1): both are the first step
        st = _adam_state(step, grads)
        w_before = st.net.weights[0].view(np.float16).astype(np.float64).copy()
        p = st.params()
        assert O.ntref_optimize_network(C.byref(p)) == 0
        w_after = st.net.weights[0].view(np.float16).astype(np.float64)
        g = grads.astype(np.float64)
        want = w_before.copy()
        want[idx] = w_before[idx] - 1e-2 * g[idx] / (np.abs(g[idx]) + 1e-8)
        assert np.allclose(w_after[idx], want[idx], atol=1e-3, rtol=1e-3)  # fp16 weights
        untouched = np.setdiff1d(np.arange(32 * 16), idx)
        assert np.array_equal(w_after[untouched], w_before[untouched])
        assert np.all(st.net.weight_grads[0][idx] == 0)  # consumed gradients are re-zeroed
        assert st.net.weight_grads[0][5 * 16 + 13] == np.float32(0.7)  # padded row untouched
        assert np.all(st.net.weight_moment1[0][untouched] == 0)
        assert np.allclose(st.net.weight_moment1[0][idx], 0.1 * grads[idx], rtol=1e-6)
        assert np.allclose(st.net.weight_moment2[0][idx], 0.001 * grads[idx] ** 2, rtol=1e-5)


def test_adam_latents_two_steps_float64():
    """Two lazy steps on fp32 latents vs a float64 Adam; zero-gradient texels keep moments."""
    rng = np.random.default_rng(15)
    st = _adam_state(1, 0)
    g = st.grids[0]
    v0 = g.values.astype(np.float64).copy()
    m1 = np.zeros_like(v0)
    m2 = np.zeros_like(v0)
    v = v0.copy()
    for step in (1, 2):
        grads = np.where(rng.uniform(size=v.size) < 0.5, rng.uniform(-1, 1, v.size), 0).astype(np.float32)
        g.grads[:] = grads
        st.step = step
        p = st.params()
        assert O.ntref_optimize_latents(C.byref(p), abi.NT_UNCONSTRAINED) == 0
        nz = grads != 0
        gg = grads.astype(np.float64)
        m1[nz] = 0.9 * m1[nz] + 0.1 * gg[nz]
        m2[nz] = 0.999 * m2[nz] + 0.001 * gg[nz] ** 2
        bc1, bc2 = 1 - 0.9 ** step, 1 - 0.999 ** step
        v[nz] -= 5e-2 * (m1[nz] / bc1) / (np.sqrt(m2[nz] / bc2) + 1e-8)
        assert np.allclose(g.values, v, rtol=1e-5, atol=1e-6)
        assert np.allclose(g.moment1, m1, rtol=1e-5, atol=1e-9)
        assert np.all(g.grads == 0)
