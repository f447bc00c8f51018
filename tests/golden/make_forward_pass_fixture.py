"""Writes tests/golden/forward_pass_test.json: the known-answer vectors of the reference's only
unit test (mavenkim2/neural_textures tests/forward_pass_test.cu).

Inputs, weights and biases are the test's closed-form values rounded to fp16
(forward_pass_test.cu:45-108); the expected outputs follow its CPU reference procedure
(:110-150): fp32 sums in input order over the fp16-rounded values, fp32 ReLU hidden layer,
no output activation. Pass criterion there: |gpu - expected| <= 2e-2 (:236).

Run: python tests/golden/make_forward_pass_fixture.py
"""
import json
import os

import numpy as np

WARP = 32     # rows (lanes) in the reference test
INPUT = 12    # NT_INPUT_SIZE
HIDDEN = 16   # NT_HIDDEN_LAYER_SIZE
OUTPUT = 16   # NT_OUTPUT_SIZE


def h(x):
    return np.float16(np.float32(x))


def main():
    inputs = np.zeros((WARP, INPUT), np.float16)
    for lane in range(WARP):
        for k in range(INPUT):
            inputs[lane, k] = h(0.125 + 0.01171875 * (lane + 1) + 0.0068359375 * (k + 1))
    w0 = np.zeros((HIDDEN, HIDDEN), np.float16)  # [out][in] == column-major in*1 + out*16
    w1 = np.zeros((HIDDEN, HIDDEN), np.float16)
    for o in range(HIDDEN):
        for i in range(HIDDEN):
            if i < INPUT:
                w0[o, i] = h(0.0625 + 0.0048828125 * ((3 * o + 1) % 7) + 0.0029296875 * ((5 * i + 2) % 11))
            if o < OUTPUT:
                w1[o, i] = h(0.09375 + 0.00341796875 * ((7 * o + 3) % 13) + 0.001953125 * ((2 * i + 5) % 9))
    b0 = np.array([h(0.046875 + 0.00390625 * ((4 * o + 1) % 9)) for o in range(HIDDEN)], np.float16)
    b1 = np.array([h(0.078125 + 0.005859375 * ((5 * o + 2) % 7)) if o < OUTPUT else h(0)
                   for o in range(HIDDEN)], np.float16)

    expected = np.zeros((WARP, OUTPUT), np.float32)
    for lane in range(WARP):
        hidden = np.zeros(HIDDEN, np.float32)
        for o in range(HIDDEN):
            s = np.float32(b0[o])
            for i in range(HIDDEN):
                x = np.float32(inputs[lane, i]) if i < INPUT else np.float32(0)
                s = np.float32(s + np.float32(x * np.float32(w0[o, i])))
            hidden[o] = max(s, np.float32(0))
        for o in range(OUTPUT):
            s = np.float32(b1[o])
            for i in range(HIDDEN):
                s = np.float32(s + np.float32(hidden[i] * np.float32(w1[o, i])))
            expected[lane, o] = s

    out = {
        "source": "mavenkim2/neural_textures tests/forward_pass_test.cu:45-150",
        "tolerance_abs": 2e-2,
        "sizes": [INPUT, HIDDEN, OUTPUT],
        "inputs_f16_bits": inputs.view(np.uint16).reshape(-1).tolist(),
        "w0_f16_bits": w0.view(np.uint16).reshape(-1).tolist(),
        "w1_f16_bits": w1.view(np.uint16).reshape(-1).tolist(),
        "b0_f16_bits": b0.view(np.uint16).tolist(),
        "b1_f16_bits": b1.view(np.uint16).tolist(),
        "expected": expected.reshape(-1).tolist(),
    }
    path = os.path.join(os.path.dirname(os.path.abspath(__file__)), "forward_pass_test.json")
    with open(path, "w") as f:
        json.dump(out, f)
    print(f"wrote {path}")


if __name__ == "__main__":
    main()
