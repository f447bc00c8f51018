"""Loads the CPU oracle (oracle/libnt_oracle.so): test infrastructure only."""
import ctypes as C
import os
import subprocess

from neural_textures_amd import abi

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_DIR = os.path.join(ROOT, "oracle")
ORACLE_PATH = os.path.join(ORACLE_DIR, "libnt_oracle.so")

P = C.POINTER
f3 = C.c_float * 3
SIGNATURES = {
    "ntref_f32_to_f16": (C.c_uint16, [C.c_float]),
    "ntref_f16_to_f32": (C.c_float, [C.c_uint16]),
    "ntref_f16_add": (C.c_uint16, [C.c_uint16, C.c_uint16]),
    "ntref_xorshift32": (C.c_uint32, [P(C.c_uint32)]),
    "ntref_uniform": (C.c_float, [P(C.c_uint32)]),
    "ntref_sample_seed": (C.c_uint32, [C.c_uint32, C.c_int]),
    "ntref_fmix32": (C.c_uint32, [C.c_uint32]),
    "ntref_sample_uvz": (None, [P(abi.nt_params), C.c_uint32, P(C.c_float)]),
    "ntref_sample_latents_bilinear": (None, [P(abi.nt_latents), P(C.c_float), P(C.c_uint16)]),
    "ntref_sample_latents_catmull_rom": (None, [P(abi.nt_latents), P(C.c_float), P(C.c_uint16)]),
    "ntref_sample_latents_bc6": (None, [P(abi.nt_latents), P(C.c_float), P(C.c_uint16)]),
    "ntref_scatter_unconstrained": (None, [P(abi.nt_latents), P(C.c_float), P(C.c_uint16)]),
    "ntref_scatter_bc6": (None, [P(abi.nt_latents), P(C.c_float), P(C.c_uint16)]),
    "ntref_catmull_rom_weights": (None, [C.c_float, P(C.c_float)]),
    "ntref_sample_texture": (None, [P(abi.nt_texture), C.c_float, C.c_float, C.c_float, P(C.c_float)]),
    "ntref_expected_values": (C.c_int, [P(abi.nt_params), P(C.c_float), P(C.c_float), P(C.c_float)]),
    "ntref_bc6_unquantize": (C.c_float, [C.c_float, C.c_int]),
    "ntref_bc6_decompress": (C.c_float, [C.c_float, C.c_float, C.c_int, C.c_float]),
    "ntref_mlp_forward_one": (None, [P(abi.nt_mlp), P(C.c_uint16), P(C.c_uint16), P(C.c_uint16)]),
    "ntref_mlp_backward_one": (None, [P(abi.nt_mlp), P(C.c_uint16), P(C.c_uint16),
                                      P(P(C.c_double)), P(P(C.c_double)), P(C.c_uint16)]),
    "ntref_train_step": (C.c_int, [P(abi.nt_params), C.c_int, C.c_int]),
    "ntref_optimize_network": (C.c_int, [P(abi.nt_params)]),
    "ntref_optimize_latents": (C.c_int, [P(abi.nt_params), C.c_int]),
    "ntref_inference": (C.c_int, [P(abi.nt_params)]),
    "ntref_mlp_forward": (C.c_int, [P(abi.nt_mlp), C.c_void_p, C.c_void_p, C.c_int]),
    "ntref_forward": (C.c_int, [P(abi.nt_latents), P(abi.nt_mlp), C.c_int, C.c_void_p, C.c_int,
                                C.c_void_p, C.c_void_p]),
    "ntref_train_intermediates": (C.c_int, [P(abi.nt_params), C.c_int, C.c_void_p, C.c_void_p,
                                            C.c_void_p]),
    "ntref_codec_key": (C.c_uint16, [C.c_uint16]),
    "ntref_codec_unkey": (C.c_uint16, [C.c_uint16]),
    "ntref_codec_interp": (C.c_uint16, [C.c_uint16, C.c_uint16, C.c_int]),
    "ntref_codec_encode": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "ntref_codec_decode": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p]),
    "ntref_decode": (C.c_int, [P(abi.nt_decode_params), C.c_int]),
    "ntref_decode_rect": (C.c_int, [P(abi.nt_decode_params), C.c_int, C.c_int, C.c_int, C.c_int, C.c_int]),
    "ntref_set_threads": (None, [C.c_int]),
    "ntref_set_dw_partial_fp16": (None, [C.c_int]),
    "ntref_set_mlp_accum_f32": (None, [C.c_int]),
    "ntref_bc6_value_to_y": (C.c_float, [C.c_float]),
    "ntref_bc6_fit_subset": (C.c_float, [C.c_void_p, C.c_void_p, C.c_int, C.c_int, C.c_int,
                                         C.c_void_p, C.c_void_p, C.c_void_p]),
    "ntref_bc6_init_block": (None, [C.c_void_p, C.c_int, C.c_int, C.c_void_p]),
    "ntref_bc6_init": (C.c_int, [P(abi.nt_latents)]),
}

_oracle = None


def load_oracle():
    global _oracle
    if _oracle is None:
        if not os.path.exists(ORACLE_PATH):
            subprocess.run(["make", "-C", ORACLE_DIR], check=True, capture_output=True)
        _oracle = abi.bind(C.CDLL(ORACLE_PATH), SIGNATURES)
    return _oracle
