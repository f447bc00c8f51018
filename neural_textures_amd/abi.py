"""ctypes mirror of include/nt/nt.h (structs, constants and function signatures).

The same structs describe device buffers for the HIP library and host buffers for the CPU
oracle used by the tests, so both are driven by one parameter block.
"""
from __future__ import annotations

import ctypes as C

NT_ABI_VERSION = 2
NT_MAX_GRIDS = 4
NT_MAX_MIPS = 16
NT_MAX_LAYERS = 6
NT_MAX_TEXTURES = 16
NT_MAX_OUTPUTS = 16
NT_DEFAULT_REGION = 512

NT_OK = 0
NT_ERR_INVALID_ARGUMENT = 1
NT_ERR_NULL_POINTER = 2
NT_ERR_MISALIGNED = 3
NT_ERR_UNSUPPORTED = 4
NT_ERR_WORKSPACE = 5
NT_ERR_HIP = 6
NT_ERR_FORMAT = 7

# model container
NT_MODEL_VERSION = 1
NT_MODEL_CODEC = 1
NT_MODEL_STATE = 2
NT_MODEL_BLOCKS = 4

# nt_kernel_type (TrainingKernelType, train.h:22-27)
NT_UNCONSTRAINED = 0
NT_BLOCK_FEATURES = 1
NT_FINALIZE = 2

# nt_sample_mode
NT_SAMPLES_REGION = 0
NT_SAMPLES_RANDOM = 1
NT_LATENT_DENSE = 0
NT_LATENT_TOUCHED = 1

# nt_filter
NT_FILTER_BILINEAR = 0
NT_FILTER_CATMULL_ROM = 1

# nt_set_test_hooks flags
NT_HOOK_DROP_MARGINS = 1
NT_HOOK_SORT_RANDOM = 2

f32p = C.POINTER(C.c_float)
u16p = C.POINTER(C.c_uint16)


class nt_adam(C.Structure):
    _fields_ = [("beta1", C.c_float), ("beta2", C.c_float), ("learning_rate", C.c_float),
                ("epsilon", C.c_float)]


class nt_grid(C.Structure):
    _fields_ = [
        ("width", C.c_int), ("height", C.c_int), ("num_mips", C.c_int), ("reserved0", C.c_int),
        ("mip_offset", C.c_int64 * NT_MAX_MIPS),
        ("values", f32p), ("grads", f32p), ("moment1", f32p), ("moment2", f32p),
        ("block_offset", C.c_int64 * NT_MAX_MIPS),
        ("block_params", f32p), ("block_grads", f32p), ("block_moment1", f32p),
        ("block_moment2", f32p),
    ]


class nt_latents(C.Structure):
    _fields_ = [("num_grids", C.c_int), ("channels", C.c_int), ("grids", nt_grid * NT_MAX_GRIDS)]


class nt_mlp(C.Structure):
    _fields_ = [
        ("num_layers", C.c_int),
        ("sizes", C.c_int * (NT_MAX_LAYERS + 1)),
        ("used_outputs", C.c_int),
        ("weights", u16p * NT_MAX_LAYERS),
        ("weight_grads", f32p * NT_MAX_LAYERS),
        ("weight_moment1", f32p * NT_MAX_LAYERS),
        ("weight_moment2", f32p * NT_MAX_LAYERS),
        ("biases", u16p * NT_MAX_LAYERS),
        ("bias_grads", f32p * NT_MAX_LAYERS),
        ("bias_moment1", f32p * NT_MAX_LAYERS),
        ("bias_moment2", f32p * NT_MAX_LAYERS),
    ]


class nt_texture(C.Structure):
    _fields_ = [
        ("texels", f32p), ("width", C.c_int), ("height", C.c_int), ("num_channels", C.c_int),
        ("num_mips", C.c_int), ("pitch", C.c_int), ("loss_weight", C.c_float),
        ("mip_offset", C.c_int64 * NT_MAX_MIPS),
    ]


class nt_params(C.Structure):
    _fields_ = [
        ("latents", nt_latents),
        ("mlp", nt_mlp),
        ("network_adam", nt_adam),
        ("feature_adam", nt_adam),
        ("textures", nt_texture * NT_MAX_TEXTURES),
        ("num_textures", C.c_int),
        ("image_width", C.c_int), ("image_height", C.c_int),
        ("texel_offset_x", C.c_int), ("texel_offset_y", C.c_int),
        ("region_width", C.c_int), ("num_samples", C.c_int), ("step", C.c_int),
        ("sample_mode", C.c_int), ("sample_mip", C.c_float), ("latent_update", C.c_int),
        ("inference_output", f32p), ("inference_mse_accum", f32p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class nt_codec_grid(C.Structure):
    _fields_ = [
        ("width", C.c_int), ("height", C.c_int), ("num_mips", C.c_int), ("reserved0", C.c_int),
        ("byte_offset", C.c_int64 * NT_MAX_MIPS), ("blocks", C.c_void_p),
    ]


class nt_decode_params(C.Structure):
    _fields_ = [
        ("num_grids", C.c_int), ("channels", C.c_int),
        ("grids", nt_codec_grid * NT_MAX_GRIDS),
        ("mlp", nt_mlp),
        ("out_width", C.c_int), ("out_height", C.c_int),
        ("seed", C.c_uint32), ("jitter", C.c_float), ("mip_min", C.c_float), ("mip_max", C.c_float),
        ("output", u16p),
        ("workspace", C.c_void_p), ("workspace_bytes", C.c_size_t),
    ]


class nt_model_info(C.Structure):
    _fields_ = [
        ("contents", C.c_uint32), ("num_grids", C.c_int), ("channels", C.c_int),
        ("width", C.c_int * NT_MAX_GRIDS), ("height", C.c_int * NT_MAX_GRIDS),
        ("num_mips", C.c_int * NT_MAX_GRIDS),
        ("num_layers", C.c_int), ("sizes", C.c_int * (NT_MAX_LAYERS + 1)),
        ("used_outputs", C.c_int), ("step", C.c_int),
    ]


class nt_model_data(C.Structure):
    _fields_ = [
        ("codec", C.c_void_p * NT_MAX_GRIDS),
        ("weights", C.c_void_p * NT_MAX_LAYERS), ("biases", C.c_void_p * NT_MAX_LAYERS),
        ("latents", C.c_void_p * NT_MAX_GRIDS),
        ("latent_moment1", C.c_void_p * NT_MAX_GRIDS),
        ("latent_moment2", C.c_void_p * NT_MAX_GRIDS),
        ("weight_moment1", C.c_void_p * NT_MAX_LAYERS),
        ("weight_moment2", C.c_void_p * NT_MAX_LAYERS),
        ("bias_moment1", C.c_void_p * NT_MAX_LAYERS),
        ("bias_moment2", C.c_void_p * NT_MAX_LAYERS),
        ("block_params", C.c_void_p * NT_MAX_GRIDS),
        ("block_moment1", C.c_void_p * NT_MAX_GRIDS),
        ("block_moment2", C.c_void_p * NT_MAX_GRIDS),
    ]


# Entry points of include/nt/nt.h: name -> (restype, argtypes)
P = C.POINTER
SIGNATURES = {
    "nt_abi_version": (C.c_int, []),
    "nt_status_string": (C.c_char_p, [C.c_int]),
    "nt_last_error": (C.c_char_p, []),
    "nt_mip_chain_layout": (C.c_int64, [C.c_int, C.c_int, C.c_int, P(C.c_int64)]),
    "nt_block_chain_layout": (C.c_int64, [C.c_int, C.c_int, C.c_int, P(C.c_int64)]),
    "nt_profile_next_launch": (C.c_int, [C.c_void_p, C.c_void_p]),
    "nt_set_test_hooks": (C.c_int, [C.c_int, C.c_int]),
    "nt_random_sample_order": (C.c_int, [P(nt_params), C.c_void_p, C.c_void_p]),
    "nt_train_workspace_bytes": (C.c_size_t, [P(nt_params), C.c_int]),
    "nt_train_step": (C.c_int, [P(nt_params), C.c_int, C.c_void_p]),
    "nt_train_step_static": (C.c_int, [P(nt_params), C.c_int, C.c_void_p]),
    "nt_train_static_scratch_bytes": (C.c_size_t, []),
    "nt_optimize_network": (C.c_int, [P(nt_params), C.c_void_p]),
    "nt_optimize_latents": (C.c_int, [P(nt_params), C.c_int, C.c_void_p]),
    "nt_train_iteration": (C.c_int, [P(nt_params), C.c_int, C.c_void_p]),
    "nt_inference": (C.c_int, [P(nt_params), C.c_void_p]),
    "nt_inference_workspace_bytes": (C.c_size_t, [P(nt_params)]),
    "nt_mlp_forward": (C.c_int, [P(nt_mlp), C.c_void_p, C.c_void_p, C.c_int, C.c_void_p]),
    "nt_forward": (C.c_int, [P(nt_latents), P(nt_mlp), C.c_int, C.c_void_p, C.c_int, C.c_void_p,
                             C.c_void_p, C.c_void_p]),
    "nt_bc6_init": (C.c_int, [P(nt_latents), C.c_void_p]),
    "nt_codec_block_bytes": (C.c_size_t, [C.c_int]),
    "nt_codec_mip_chain_layout": (C.c_size_t, [C.c_int, C.c_int, C.c_int, C.c_int, P(C.c_int64)]),
    "nt_codec_encode": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "nt_codec_decode": (C.c_int, [C.c_void_p, C.c_int, C.c_int, C.c_int, C.c_void_p, C.c_void_p]),
    "nt_decode_workspace_bytes": (C.c_size_t, [P(nt_decode_params)]),
    "nt_decode": (C.c_int, [P(nt_decode_params), C.c_void_p]),
    "nt_model_bytes": (C.c_size_t, [P(nt_model_info)]),
    "nt_model_save": (C.c_int, [P(nt_model_info), P(nt_model_data), C.c_void_p, C.c_size_t]),
    "nt_model_load": (C.c_int, [C.c_void_p, C.c_size_t, P(nt_model_info), P(nt_model_data)]),
}


def bind(lib: C.CDLL, signatures: dict = SIGNATURES) -> C.CDLL:
    for name, (res, args) in signatures.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def pad16(x: int) -> int:
    return (x + 15) & ~15
