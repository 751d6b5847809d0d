"""ctypes binding of libzealot_hip.so (the C ABI declared in include/zealot_hip.h).

The product path is this shared library plus its gfx950 code object; loading
fails loudly when either is missing (there is no CPU fallback).
"""

from __future__ import annotations

import ctypes as C
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(_HERE, "lib")
# ZL_LIBRARY selects another build of the library (e.g. the sanitizer build
# of the host runtime, zealot_amd/lib/asan/libzealot_hip.so).
LIB_PATH = os.environ.get("ZL_LIBRARY") or os.path.join(LIB_DIR, "libzealot_hip.so")
CODE_OBJECT_PATH = os.path.join(LIB_DIR, "zealot_kernels.hsaco")

ZL_OK = 0
ZL_ERR_INVALID = 1
ZL_ERR_HIP = 2
ZL_ERR_CODE_OBJECT = 3
ZL_ERR_SELF_TEST = 4

ZL_SEMANTICS_ACTOR_CRITIC = 0
ZL_SEMANTICS_GPU_TRAINER = 1

fp = C.POINTER(C.c_float)
ip = C.POINTER(C.c_int)
vp = C.c_void_p


class zl_ppo_config(C.Structure):
    _fields_ = [
        ("semantics", C.c_int),
        ("clip", C.c_float),
        ("entropy_coef", C.c_float),
        ("value_coef", C.c_float),
        ("epochs", C.c_int),
        ("minibatches", C.c_int),
        ("max_grad_norm", C.c_float),
        ("desired_kl", C.c_float),
        ("lr_min", C.c_float),
        ("lr_max", C.c_float),
        ("adaptive_lr", C.c_int),
        ("early_stop", C.c_int),
        ("shuffle", C.c_int),
        ("normalize_adv", C.c_int),
        ("clamp_log_std", C.c_int),
    ]


class zl_batch(C.Structure):
    _fields_ = [
        ("n", C.c_longlong),
        ("obs", vp),
        ("ld_obs", C.c_int),
        ("critic_obs", vp),
        ("ld_critic_obs", C.c_int),
        ("action", vp),
        ("ld_action", C.c_int),
        ("mean_old", vp),
        ("ld_mean_old", C.c_int),
        ("logp_old", vp),
        ("value_old", vp),
        ("adv", vp),
        ("ret", vp),
        ("feature_major", C.c_uint),
    ]


ZL_FM_OBS = 1
ZL_FM_CRITIC_OBS = 2
ZL_FM_ACTION = 4
ZL_FM_MEAN_OLD = 8


class zl_tensor(C.Structure):
    _fields_ = [("ptr", vp), ("n", C.c_size_t)]


class zl_adam_tensor(C.Structure):
    _fields_ = [("p", vp), ("g", vp), ("m", vp), ("v", vp), ("n", C.c_size_t)]


class zl_ppo_stats(C.Structure):
    _fields_ = [
        ("kl", C.c_float),
        ("surrogate", C.c_float),
        ("value_loss", C.c_float),
        ("entropy", C.c_float),
        ("lr", C.c_float),
        ("epochs_run", C.c_int),
        ("last_kl", C.c_float),
        ("grad_norm", C.c_float * 3),
    ]


# name -> (restype, argtypes); one entry per function of include/zealot_hip.h.
SIGNATURES = {
    "zl_init": (C.c_int, [C.c_int, C.POINTER(vp)]),
    "zl_destroy": (None, [vp]),
    "zl_last_error": (C.c_char_p, [vp]),
    "zl_global_error": (C.c_char_p, []),
    "zl_stream": (vp, [vp]),
    "zl_self_test_error": (C.c_double, [vp]),
    "zl_synchronize": (C.c_int, [vp]),
    "zl_version": (C.c_char_p, []),
    "zl_abi_struct_sizes": (None, [C.POINTER(C.c_size_t)]),
    "zl_timing_begin": (C.c_int, [vp, C.c_char_p]),
    "zl_timing_end": (
        C.c_int, [vp, C.POINTER(C.c_double), C.POINTER(C.c_longlong), C.POINTER(C.c_double)]
    ),
    "zl_kernel_count": (C.c_int, []),
    "zl_timing_launch_count": (C.c_longlong, [vp]),
    "zl_timing_launch": (
        C.c_int,
        [vp, C.c_longlong, C.POINTER(C.c_char_p), C.POINTER(C.c_double), C.POINTER(C.c_double),
         C.POINTER(C.c_int)],
    ),
    "zl_timing_kernel": (
        C.c_int,
        [vp, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_double), C.POINTER(C.c_longlong),
         C.POINTER(C.c_double)],
    ),
    "zl_alloc": (C.c_int, [vp, C.c_size_t, C.POINTER(vp)]),
    "zl_free": (C.c_int, [vp, vp]),
    "zl_upload": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "zl_download": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "zl_copy_d2d": (C.c_int, [vp, vp, vp, C.c_size_t]),
    "zl_gemm": (C.c_int, [vp, vp, vp, C.c_int, vp, C.c_int, C.c_int, C.c_int, C.c_int]),
    "zl_gemm_bias_act": (
        C.c_int,
        [vp, vp, vp, vp, C.c_int, C.c_int, C.c_int, vp, C.c_int, C.c_int],
    ),
    "zl_elu_backward": (C.c_int, [vp, vp, vp, C.c_int, C.c_int]),
    "zl_row_sum": (C.c_int, [vp, vp, vp, C.c_int, C.c_int]),
    "zl_ppo_actor_grad": (
        C.c_int,
        [vp, vp, C.c_int, vp, C.c_int, vp, vp, vp, vp, C.c_int, C.c_int, C.c_int,
         C.c_float, C.c_float, C.c_float, vp, C.c_int, vp, vp, C.c_int],
    ),
    "zl_ppo_value_grad": (
        C.c_int,
        [vp, vp, vp, vp, C.c_int, C.c_float, C.c_float, C.c_float, vp, vp],
    ),
    "zl_adam_step": (
        C.c_int,
        [vp, vp, vp, vp, vp, C.c_size_t, C.c_float, C.c_float, C.c_float, C.c_float,
         C.c_float, C.c_float],
    ),
    "zl_grad_sqnorm": (C.c_int, [vp, vp, C.c_size_t, vp]),
    "zl_grad_clip_scale": (C.c_int, [vp, C.POINTER(zl_tensor), C.c_int, C.c_float, vp, vp]),
    "zl_grad_clip_scale_noalloc": (C.c_int, [vp, C.POINTER(zl_tensor), C.c_int, C.c_float, vp, vp]),
    "zl_adam_multi": (
        C.c_int,
        [vp, C.POINTER(zl_adam_tensor), C.c_int, C.c_float, C.c_float, C.c_float, C.c_float,
         C.c_float, C.c_float, vp],
    ),
    "zl_adam_multi_clip": (C.c_int, [vp, C.POINTER(zl_adam_tensor), C.c_int, C.c_float, C.c_float, C.c_float,
                                     C.c_float, C.c_float, C.c_float, C.c_float, vp, vp]),
    "zl_gae": (
        C.c_int,
        [vp, vp, vp, vp, vp, C.c_int, C.c_int, C.c_longlong, C.c_longlong, C.c_longlong,
         C.c_longlong, C.c_float, C.c_float, vp, vp],
    ),
    "zl_adv_normalize": (C.c_int, [vp, vp, C.c_size_t]),
    "zl_sample_actions": (
        C.c_int,
        [vp, vp, C.c_int, vp, vp, C.c_int, C.c_int, vp, vp],
    ),
    "zl_norm_reset": (C.c_int, [vp, vp, C.c_int, C.c_int]),
    "zl_norm_update": (C.c_int, [vp, vp, C.c_int, vp, C.c_int, C.c_longlong]),
    "zl_norm_commit": (C.c_int, [vp, vp, vp, C.c_int]),
    "zl_norm_normalize": (C.c_int, [vp, vp, C.c_int, vp, C.c_int, C.c_longlong, vp, C.c_int]),
    "zl_ppo_act": (
        C.c_int,
        [vp, vp, vp, C.c_int, vp, vp, C.c_int, C.c_longlong, vp, vp, vp, vp, C.c_int, vp],
    ),
    "zl_ppo_save": (C.c_int, [vp, vp, vp, C.c_int, C.c_char_p]),
    "zl_ppo_save_bytes": (C.c_int, [vp, vp, vp, C.c_int, vp, C.c_size_t, C.POINTER(C.c_size_t)]),
    "zl_ppo_load": (C.c_int, [vp, vp, vp, C.c_int, C.c_char_p]),
    "zl_ppo_load_bytes": (C.c_int, [vp, vp, vp, C.c_int, vp, C.c_size_t]),
    "zl_checkpoint_dims": (C.c_int, [vp, C.c_size_t, ip, ip, ip, ip, C.c_int]),
    "zl_mlp_create": (C.c_int, [vp, ip, C.c_int, C.c_int, C.POINTER(vp)]),
    "zl_mlp_create_ex": (C.c_int, [vp, ip, C.c_int, C.c_int, C.c_int, C.POINTER(vp)]),
    "zl_mlp_destroy": (None, [vp]),
    "zl_mlp_num_params": (C.c_longlong, [vp]),
    "zl_mlp_write_weights": (C.c_int, [vp, vp]),
    "zl_mlp_read_weights": (C.c_int, [vp, vp]),
    "zl_mlp_forward": (C.c_int, [vp, vp, C.c_int, C.c_int]),
    "zl_mlp_output": (vp, [vp, ip]),
    "zl_mlp_backward": (C.c_int, [vp, vp, C.c_int]),
    "zl_mlp_read_grads": (C.c_int, [vp, vp]),
    "zl_mlp_adam": (C.c_int, [vp, C.c_float, C.c_float, C.c_float]),
    "zl_mlp_read_moments": (C.c_int, [vp, vp, vp]),
    "zl_mlp_write_moments": (C.c_int, [vp, vp, vp]),
    "zl_ppo_create": (C.c_int, [vp, ip, C.c_int, ip, C.c_int, C.c_int, C.POINTER(vp)]),
    "zl_ppo_destroy": (None, [vp]),
    "zl_ppo_set_params": (C.c_int, [vp, vp, vp, vp, C.c_float]),
    "zl_ppo_get_params": (C.c_int, [vp, vp, vp, vp, fp]),
    "zl_ppo_get_moments": (C.c_int, [vp, vp, vp, vp, vp, vp, vp]),
    "zl_ppo_reset_optimizer": (C.c_int, [vp]),
    "zl_ppo_get_counters": (C.c_int, [vp, ip, C.POINTER(C.c_ulonglong)]),
    "zl_ppo_update": (
        C.c_int,
        [vp, C.POINTER(zl_batch), C.POINTER(zl_ppo_config), C.POINTER(zl_ppo_stats)],
    ),
    "zl_ppo_minibatch_grads": (
        C.c_int,
        [vp, C.POINTER(zl_batch), C.POINTER(zl_ppo_config), C.c_longlong, C.c_int, vp, fp],
    ),
    "zl_ppo_get_grads": (C.c_int, [vp, vp, vp, vp]),
    "zl_ppo_graph_info": (C.c_int, [vp, C.POINTER(C.c_longlong), C.POINTER(C.c_double)]),
    "zl_ppo_values": (C.c_int, [vp, vp, C.c_int, C.c_longlong, vp]),
    "zl_ppo_actor_mean": (C.c_int, [vp, vp, C.c_int, C.c_longlong, vp, C.c_int]),
}

_lib = None


def load_library() -> C.CDLL:
    """Load libzealot_hip.so (raises if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it first (python -c 'import __graft_entry__ as g; g.build()')"
        )
    if not os.environ.get("ZL_LIBRARY") and not os.path.exists(CODE_OBJECT_PATH):
        raise RuntimeError(f"{CODE_OBJECT_PATH} (gfx950 code object) is missing: build it first")
    lib = C.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        f = getattr(lib, name)
        f.restype = res
        f.argtypes = args
    _lib = lib
    return lib
