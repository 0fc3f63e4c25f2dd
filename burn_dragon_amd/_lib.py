"""ctypes binding of libbdh_hip.so (the C ABI declared in include/bdh_hip.h).

The library is loaded from this package directory only.  There is no
fallback: if it is missing, importing the kernels raises, so nothing can run
silently on another path.
"""
from __future__ import annotations

import ctypes
import os
import threading

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libbdh_hip.so")

BDH_OK = 0
BDH_UNSUPPORTED = 1
BDH_EINVAL = -1
BDH_EHIP = -2

BDH_F32 = 0
BDH_BF16 = 1

BDH_KERNEL_PREFILL, BDH_KERNEL_DECODE = 0, 1
BDH_CALIB_READ, BDH_CALIB_COPY, BDH_CALIB_RMW, BDH_CALIB_RMW_ROWS = 0, 1, 2, 3
BDH_CALIB_MFMA_16X16X32_BF16, BDH_CALIB_MFMA_32X32X16_BF16, BDH_CALIB_MFMA_32X32X2_F32 = 0, 1, 2
BDH_ROPE_SEQUENTIAL = 0
BDH_ROPE_FIXED = 1


class BdhRope(ctypes.Structure):
    _fields_ = [("mode", ctypes.c_int32), ("_pad", ctypes.c_int32), ("pos0", ctypes.c_int64),
                ("theta", ctypes.c_float)]


class BdhRecurrentPlan(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in
                ("batch", "heads", "value_heads", "time", "latent", "embd")]


class BdhLayerPlan(ctypes.Structure):
    _fields_ = [(n, ctypes.c_int64) for n in ("batch", "heads", "time", "latent", "embd")]


class BdhLayerOptions(ctypes.Structure):
    _fields_ = [("relu_threshold", ctypes.c_float), ("_pad", ctypes.c_int32),
                ("latent_mask", ctypes.c_void_p)]


class BdhLayerStateDesc(ctypes.Structure):
    _fields_ = [("batch", ctypes.c_int64), ("heads", ctypes.c_int64), ("latent", ctypes.c_int64),
                ("embd", ctypes.c_int64), ("persist_sequence_state", ctypes.c_int32),
                ("retain_terminal_sequence_state", ctypes.c_int32)]


class BdhProfileSnapshot(ctypes.Structure):
    _fields_ = [(n, ctypes.c_uint64) for n in (
        "calls", "launches", "total_ns", "setup_ns", "copy_ns", "dispatch_ns",
        "transient_allocations", "metadata_upload_bytes", "metadata_reuse_hits",
        "metadata_reuse_bytes", "resident_rollout_steps")]


# Every exported symbol of include/bdh_hip.h with its ctypes signature.
_vp = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
SIGNATURES = {
    "bdh_rope_freqs": (_i32, [_i64, ctypes.c_float, ctypes.POINTER(ctypes.c_float)]),
    "bdh_recurrent_plan_new": (_i32, [_i64] * 6 + [ctypes.POINTER(BdhRecurrentPlan)]),
    "bdh_supports_backend": (_i32, []),
    "bdh_recurrent_attention_fwd": (_i32, [ctypes.POINTER(BdhRecurrentPlan), _i32, _vp, _vp, _vp,
                                           _vp, _vp, _vp, _i32, _vp]),
    "bdh_recurrent_attention_rope_fwd": (_i32, [ctypes.POINTER(BdhRecurrentPlan), _i32, _vp, _vp,
                                                _vp, _vp, ctypes.POINTER(BdhRope), _vp, _vp, _i32,
                                                _vp]),
    "bdh_decode_step": (_i32, [_i64] * 5 + [_vp, _vp, _vp, _vp, ctypes.POINTER(BdhRope), _vp,
                                            _vp, _vp, _vp]),
    "bdh_decode_step_noalloc": (_i32, [_i64] * 5 + [_vp, _vp, _vp, _vp, ctypes.POINTER(BdhRope),
                                                    _vp, _vp, _vp, _vp]),
    "bdh_dense_causal_attention_fwd": (_i32, [ctypes.POINTER(BdhRecurrentPlan), _i32, _vp, _vp,
                                              _vp, _vp, _vp]),
    "bdh_dense_causal_attention_vjp": (_i32, [ctypes.POINTER(BdhRecurrentPlan)] + [_vp] * 10),
    "bdh_recurrent_attention_vjp": (_i32, [ctypes.POINTER(BdhRecurrentPlan)] + [_vp] * 10),
    "bdh_lowrank_pack_weights": (_i32, [_i64] * 3 + [_vp] * 7),
    "bdh_lowrank_layer_fwd": (_i32, [ctypes.POINTER(BdhLayerPlan), _vp, _vp, _vp, _vp,
                                     ctypes.POINTER(BdhRope), _vp, _vp, _vp, _vp]),
    "bdh_lowrank_layer_fwd_ex": (_i32, [ctypes.POINTER(BdhLayerPlan), _vp, _vp, _vp, _vp,
                                        ctypes.POINTER(BdhRope), _vp, _vp, _vp,
                                        ctypes.POINTER(BdhLayerOptions), _vp]),
    "bdh_embed_norm": (_i32, [_vp, _i64, _vp, _i64, _i64, _vp, _vp]),
    "bdh_lm_head_pack": (_i32, [_i64, _i64, _vp, _vp, _vp]),
    "bdh_lm_logits": (_i32, [_vp, _i64, _i64, _vp, _i64, _vp, _vp]),
    "bdh_state_record_save": (_i32, [ctypes.c_char_p, _i64, _i32, ctypes.POINTER(BdhLayerStateDesc),
                                     ctypes.POINTER(_vp), _vp]),
    "bdh_state_record_info": (_i32, [ctypes.c_char_p, ctypes.POINTER(_i64), ctypes.POINTER(_i32),
                                     ctypes.POINTER(BdhLayerStateDesc), _i32]),
    "bdh_state_record_load": (_i32, [ctypes.c_char_p, _i32, ctypes.POINTER(BdhLayerStateDesc),
                                     ctypes.POINTER(_vp), _vp]),
    "bdh_profile_enable": (None, [_i32]),
    "bdh_profile_reset": (None, []),
    "bdh_profile_get": (None, [ctypes.POINTER(BdhProfileSnapshot)]),
    "bdh_profile_kernel_timing": (_i32, [_i32]),
    "bdh_profile_kernel_get": (_i32, [_i32, ctypes.POINTER(ctypes.c_double),
                                      ctypes.POINTER(ctypes.c_int64)]),
    "bdh_scratch_release": (_i32, [_vp]),
    "bdh_selftest_rot8": (_i32, [_vp] * 6 + [_i64, _vp]),
    "bdh_calib_hbm": (_i32, [_i32, _vp, _vp, _i64, _vp, _i64, _vp]),
    "bdh_calib_mfma": (_i32, [_i32, _i64, _vp, _vp, _vp]),
    "bdh_last_error": (ctypes.c_char_p, []),
    "bdh_version": (ctypes.c_char_p, []),
}

_lib = None
_lock = threading.Lock()


class BdhError(RuntimeError):
    pass


def load() -> ctypes.CDLL:
    """Loads the in-tree library (raises if it has not been built)."""
    global _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"{LIB_PATH} is missing: build the HIP extension first "
                    "(python -m burn_dragon_amd.build or __graft_entry__.build())")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def last_error() -> str:
    msg = load().bdh_last_error()
    return msg.decode() if msg else ""


def check(status: int) -> bool:
    """True for BDH_OK, False for BDH_UNSUPPORTED (the reference's None);
    raises for errors."""
    if status == BDH_OK:
        return True
    if status == BDH_UNSUPPORTED:
        return False
    raise BdhError(f"bdh status {status}: {last_error()}")
