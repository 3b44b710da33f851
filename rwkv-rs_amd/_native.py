"""ctypes binding of libwkv7_hip.so, the C ABI declared in include/wkv7.h and
include/rwkv_neighbors.h.

The library is built in-tree by rwkv-rs_amd/build.py. Loading fails loudly when
it is missing: there is no fallback implementation.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libwkv7_hip.so")

WKV7_OK = 0
WKV7_ERR_HANDOVER = 11
DTYPE_F32 = 0
DTYPE_BF16 = 1
KERNELS_AUTO = 0
KERNELS_STEP = 1

STATUS_NAMES = {
    0: "WKV7_OK", 1: "WKV7_ERR_NULL_POINTER", 2: "WKV7_ERR_SHAPE",
    3: "WKV7_ERR_CHUNK_LEN", 4: "WKV7_ERR_HEAD_SIZE", 5: "WKV7_ERR_DTYPE",
    6: "WKV7_ERR_ALIGNMENT", 7: "WKV7_ERR_OVERLAP", 8: "WKV7_ERR_FLAGS",
    9: "WKV7_ERR_HIP", 10: "WKV7_ERR_SCRATCH_LIMIT", 11: "WKV7_ERR_HANDOVER",
}


class Wkv7Options(ctypes.Structure):
    """struct wkv7_options (include/wkv7.h)."""
    _fields_ = [("kernels", ctypes.c_int), ("handover_spin_limit", ctypes.c_uint32)]


def options_ref(opts):
    """A pointer argument for an optional wkv7_options (None -> NULL)."""
    return None if opts is None else ctypes.cast(ctypes.pointer(opts), ctypes.c_void_p)

# every symbol include/wkv7.h declares
EXPORTS = (
    "wkv7_abi_version", "wkv7_strerror", "wkv7_last_hip_error", "wkv7_checkpoint_numel",
    "wkv7_forward", "wkv7_backward", "wkv7_forward_ex", "wkv7_backward_ex", "wkv7_take_faults",
    "wkv7_pretrain_forward", "wkv7_pretrain_backward",
    "wkv7_statepass_forward", "wkv7_statepass_backward",
    "wkv7_statetune_forward", "wkv7_statetune_backward",
    "wkv7_infer_forward", "wkv7_selftest_bf16_ops",
    "rwkv_token_shift_mix_workspace_bytes", "rwkv_token_shift_mix_forward",
    "rwkv_token_shift_mix_backward", "rwkv_gated_readout_workspace_bytes",
    "rwkv_gated_readout_forward", "rwkv_gated_readout_backward",
    "rwkv_gated_readout_backward_noalloc",
    "rwkv_weight_prepare_workspace_bytes", "rwkv_weight_prepare_forward",
    "rwkv_weight_prepare_backward",
    "rwkv_cross_entropy_l2wrap_forward", "rwkv_cross_entropy_l2wrap_backward",
)

_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_INT = ctypes.c_int

_SIGNATURES = {
    "wkv7_abi_version": ([], _INT),
    "wkv7_strerror": ([_INT], ctypes.c_char_p),
    "wkv7_last_hip_error": ([], _INT),
    "wkv7_checkpoint_numel": ([_I64] * 5, _I64),
    "wkv7_forward": ([_P] * 7 + [_I64] * 5 + [_INT] * 3 + [_P] * 5, _INT),
    "wkv7_backward": ([_P] * 10 + [_I64] * 5 + [_INT] * 3 + [_P] * 8, _INT),
    "wkv7_forward_ex": ([_P] * 7 + [_I64] * 5 + [_INT] * 3 + [_P] * 6, _INT),
    "wkv7_backward_ex": ([_P] * 10 + [_I64] * 5 + [_INT] * 3 + [_P] * 9, _INT),
    "wkv7_take_faults": ([_P, _P], _INT),
    "wkv7_pretrain_forward": ([_P] * 6 + [_I64] * 5 + [_INT] + [_P] * 4, _INT),
    "wkv7_pretrain_backward": ([_P] * 9 + [_I64] * 5 + [_INT] + [_P] * 7, _INT),
    "wkv7_statepass_forward": ([_P] * 7 + [_I64] * 5 + [_INT] + [_P] * 5, _INT),
    "wkv7_statepass_backward": ([_P] * 10 + [_I64] * 5 + [_INT] + [_P] * 8, _INT),
    "wkv7_statetune_forward": ([_P] * 7 + [_I64] * 5 + [_INT] + [_P] * 4, _INT),
    "wkv7_statetune_backward": ([_P] * 9 + [_I64] * 5 + [_INT] + [_P] * 8, _INT),
    "wkv7_infer_forward": ([_P] * 10 + [_I64] * 5 + [_INT] * 3 + [_P] * 2, _INT),
    "wkv7_selftest_bf16_ops": ([_P, _P, _I64, _P, _P, _P], _INT),
    "rwkv_token_shift_mix_workspace_bytes": ([_I64] * 4, _I64),
    "rwkv_token_shift_mix_forward": ([_P] * 5 + [_I64] * 5 + [_INT] * 2 + [_P] * 4, _INT),
    "rwkv_token_shift_mix_backward": ([_P] * 5 + [_I64] * 5 + [_INT] * 2 + [_P] * 6 + [_I64, _P],
                                      _INT),
    "rwkv_gated_readout_workspace_bytes": ([_I64] * 3, _I64),
    "rwkv_gated_readout_forward": ([_P] * 8 + [ctypes.c_float] + [_I64] * 3 + [_INT] * 2
                                   + [_P] * 2, _INT),
    "rwkv_gated_readout_backward": ([_P] * 8 + [ctypes.c_float] + [_I64] * 3 + [_INT] * 2
                                    + [_P] * 10 + [_I64, _P], _INT),
    "rwkv_gated_readout_backward_noalloc": ([_P] * 8 + [ctypes.c_float] + [_I64] * 3
                                            + [_INT] * 2 + [_P] * 10, _INT),
    "rwkv_weight_prepare_workspace_bytes": ([_I64] * 3, _I64),
    "rwkv_weight_prepare_forward": ([_P] * 11 + [_I64] * 3 + [_INT] * 2 + [_P] * 6, _INT),
    "rwkv_weight_prepare_backward": ([_P] * 11 + [_I64] * 3 + [_INT] * 2 + [_P] * 17
                                     + [_I64, _P], _INT),
    "rwkv_cross_entropy_l2wrap_forward": ([_P] * 2 + [_I64] * 2 + [_INT] + [_P] * 5, _INT),
    "rwkv_cross_entropy_l2wrap_backward": ([_P] * 6 + [ctypes.c_float] + [_I64] * 2 + [_INT]
                                           + [_P] * 2, _INT),
}

_lib = None


class Wkv7Error(RuntimeError):
    """A non-zero wkv7_status from the C ABI."""

    def __init__(self, status: int, message: str):
        super().__init__(f"{message} ({STATUS_NAMES.get(status, status)})")
        self.status = status


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"WKV7 HIP library not built: {LIB_PATH} is missing "
            "(run `python rwkv-rs_amd/build.py`)")
    handle = ctypes.CDLL(LIB_PATH)
    for name, (args, res) in _SIGNATURES.items():
        fn = getattr(handle, name)
        fn.argtypes = args
        fn.restype = res
    _lib = handle
    return handle


def check(status: int) -> None:
    if status != WKV7_OK:
        l = lib()
        msg = l.wkv7_strerror(status).decode()
        if status == 9:
            msg += f": hipError {l.wkv7_last_hip_error()}"
        raise Wkv7Error(status, msg)


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args))
