"""TEST INFRASTRUCTURE ONLY -- the CPU oracle for the WKV7 recurrence.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this package, and only as the checker (or the timed
CPU baseline). The product path in ``rwkv-rs_amd/`` never touches it.

Functions (numpy in, numpy out) wrap ``libwkv7_oracle.so`` built from
``wkv7_oracle.c`` by the Makefile beside it:

* ``forward_f32``  -- reference-order fp32 forward,
  /root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:6-114
* ``backward_f32`` -- reference-order fp32 backward (divide-by-decay reversal,
  checkpoint reload every ``chunk_len`` steps), kernel.rs:116-308
* ``forward_f64`` / ``grad_f64`` -- fp64 forward and a back-propagation
  through time that stores every state (no reversal)
* ``infer_f32``    -- slot-mapped decode, wkv7_infer/kernel.rs:15-114
* ``infer_bf16``   -- the same kernel with element type bf16: bf16 state,
  decay (plus dither) rounded to bf16, every product and sum rounded to bf16
* ``dither``       -- deterministic_dither, wkv7_infer/kernel.rs:8-13

How each function is pinned (tests/test_oracle_*.py):

* forward: N=1 geometric-series closed form; a=b=0 decayed linear attention
  closed form; matrix (DPLR) form of the transition in fp64; chunk_len and
  sequence-split invariance; fp32 vs fp64 agreement.
* backward: fp64 central finite differences of L=<dy,y>+<ds_T,s_T> on tiny
  shapes pin ``grad_f64``; the adjoint identity <dy, J d> = <J^T dy, d>;
  ``backward_f32`` against ``grad_f64`` within the reversal's error bound.
* checkpoints: equal to the fp64 forward state after each chunk, transposed.
* infer: T=1 infer == one forward step (bitwise), masked steps are no-ops, the
  reference's two scalar dither/mask tests (wkv7_infer/mod.rs:189-269), and
  integer known answers of the dither hash.
* infer_bf16: the reference's two scalar tests (wkv7_infer/mod.rs:143-269) at
  N=1 with every F operation rounded to bf16; inputs whose every
  intermediate is a small integer (bf16 arithmetic is then exact: causal
  linear attention, a closed form); agreement with infer_f32 to bf16
  rounding; a row-vectorised numpy evaluation of the same rounding points
  (tests/test_oracle_infer_bf16.py).
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "libwkv7_oracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_f64p = ctypes.POINTER(ctypes.c_double)
_i64 = ctypes.c_int64


def build(force: bool = False) -> str:
    """Compile libwkv7_oracle.so with the Makefile beside this file."""
    if force and os.path.exists(_LIB_PATH):
        os.remove(_LIB_PATH)
    subprocess.run(["make", "-s", "-C", _HERE], check=True)
    return _LIB_PATH


def build_native(out_path: str) -> str:
    """Compile the same source with -march=native for the host it runs on
    (the CPU baseline's build), to ``out_path``, and use it from then on."""
    global _LIB_PATH, _lib
    subprocess.run(["make", "-s", "-C", _HERE, "native", f"NATIVE_OUT={out_path}"], check=True)
    _LIB_PATH, _lib = out_path, None
    return out_path


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        raise RuntimeError(
            f"oracle library missing: {_LIB_PATH} (run `make -C oracle`)")
    lib = ctypes.CDLL(_LIB_PATH)
    lib.wkv7o_forward_f32.argtypes = [_i64] * 5 + [_f32p] * 11 + [ctypes.c_int]
    lib.wkv7o_backward_f32.argtypes = [_i64] * 5 + [_f32p] * 17 + [ctypes.c_int]
    lib.wkv7o_forward_f64.argtypes = [_i64] * 4 + [_f64p] * 9
    lib.wkv7o_grad_f64.argtypes = [_i64] * 4 + [_f64p] * 15
    lib.wkv7o_infer_f32.argtypes = (
        [_i64] * 5 + [_f32p] * 6 + [ctypes.POINTER(ctypes.c_int32), _f32p, _f32p,
                                    ctypes.POINTER(ctypes.c_uint32), ctypes.c_int,
                                    _f32p])
    lib.wkv7o_infer_bf16.argtypes = lib.wkv7o_infer_f32.argtypes
    lib.wkv7o_round_bf16.argtypes = [ctypes.c_float]
    lib.wkv7o_round_bf16.restype = ctypes.c_float
    lib.wkv7o_dither.argtypes = [ctypes.c_uint32]
    lib.wkv7o_dither.restype = ctypes.c_float
    for fn in ("wkv7o_forward_f32", "wkv7o_backward_f32", "wkv7o_forward_f64",
               "wkv7o_grad_f64", "wkv7o_infer_f32", "wkv7o_infer_bf16"):
        getattr(lib, fn).restype = ctypes.c_int
    _lib = lib
    return lib


def _c(x, dtype):
    if x is None:
        return None
    return np.ascontiguousarray(x, dtype=dtype)


def _p(x, ptype):
    if x is None:
        return ctypes.cast(None, ptype)
    return x.ctypes.data_as(ptype)


def _dims(x):
    if x.ndim != 4:
        raise ValueError("expected a [B, T, H, N] array")
    return x.shape


def forward_f32(w, r, k, v, a, b, s0=None, chunk_len=16, return_final_state=True,
                nthreads=0):
    """Reference-order fp32 forward. Returns dict(state, removal_state, output,
    final_state) with the reference's output names (wkv7_common/mod.rs:185-191).
    """
    lib = _load()
    w, r, k, v, a, b = (_c(x, np.float32) for x in (w, r, k, v, a, b))
    s0 = _c(s0, np.float32)
    B, T, H, N = _dims(w)
    if chunk_len <= 0 or T % chunk_len != 0:
        raise ValueError("chunk_len must divide sequence length")
    ckpt = np.empty((B, H, T // chunk_len, N, N), np.float32)
    sa = np.empty_like(w)
    y = np.empty_like(w)
    sT = np.empty((B, H, N, N), np.float32) if return_final_state else None
    rc = lib.wkv7o_forward_f32(B, T, H, N, chunk_len, *(_p(x, _f32p) for x in (
        w, r, k, v, a, b, s0, ckpt, sa, y, sT)), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"wkv7o_forward_f32 failed ({rc})")
    return {"state": ckpt, "removal_state": sa, "output": y, "final_state": sT}


def backward_f32(w, r, k, v, a, b, state, removal_state, dy, ds_T=None,
                 chunk_len=16, write_initial_state_grad=True, nthreads=0):
    """Reference-order fp32 backward. Returns the reference's gradient names
    (wkv7_common/mod.rs:196-204)."""
    lib = _load()
    w, r, k, v, a, b, dy = (_c(x, np.float32) for x in (w, r, k, v, a, b, dy))
    state, removal_state, ds_T = (_c(x, np.float32) for x in (state, removal_state, ds_T))
    B, T, H, N = _dims(w)
    if chunk_len <= 0 or T % chunk_len != 0:
        raise ValueError("chunk_len must divide sequence length")
    outs = [np.empty_like(w) for _ in range(6)]
    ds0 = np.empty((B, H, N, N), np.float32) if write_initial_state_grad else None
    rc = lib.wkv7o_backward_f32(B, T, H, N, chunk_len, *(_p(x, _f32p) for x in (
        w, r, k, v, a, b, state, removal_state, dy, ds_T, *outs, ds0)), int(nthreads))
    if rc != 0:
        raise RuntimeError(f"wkv7o_backward_f32 failed ({rc})")
    dw, dr, dk, dv, da, db = outs
    return {"weight_decay_grad": dw, "receptance_grad": dr, "key_grad": dk,
            "value_grad": dv, "removal_grad": da, "replacement_grad": db,
            "initial_state_grad": ds0}


def forward_f64(w, r, k, v, a, b, s0=None):
    lib = _load()
    w, r, k, v, a, b = (_c(x, np.float64) for x in (w, r, k, v, a, b))
    s0 = _c(s0, np.float64)
    B, T, H, N = _dims(w)
    y = np.empty_like(w)
    sT = np.empty((B, H, N, N), np.float64)
    rc = lib.wkv7o_forward_f64(B, T, H, N, *(_p(x, _f64p) for x in (
        w, r, k, v, a, b, s0, y, sT)))
    if rc != 0:
        raise RuntimeError(f"wkv7o_forward_f64 failed ({rc})")
    return {"output": y, "final_state": sT}


def grad_f64(w, r, k, v, a, b, s0, dy, ds_T=None):
    """Gradient of <dy, y> + <ds_T, s_T> by stored-state BPTT in fp64."""
    lib = _load()
    w, r, k, v, a, b, dy = (_c(x, np.float64) for x in (w, r, k, v, a, b, dy))
    s0, ds_T = _c(s0, np.float64), _c(ds_T, np.float64)
    B, T, H, N = _dims(w)
    outs = [np.empty_like(w) for _ in range(6)]
    ds0 = np.empty((B, H, N, N), np.float64)
    rc = lib.wkv7o_grad_f64(B, T, H, N, *(_p(x, _f64p) for x in (
        w, r, k, v, a, b, s0, dy, ds_T, *outs, ds0)))
    if rc != 0:
        raise RuntimeError(f"wkv7o_grad_f64 failed ({rc})")
    dw, dr, dk, dv, da, db = outs
    return {"weight_decay_grad": dw, "receptance_grad": dr, "key_grad": dk,
            "value_grad": dv, "removal_grad": da, "replacement_grad": db,
            "initial_state_grad": ds0}


def infer_f32(w, r, k, v, a, b, batch_ids, state, context_mask=None,
              elapsed_t=None, use_dither=False):
    """Slot-mapped decode. ``state`` ([full_batch, H, N, N] fp32) is updated in
    place, as the reference kernel does (wkv7_infer/kernel.rs:103-113).
    Returns the output [Ba, T, H, N]."""
    return _infer("wkv7o_infer_f32", w, r, k, v, a, b, batch_ids, state, context_mask,
                  elapsed_t, use_dither)


def infer_bf16(w, r, k, v, a, b, batch_ids, state, context_mask=None,
               elapsed_t=None, use_dither=True):
    """Slot-mapped decode with element type bf16 (the reference kernel at
    F = bf16; its host turns the dither on for every F that is not f32,
    wkv7_infer/host.rs:157). Operands, mask and ``state`` are float32 arrays
    holding bf16 values; ``state`` is updated in place and stays bf16-valued.
    Returns the output [Ba, T, H, N] (bf16 values)."""
    for x in (w, r, k, v, a, b, state):
        if np.any(np.asarray(x, np.float32) != _round_bf16_np(x)):
            raise ValueError("infer_bf16 takes bf16 values")
    return _infer("wkv7o_infer_bf16", w, r, k, v, a, b, batch_ids, state, context_mask,
                  elapsed_t, use_dither)


def _round_bf16_np(x):
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    return ((u + np.uint32(0x7FFF) + ((u >> 16) & 1)) & np.uint32(0xFFFF0000)).view(np.float32)


def round_bf16(x: float) -> float:
    return float(_load().wkv7o_round_bf16(ctypes.c_float(x)))


def _infer(fn, w, r, k, v, a, b, batch_ids, state, context_mask, elapsed_t, use_dither):
    lib = _load()
    w, r, k, v, a, b = (_c(x, np.float32) for x in (w, r, k, v, a, b))
    if state.dtype != np.float32 or not state.flags.c_contiguous:
        raise ValueError("state must be a C-contiguous float32 array")
    Ba, T, H, N = _dims(w)
    full_batch = state.shape[0]
    batch_ids = _c(batch_ids, np.int32)
    mask = _c(context_mask, np.float32)
    et = _c(elapsed_t, np.uint32)
    y = np.empty_like(w)
    rc = getattr(lib, fn)(
        Ba, T, H, N, full_batch, *(_p(x, _f32p) for x in (w, r, k, v, a, b)),
        _p(batch_ids, ctypes.POINTER(ctypes.c_int32)), _p(state, _f32p),
        _p(mask, _f32p), _p(et, ctypes.POINTER(ctypes.c_uint32)),
        int(bool(use_dither)), _p(y, _f32p))
    if rc != 0:
        raise RuntimeError(f"{fn} failed ({rc})")
    return y


def dither(seed: int) -> float:
    return float(_load().wkv7o_dither(ctypes.c_uint32(seed & 0xFFFFFFFF)))
