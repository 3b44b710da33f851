"""Host-side mirror of rwkv-nn's WKV7 operator API over the gfx950 C ABI.

Names, argument order and meaning follow the reference
(/root/reference/crates/rwkv-nn/src/kernels/):

* backend-trait methods -> ``wkv7_{pretrain,statepass,statetune}_{forward,backward}``
  and ``wkv7_infer_forward`` (wkv7_pretrain/mod.rs:18-104,
  wkv7_statepass/mod.rs:18-116, wkv7_statetune/mod.rs:18-110,
  wkv7_infer/mod.rs:30-82); the pretrain forward takes a ``Wkv7ForwardInput``
  like its Rust free function (wkv7_pretrain/mod.rs:46-69)
* output structs -> ``Wkv7ForwardOutput``, ``Wkv7StatePassForwardOutput``,
  ``Wkv7BackwardOutput``, ``Wkv7StateBackwardOutput``,
  ``Wkv7InferForwardOutput`` (wkv7_common/mod.rs:161-204, wkv7_infer/mod.rs:21-24)
* Autodiff wrappers -> ``torch.autograd.Function`` subclasses
  (wkv7_pretrain/backward.rs:16-234, wkv7_statepass/backward.rs:16-265,
  wkv7_statetune/backward.rs:16-254)
* ``Wkv7Kernel`` dispatch -> ``KernelPretrain``, ``KernelStatePass``,
  ``KernelStateTune``, ``KernelInfer`` (wkv7_common/mod.rs:25-153)

Tensors live on the GPU (torch is only the device-memory and stream
plumbing); every computation is one call into libwkv7_hip.so on the current
stream. Operands are made contiguous like the reference's ``into_contiguous``;
outputs are allocated here like its ``empty_device`` (wkv7_common/host.rs:114-137).
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass
from typing import List, Optional, Tuple

import torch

from . import _native

HEAD_SIZE = 64


# --------------------------------------------------------------------- structs
@dataclass
class Wkv7ForwardInput:
    """wkv7_common/mod.rs:161-168"""
    receptance: torch.Tensor
    weight_decay: torch.Tensor
    replacement_key: torch.Tensor
    value: torch.Tensor
    removal_key_normalized: torch.Tensor
    replacement: torch.Tensor


@dataclass
class Wkv7ForwardOutput:
    """wkv7_common/mod.rs:171-175 (Wkv7ForwardOutput)"""
    state: torch.Tensor
    removal_state: torch.Tensor
    output: torch.Tensor


@dataclass
class Wkv7StatePassForwardOutput:
    """wkv7_common/mod.rs:178-183"""
    state: torch.Tensor
    removal_state: torch.Tensor
    output: torch.Tensor
    final_state: torch.Tensor


@dataclass
class Wkv7BackwardOutput:
    """wkv7_common/mod.rs:186-193"""
    weight_decay_grad: torch.Tensor
    receptance_grad: torch.Tensor
    key_grad: torch.Tensor
    value_grad: torch.Tensor
    removal_grad: torch.Tensor
    replacement_grad: torch.Tensor


@dataclass
class Wkv7StateBackwardOutput:
    """wkv7_common/mod.rs:196-204"""
    weight_decay_grad: torch.Tensor
    receptance_grad: torch.Tensor
    key_grad: torch.Tensor
    value_grad: torch.Tensor
    removal_grad: torch.Tensor
    replacement_grad: torch.Tensor
    initial_state_grad: torch.Tensor


@dataclass
class Wkv7InferForwardOutput:
    """wkv7_infer/mod.rs:21-24"""
    output: torch.Tensor
    final_state: torch.Tensor


@dataclass
class KernelOutput:
    """wkv7_common/mod.rs:155-158"""
    output: torch.Tensor
    next_state: Optional[torch.Tensor]


# --------------------------------------------------------------------- helpers
def _dtype_code(t: torch.Tensor) -> int:
    if t.dtype == torch.float32:
        return _native.DTYPE_F32
    if t.dtype == torch.bfloat16:
        return _native.DTYPE_BF16
    raise TypeError(f"WKV7 operands must be float32 or bfloat16, got {t.dtype}")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _tokens(*ts: torch.Tensor):
    """Contiguous per-token operands with one shape, dtype and device."""
    ref = ts[0]
    if ref.dim() != 4:
        raise ValueError(f"expected [batch, context_len, num_heads, head_size], got {tuple(ref.shape)}")
    if not ref.is_cuda:
        raise ValueError("WKV7 operands must be GPU tensors")
    out = []
    for t in ts:
        if t.shape != ref.shape or t.dtype != ref.dtype or t.device != ref.device:
            raise ValueError("all per-token operands must share shape, dtype and device")
        out.append(t.contiguous())
    return out


def _state(t: Optional[torch.Tensor], shape, device) -> Optional[torch.Tensor]:
    if t is None:
        return None
    if tuple(t.shape) != tuple(shape):
        raise ValueError(f"state tensor must have shape {tuple(shape)}, got {tuple(t.shape)}")
    return t.to(device=device, dtype=torch.float32).contiguous()


# --------------------------------------------------------------- kernel timing
_event_log: Optional[List[Tuple[str, "torch.cuda.Event", "torch.cuda.Event"]]] = None


@contextlib.contextmanager
def kernel_events(log: list):
    """Record a (name, start, end) pair of timing events on the launch stream
    around every forward and backward call into the library while the block
    runs; ``name`` is "forward" or "backward". The caller synchronises and
    reads ``start.elapsed_time(end)``. Used to report the operator's share of
    a model step."""
    global _event_log
    prev, _event_log = _event_log, log
    try:
        yield log
    finally:
        _event_log = prev


def _mark(name: str, device: torch.device):
    if _event_log is None:
        return None
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(torch.cuda.current_stream(device))
    _event_log.append((name, start, end))
    return end


def _close(end, device: torch.device) -> None:
    if end is not None:
        end.record(torch.cuda.current_stream(device))


def _check_chunk(T: int, chunk_len: int) -> None:
    # wkv7_common/host.rs:109-112 (the reference panics with this message)
    if chunk_len <= 0 or T % chunk_len != 0:
        raise ValueError("chunk_len must divide sequence length")


# ---------------------------------------------------------- forward / backward
def _options(kernels: str = "auto", handover_spin_limit: int = 0):
    """A ``wkv7_options`` for the ``_ex`` entry points (kernels "auto" or
    "step"), or None for the defaults."""
    codes = {"auto": _native.KERNELS_AUTO, "step": _native.KERNELS_STEP}
    if kernels not in codes:
        raise ValueError(f"kernels must be one of {sorted(codes)}")
    if kernels == "auto" and handover_spin_limit == 0:
        return None
    return _native.Wkv7Options(codes[kernels], int(handover_spin_limit))


def _forward(w, r, k, v, a, b, initial_state, chunk_len, use_initial_state, return_final_state,
             options=None):
    w, r, k, v, a, b = _tokens(w, r, k, v, a, b)
    B, T, H, N = w.shape
    _check_chunk(T, chunk_len)
    dev = w.device
    s0 = _state(initial_state, (B, H, N, N), dev) if use_initial_state else None
    state = torch.empty((B, H, T // chunk_len, N, N), dtype=torch.float32, device=dev)
    removal_state = torch.empty((B, T, H, N), dtype=torch.float32, device=dev)
    output = torch.empty_like(w)
    final_state = (torch.empty((B, H, N, N), dtype=torch.float32, device=dev)
                   if return_final_state else None)
    end = _mark("forward", dev)
    _native.call("wkv7_forward_ex", _ptr(w), _ptr(r), _ptr(k), _ptr(v), _ptr(a), _ptr(b),
                 _ptr(s0), B, T, H, N, chunk_len, _dtype_code(w), int(use_initial_state),
                 int(return_final_state), _ptr(state), _ptr(removal_state), _ptr(output),
                 _ptr(final_state), _native.options_ref(options), _stream(dev))
    _close(end, dev)
    return state, removal_state, output, final_state


def _backward(w, r, k, v, a, b, state, removal_state, output_grad, final_state_grad, chunk_len,
              use_final_state_grad, write_initial_state_grad, options=None):
    w, r, k, v, a, b, output_grad = _tokens(w, r, k, v, a, b, output_grad)
    B, T, H, N = w.shape
    _check_chunk(T, chunk_len)
    dev = w.device
    state = _state(state, (B, H, T // chunk_len, N, N), dev)
    removal_state = _state(removal_state, (B, T, H, N), dev)
    dsT = _state(final_state_grad, (B, H, N, N), dev) if use_final_state_grad else None
    grads = [torch.empty_like(w) for _ in range(6)]
    ds0 = (torch.empty((B, H, N, N), dtype=torch.float32, device=dev)
           if write_initial_state_grad else None)
    end = _mark("backward", dev)
    _native.call("wkv7_backward_ex", _ptr(w), _ptr(r), _ptr(k), _ptr(v), _ptr(a), _ptr(b),
                 _ptr(state), _ptr(removal_state), _ptr(output_grad), _ptr(dsT),
                 B, T, H, N, chunk_len, _dtype_code(w), int(use_final_state_grad),
                 int(write_initial_state_grad), *(_ptr(g) for g in grads), _ptr(ds0),
                 _native.options_ref(options), _stream(dev))
    _close(end, dev)
    return grads, ds0


# ----------------------------------------------- explicit kernel choice (_ex)
def wkv7_forward_ex(weight_decay, receptance, key, value, removal, replacement, initial_state,
                    chunk_len, use_initial_state=True, return_final_state=True,
                    kernels: str = "auto", handover_spin_limit: int = 0
                    ) -> Wkv7StatePassForwardOutput:
    """wkv7_forward_ex (include/wkv7.h): the generic forward with an explicit
    kernel family ("auto", or "step" for the step-by-step kernels, the
    reference's operation order, in every case) and hand-over bound. No
    counterpart in the reference."""
    state, sa, y, sT = _forward(weight_decay, receptance, key, value, removal, replacement,
                                initial_state, chunk_len, use_initial_state, return_final_state,
                                _options(kernels, handover_spin_limit))
    return Wkv7StatePassForwardOutput(state=state, removal_state=sa, output=y, final_state=sT)


def wkv7_backward_ex(weight_decay, receptance, key, value, removal, replacement, state,
                     removal_state, output_grad, final_state_grad, chunk_len,
                     use_final_state_grad=True, write_initial_state_grad=True,
                     kernels: str = "auto") -> Wkv7StateBackwardOutput:
    """wkv7_backward_ex (include/wkv7.h) with an explicit kernel family."""
    g, ds0 = _backward(weight_decay, receptance, key, value, removal, replacement, state,
                       removal_state, output_grad, final_state_grad, chunk_len,
                       use_final_state_grad, write_initial_state_grad, _options(kernels))
    return Wkv7StateBackwardOutput(*g, initial_state_grad=ds0)


def take_faults(device=None) -> int:
    """wkv7_take_faults: waits for the current stream, resets the device's
    counter and returns the number of chunked-forward launches on the device
    that gave up a hand-over wait since the last call (their outputs are NaN).
    Other failures of the call raise Wkv7Error."""
    import ctypes
    dev = torch.device("cuda", torch.cuda.current_device()) if device is None else device
    n = ctypes.c_uint32(0)
    status = _native.lib().wkv7_take_faults(_stream(dev), ctypes.byref(n))
    if status not in (_native.WKV7_OK, _native.WKV7_ERR_HANDOVER):
        _native.check(status)
    return int(n.value)


def check_faults(device=None) -> None:
    """Raises Wkv7Error (WKV7_ERR_HANDOVER) when a chunked forward on the
    device gave up a hand-over wait since the last take_faults/check_faults,
    i.e. when some of the outputs computed since then are NaN by that cause.
    Waits for the current stream: call it where the caller synchronises
    anyway (the end of a step, a logged loss), not inside a captured graph."""
    n = take_faults(device)
    if n:
        raise _native.Wkv7Error(_native.WKV7_ERR_HANDOVER,
                                f"{_native.lib().wkv7_strerror(_native.WKV7_ERR_HANDOVER).decode()}"
                                f" ({n} (batch, head) pairs)")


# ------------------------------------------------- Wkv7PretrainBackend (mirror)
def wkv7_pretrain_forward(wkv7_forward_input: Wkv7ForwardInput, chunk_len: int) -> Wkv7ForwardOutput:
    """wkv7_pretrain/mod.rs:46-69 (free function over Wkv7ForwardInput)."""
    i = wkv7_forward_input
    state, sa, y, _ = _forward(i.weight_decay, i.receptance, i.replacement_key, i.value,
                               i.removal_key_normalized, i.replacement, None, chunk_len,
                               False, False)
    return Wkv7ForwardOutput(state=state, removal_state=sa, output=y)


def wkv7_pretrain_backward(weight_decay, receptance, key, value, removal, replacement, state,
                           removal_state, output_grad, chunk_len) -> Wkv7BackwardOutput:
    """wkv7_pretrain/mod.rs:71-104."""
    g, _ = _backward(weight_decay, receptance, key, value, removal, replacement, state,
                     removal_state, output_grad, None, chunk_len, False, False)
    return Wkv7BackwardOutput(*g)


# ------------------------------------------------ Wkv7StatePassBackend (mirror)
def wkv7_statepass_forward(weight_decay, receptance, key, value, removal, replacement,
                           initial_state, chunk_len) -> Wkv7StatePassForwardOutput:
    """wkv7_statepass/mod.rs:48-76."""
    state, sa, y, sT = _forward(weight_decay, receptance, key, value, removal, replacement,
                                initial_state, chunk_len, True, True)
    return Wkv7StatePassForwardOutput(state=state, removal_state=sa, output=y, final_state=sT)


def wkv7_statepass_backward(weight_decay, receptance, key, value, removal, replacement, state,
                            removal_state, output_grad, final_state_grad,
                            chunk_len) -> Wkv7StateBackwardOutput:
    """wkv7_statepass/mod.rs:78-116."""
    g, ds0 = _backward(weight_decay, receptance, key, value, removal, replacement, state,
                       removal_state, output_grad, final_state_grad, chunk_len, True, True)
    return Wkv7StateBackwardOutput(*g, initial_state_grad=ds0)


# ------------------------------------------------ Wkv7StateTuneBackend (mirror)
def wkv7_statetune_forward(weight_decay, receptance, key, value, removal, replacement,
                           initial_state, chunk_len) -> Wkv7ForwardOutput:
    """wkv7_statetune/mod.rs:47-74."""
    state, sa, y, _ = _forward(weight_decay, receptance, key, value, removal, replacement,
                               initial_state, chunk_len, True, False)
    return Wkv7ForwardOutput(state=state, removal_state=sa, output=y)


def wkv7_statetune_backward(weight_decay, receptance, key, value, removal, replacement, state,
                            removal_state, output_grad, chunk_len) -> Wkv7StateBackwardOutput:
    """wkv7_statetune/mod.rs:76-110."""
    g, ds0 = _backward(weight_decay, receptance, key, value, removal, replacement, state,
                       removal_state, output_grad, None, chunk_len, False, True)
    return Wkv7StateBackwardOutput(*g, initial_state_grad=ds0)


# ---------------------------------------------------- Wkv7InferBackend (mirror)
def wkv7_infer_forward(weight_decay, receptance, key, value, removal, replacement, batch_ids,
                       initial_state, context_mask, elapsed_t,
                       use_dither: Optional[bool] = None) -> Wkv7InferForwardOutput:
    """wkv7_infer/mod.rs:58-82. ``initial_state`` ([full_batch, H, 64, 64])
    is updated in place and returned as ``final_state``, like the reference's
    aliasing (wkv7_infer/host.rs:151). Its dtype picks the reference kernel's
    element type: float32 (operands float32 or bfloat16, used as exact fp32
    values) or bfloat16 (operands bfloat16; the state and every operation of
    the step in bf16). ``use_dither`` defaults to the reference's switch,
    "element type is not f32" (host.rs:157), i.e. on for a bfloat16 state; a
    float32 state cannot be dithered."""
    w, r, k, v, a, b = _tokens(weight_decay, receptance, key, value, removal, replacement)
    Ba, T, H, N = w.shape
    dev = w.device
    if initial_state.dtype not in (torch.float32, torch.bfloat16) \
            or not initial_state.is_contiguous() or initial_state.device != dev:
        raise ValueError("initial_state must be a contiguous float32 or bfloat16 tensor on the "
                         "operands' device")
    if initial_state.dtype == torch.bfloat16 and w.dtype != torch.bfloat16:
        raise TypeError("a bfloat16 state needs bfloat16 operands (the reference kernel at "
                        "element type bf16)")
    if use_dither is None:
        use_dither = initial_state.dtype != torch.float32
    if use_dither and initial_state.dtype == torch.float32:
        raise ValueError("the dither applies to a bfloat16 state only (wkv7_infer/host.rs:157)")
    full_batch = initial_state.shape[0]
    if tuple(initial_state.shape[1:]) != (H, N, N):
        raise ValueError("initial_state must be [full_batch, num_heads, 64, 64]")
    ids = batch_ids.to(device=dev, dtype=torch.int32).contiguous()
    if ids.shape != (Ba,):
        raise ValueError("batch_ids must be [active_batch_size]")
    mask = None
    if context_mask is not None:
        mask = context_mask.to(device=dev, dtype=w.dtype).contiguous()
        if mask.shape != (Ba, T):
            raise ValueError("context_mask must be [active_batch_size, context_len]")
    et = None
    if elapsed_t is not None:
        et = elapsed_t.to(device=dev, dtype=torch.int32).contiguous()
        if et.shape != (full_batch,):
            raise ValueError("elapsed_t must be [full_batch_size]")
    output = torch.empty_like(w)
    _native.call("wkv7_infer_forward", _ptr(w), _ptr(r), _ptr(k), _ptr(v), _ptr(a), _ptr(b),
                 _ptr(ids), _ptr(initial_state), _ptr(mask), _ptr(et), Ba, T, H, N, full_batch,
                 _dtype_code(w), _dtype_code(initial_state), int(bool(use_dither)), _ptr(output),
                 _stream(dev))
    return Wkv7InferForwardOutput(output=output, final_state=initial_state)


# ------------------------------------------------------------- Autodiff mirror
class Wkv7PretrainFunction(torch.autograd.Function):
    """Autodiff<B>::wkv7_pretrain_forward (wkv7_pretrain/backward.rs:16-196):
    the six inputs are saved with (state, removal_state, chunk_len); the
    backward returns the six input gradients."""

    @staticmethod
    def forward(ctx, weight_decay, receptance, key, value, removal, replacement, chunk_len):
        state, sa, y, _ = _forward(weight_decay, receptance, key, value, removal, replacement,
                                   None, chunk_len, False, False)
        ctx.save_for_backward(weight_decay, receptance, key, value, removal, replacement, state, sa)
        ctx.chunk_len = chunk_len
        return y

    @staticmethod
    def backward(ctx, dy):
        w, r, k, v, a, b, state, sa = ctx.saved_tensors
        g, _ = _backward(w, r, k, v, a, b, state, sa, dy, None, ctx.chunk_len, False, False)
        return (*g, None)


class Wkv7StatePassFunction(torch.autograd.Function):
    """Autodiff<B>::wkv7_statepass_forward (wkv7_statepass/backward.rs:16-221):
    seven parents including the initial state; the final-state gradient fed to
    the backward kernel is zero (backward.rs:90-95) and the returned final
    state is not tracked (``from_inner``)."""

    @staticmethod
    def forward(ctx, weight_decay, receptance, key, value, removal, replacement, initial_state,
                chunk_len):
        state, sa, y, sT = _forward(weight_decay, receptance, key, value, removal, replacement,
                                    initial_state, chunk_len, True, True)
        ctx.save_for_backward(weight_decay, receptance, key, value, removal, replacement, state, sa)
        ctx.chunk_len = chunk_len
        ctx.s0_dtype = initial_state.dtype
        ctx.mark_non_differentiable(sT)
        return y, sT

    @staticmethod
    def backward(ctx, dy, _dsT_ignored):
        w, r, k, v, a, b, state, sa = ctx.saved_tensors
        zeros = torch.zeros(state.shape[0], state.shape[1], HEAD_SIZE, HEAD_SIZE,
                            dtype=torch.float32, device=w.device)
        g, ds0 = _backward(w, r, k, v, a, b, state, sa, dy, zeros, ctx.chunk_len, True, True)
        return (*g, ds0.to(ctx.s0_dtype), None)


class Wkv7StateTuneFunction(torch.autograd.Function):
    """Autodiff<B>::wkv7_statetune_forward (wkv7_statetune/backward.rs:16-254):
    the initial state is a trainable parent; no final state."""

    @staticmethod
    def forward(ctx, weight_decay, receptance, key, value, removal, replacement, initial_state,
                chunk_len):
        state, sa, y, _ = _forward(weight_decay, receptance, key, value, removal, replacement,
                                   initial_state, chunk_len, True, False)
        ctx.save_for_backward(weight_decay, receptance, key, value, removal, replacement, state, sa)
        ctx.chunk_len = chunk_len
        ctx.s0_dtype = initial_state.dtype
        ctx.mark_non_differentiable(state)
        return y, state

    @staticmethod
    def backward(ctx, dy, _dstate_ignored):
        w, r, k, v, a, b, state, sa = ctx.saved_tensors
        g, ds0 = _backward(w, r, k, v, a, b, state, sa, dy, None, ctx.chunk_len, False, True)
        return (*g, ds0.to(ctx.s0_dtype), None)


# ---------------------------------------------------- Wkv7Kernel dispatch mirror
class KernelPretrain:
    """wkv7_common/mod.rs:36-53: differentiable, the state passes through."""

    @staticmethod
    def forward(input: Wkv7ForwardInput, state, batch_ids, elapsed_t, chunk_len,
                context_mask) -> KernelOutput:
        y = Wkv7PretrainFunction.apply(input.weight_decay, input.receptance, input.replacement_key,
                                       input.value, input.removal_key_normalized,
                                       input.replacement, chunk_len)
        return KernelOutput(output=y, next_state=state)


class KernelStatePass:
    """wkv7_common/mod.rs:55-82: the final state becomes the next state."""

    @staticmethod
    def forward(input: Wkv7ForwardInput, state, batch_ids, elapsed_t, chunk_len,
                context_mask) -> KernelOutput:
        if state is None:
            raise ValueError("KernelStatePass requires a state")
        y, sT = Wkv7StatePassFunction.apply(input.weight_decay, input.receptance,
                                            input.replacement_key, input.value,
                                            input.removal_key_normalized, input.replacement,
                                            state, chunk_len)
        return KernelOutput(output=y, next_state=sT)


class KernelStateTune:
    """wkv7_common/mod.rs:84-111: next_state is the checkpoint tensor, as in
    the reference (``next_state: Some(output.state)``)."""

    @staticmethod
    def forward(input: Wkv7ForwardInput, state, batch_ids, elapsed_t, chunk_len,
                context_mask) -> KernelOutput:
        if state is None:
            raise ValueError("KernelStateTune requires a state")
        y, ckpt = Wkv7StateTuneFunction.apply(input.weight_decay, input.receptance,
                                              input.replacement_key, input.value,
                                              input.removal_key_normalized, input.replacement,
                                              state, chunk_len)
        return KernelOutput(output=y, next_state=ckpt)


class KernelInfer:
    """wkv7_common/mod.rs:113-153: slot-mapped decode; the context mask
    defaults to all ones."""

    @staticmethod
    def forward(input: Wkv7ForwardInput, state, batch_ids, elapsed_t, chunk_len,
                context_mask, use_dither: Optional[bool] = None) -> KernelOutput:
        if state is None:
            raise ValueError("initial_state required")
        if elapsed_t is None:
            raise ValueError("elapsed_t required")
        out = wkv7_infer_forward(input.weight_decay, input.receptance, input.replacement_key,
                                 input.value, input.removal_key_normalized, input.replacement,
                                 batch_ids, state, context_mask, elapsed_t, use_dither)
        return KernelOutput(output=out.output, next_state=out.final_state)
