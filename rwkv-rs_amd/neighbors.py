"""The ops on either side of the WKV7 operator in a time mixer, on the gfx950
kernels of include/rwkv_neighbors.h, as torch autograd Functions.

* ``token_shift_mix`` -- ``token_shift_diff`` followed by ``addcmul5`` /
  ``addcmul`` on its difference, fused: one pass reads x and writes the
  mixes (kernels/token_shift_diff/kernel.rs:17-64, kernels/addcmul/kernel.rs:
  4-53; backward token_shift_diff/backward.rs:34-101, addcmul/backward.rs:
  28-58). ``WeightPrepare`` takes five mixes of one shift and the gated
  readout's gate input is a sixth (gated_readout.rs:122); ``ChannelMixer``
  takes one (channel_mixer/mod.rs:96-106).
* ``weight_prepare_end`` -- the element-wise end of ``WeightPrepare``: the
  learning rate, replacement key, value residual, decay, normalized removal
  key and replacement from the projections and the LoRA products, with the
  LoRA biases (weight_prepare.rs:282-317, layers/lora.rs:118-123), fused.
* ``gated_readout`` -- GroupNorm over heads, the r.k~.bonus term and the gate
  (gated_readout.rs:126-145), fused; the output projection stays a GEMM.

The mixes can be written in another dtype than their input (fp32 residual
stream in, bf16 out for the matrix products that read them, as autocast
would cast them). Gradients of per-channel parameters are reduced on the GPU
in a fixed order. Operands live on the GPU; there is no CPU path.
"""

from __future__ import annotations

import ctypes
from typing import Optional, Sequence

import torch

from . import _native

MAX_MIXES = 8


def _code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return _native.DTYPE_F32
    if dtype == torch.bfloat16:
        return _native.DTYPE_BF16
    raise TypeError(f"expected float32 or bfloat16, got {dtype}")


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else t.data_ptr()


def _ptrs(ts: Sequence[torch.Tensor]):
    arr = (ctypes.c_void_p * max(len(ts), 1))()
    for i, t in enumerate(ts):
        arr[i] = t.data_ptr()
    return arr


def _stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _gpu(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_cuda:
        raise ValueError(f"{what} must be a GPU tensor")
    return t.contiguous()


# --------------------------------------------------------------- token shift
class _TokenShiftMix(torch.autograd.Function):
    @staticmethod
    def forward(ctx, x, scales, token_shift, batch_ids, context_mask, out_dtype, want_next):
        B, T, C = x.shape
        K = scales.shape[0]
        dev = x.device
        mixes = [torch.empty((B, T, C), dtype=out_dtype, device=dev) for _ in range(K)]
        full = token_shift.shape[0] if token_shift is not None else B
        nxt = None
        if want_next:
            nxt = (token_shift.clone() if token_shift is not None
                   else torch.zeros((B, C), dtype=x.dtype, device=dev))
        _native.call("rwkv_token_shift_mix_forward", _ptr(x), _ptr(token_shift), _ptr(batch_ids),
                     _ptr(context_mask), _ptr(scales), K, B, T, C, full, _code(x.dtype),
                     _code(out_dtype), _ptrs(mixes), None, _ptr(nxt), _stream(dev))
        ctx.save_for_backward(x, scales, token_shift, batch_ids, context_mask)
        ctx.out_dtype = out_dtype
        ctx.full = full
        if nxt is not None:
            ctx.mark_non_differentiable(nxt)
            return (*mixes, nxt)
        return tuple(mixes)

    @staticmethod
    def backward(ctx, *grads):
        x, scales, token_shift, batch_ids, context_mask = ctx.saved_tensors
        B, T, C = x.shape
        K = scales.shape[0]
        dev = x.device
        gs = [torch.zeros((B, T, C), dtype=ctx.out_dtype, device=dev) if g is None
              else g.to(ctx.out_dtype).contiguous() for g in grads[:K]]
        dx = torch.empty_like(x)
        dscales = torch.empty((K, C), dtype=torch.float32, device=dev)
        want_shift = token_shift is not None and ctx.needs_input_grad[2]
        dshift = (torch.empty((ctx.full, C), dtype=torch.float32, device=dev)
                  if want_shift else None)
        nbytes = _native.lib().rwkv_token_shift_mix_workspace_bytes(K, B, T, C)
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev)
        _native.call("rwkv_token_shift_mix_backward", _ptr(x), _ptr(token_shift), _ptr(batch_ids),
                     _ptr(context_mask), _ptr(scales), K, B, T, C, ctx.full, _code(x.dtype),
                     _code(ctx.out_dtype), _ptrs(gs), None, _ptr(dx), _ptr(dshift),
                     _ptr(dscales), _ptr(ws), nbytes, _stream(dev))
        if dshift is not None:
            dshift = dshift.to(token_shift.dtype)
        return dx, dscales, dshift, None, None, None, None


def token_shift_mix(embedded_context: torch.Tensor, scales: Sequence[torch.Tensor],
                    embedded_token_shift: Optional[torch.Tensor] = None,
                    batch_ids: Optional[torch.Tensor] = None,
                    context_mask: Optional[torch.Tensor] = None,
                    out_dtype: Optional[torch.dtype] = None,
                    return_next_token_shift: bool = False):
    """``mix_i = x + token_shift_diff(x) * scales[i]`` for each scale
    ([1, 1, C] or [C], fp32), differentiable in x, the scales and the
    external shift. ``embedded_token_shift`` is [full_batch, C] (rows picked
    by ``batch_ids``, default arange(batch); None = zeros). Returns the tuple
    of mixes, and with ``return_next_token_shift`` also the next shift
    ([full_batch, C], a new buffer with the active slots updated, not
    differentiable)."""
    x = _gpu(embedded_context, "embedded_context")
    if x.dim() != 3:
        raise ValueError("embedded_context must be [batch, context_len, embedded_dim]")
    B, T, C = x.shape
    if len(scales) > MAX_MIXES:
        raise ValueError(f"at most {MAX_MIXES} mixes")
    if not scales and not return_next_token_shift:
        raise ValueError("nothing to compute: no scales and no next token shift")
    sc = (torch.stack([s.reshape(C) for s in scales]).float().contiguous() if scales
          else torch.zeros((0, C), dtype=torch.float32, device=x.device))
    shift = None
    if embedded_token_shift is not None:
        shift = _gpu(embedded_token_shift, "embedded_token_shift").to(x.dtype)
        if shift.dim() != 2 or shift.shape[1] != C:
            raise ValueError("embedded_token_shift must be [full_batch, embedded_dim]")
    ids = None
    if batch_ids is not None:
        ids = batch_ids.to(device=x.device, dtype=torch.int32).contiguous()
        if ids.shape != (B,):
            raise ValueError("batch_ids must be [batch]")
    mask = None
    if context_mask is not None:
        mask = context_mask.to(device=x.device, dtype=x.dtype).contiguous()
        if mask.shape != (B, T):
            raise ValueError("context_mask must be [batch, context_len]")
    out_dtype = out_dtype or x.dtype
    outs = _TokenShiftMix.apply(x, sc, shift, ids, mask, out_dtype, bool(return_next_token_shift))
    if isinstance(outs, torch.Tensor):
        outs = (outs,)
    if return_next_token_shift:
        return tuple(outs[:-1]), outs[-1]
    return tuple(outs)


# -------------------------------------------------------------- gated readout
class _GatedReadout(torch.autograd.Function):
    @staticmethod
    def forward(ctx, y, r, k, v, gate, bonus, weight, bias, eps):
        B, T, H, N = y.shape
        out = torch.empty((B, T, H * N), dtype=gate.dtype, device=y.device)
        _native.call("rwkv_gated_readout_forward", _ptr(y), _ptr(r), _ptr(k), _ptr(v), _ptr(gate),
                     _ptr(bonus), _ptr(weight), _ptr(bias), float(eps), B * T, H, N,
                     _code(y.dtype), _code(gate.dtype), _ptr(out), _stream(y.device))
        ctx.save_for_backward(y, r, k, v, gate, bonus, weight, bias)
        ctx.eps = eps
        return out

    @staticmethod
    def backward(ctx, dout):
        y, r, k, v, gate, bonus, weight, bias = ctx.saved_tensors
        B, T, H, N = y.shape
        dev = y.device
        dout = dout.to(gate.dtype).contiguous()
        dy, dr, dk, dv = (torch.empty_like(t) for t in (y, r, k, v))
        dgate = torch.empty_like(gate)
        dbonus = torch.empty_like(bonus)
        dweight = torch.empty_like(weight)
        dbias = torch.empty_like(bias)
        nbytes = _native.lib().rwkv_gated_readout_workspace_bytes(B * T, H, N)
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev)
        _native.call("rwkv_gated_readout_backward", _ptr(y), _ptr(r), _ptr(k), _ptr(v), _ptr(gate),
                     _ptr(bonus), _ptr(weight), _ptr(bias), float(ctx.eps), B * T, H, N,
                     _code(y.dtype), _code(gate.dtype), _ptr(dout), _ptr(dy), _ptr(dr), _ptr(dk),
                     _ptr(dv), _ptr(dgate), _ptr(dbonus), _ptr(dweight), _ptr(dbias), _ptr(ws),
                     nbytes, _stream(dev))
        return dy, dr, dk, dv, dgate, dbonus, dweight, dbias, None


def gated_readout(wkv7_output: torch.Tensor, receptance: torch.Tensor,
                  replacement_key: torch.Tensor, value: torch.Tensor, gate: torch.Tensor,
                  receptance_key_bonus: torch.Tensor, group_norm_weight: torch.Tensor,
                  group_norm_bias: torch.Tensor, eps: float = 64e-5) -> torch.Tensor:
    """``(GroupNorm_heads(y) + (r k~ bonus).sum(-1) v) * gate`` as
    gated_readout.rs:126-145 computes it before the output projection.
    y, r, k~, v are [B, T, H, 64] in one dtype; gate is [B, T, H*64] and sets
    the output dtype; the parameters are fp32 ([H, 64], [H*64], [H*64])."""
    y, r, k, v = (_gpu(t, "operand") for t in (wkv7_output, receptance, replacement_key, value))
    if y.dim() != 4 or any(t.shape != y.shape or t.dtype != y.dtype for t in (r, k, v)):
        raise ValueError("y, r, k, v must share one [B, T, H, 64] shape and dtype")
    B, T, H, N = y.shape
    g = _gpu(gate, "gate")
    if g.shape != (B, T, H * N):
        raise ValueError("gate must be [B, T, H * 64]")
    bonus = _gpu(receptance_key_bonus, "bonus")
    w = _gpu(group_norm_weight, "weight")
    b = _gpu(group_norm_bias, "bias")
    if bonus.dtype != torch.float32 or w.dtype != torch.float32 or b.dtype != torch.float32:
        raise TypeError("receptance_key_bonus and the group-norm parameters must be float32")
    if bonus.shape != (H, N) or w.shape != (H * N,) or b.shape != (H * N,):
        raise ValueError("parameter shapes must be [H, 64], [H * 64], [H * 64]")
    return _GatedReadout.apply(y, r, k, v, g, bonus, w, b, eps)


class _WeightPrepareEnd(torch.autograd.Function):
    @staticmethod
    def forward(ctx, key, value, value_first, lr, wd, vr, lr_bias, wd_bias, vr_bias,
                key_replacement, key_removal, num_heads, out_dtype):
        B, T, C = key.shape
        outs = [torch.empty((B, T, C), dtype=out_dtype, device=key.device) for _ in range(5)]
        _native.call("rwkv_weight_prepare_forward", _ptr(key), _ptr(value), _ptr(value_first),
                     _ptr(lr), _ptr(wd), _ptr(vr), _ptr(lr_bias), _ptr(wd_bias), _ptr(vr_bias),
                     _ptr(key_replacement), _ptr(key_removal), B * T, num_heads, C // num_heads,
                     _code(key.dtype), _code(out_dtype), *[_ptr(t) for t in outs],
                     _stream(key.device))
        ctx.save_for_backward(key, value, value_first, lr, wd, vr, lr_bias, wd_bias, vr_bias,
                              key_replacement, key_removal)
        ctx.num_heads, ctx.out_dtype = num_heads, out_dtype
        return tuple(outs)

    @staticmethod
    def backward(ctx, *grads):
        key, value, value_first, lr, wd, vr, lr_bias, wd_bias, vr_bias, ka, kk = ctx.saved_tensors
        B, T, C = key.shape
        H = ctx.num_heads
        dev = key.device
        g = [torch.zeros((B, T, C), dtype=ctx.out_dtype, device=dev) if d is None
             else d.to(ctx.out_dtype).contiguous() for d in grads]
        res = vr_bias is not None
        dkey, dvalue, dlr, dwd = (torch.empty_like(t) for t in (key, value, lr, wd))
        dvf = torch.empty_like(value_first) if res else None
        dvr = torch.empty_like(vr) if res else None
        dlr_b, dwd_b, dka, dkk = (torch.empty_like(t) for t in (lr_bias, wd_bias, ka, kk))
        dvr_b = torch.empty_like(vr_bias) if res else None
        nbytes = _native.lib().rwkv_weight_prepare_workspace_bytes(B * T, H, C // H)
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device=dev)
        _native.call("rwkv_weight_prepare_backward", _ptr(key), _ptr(value), _ptr(value_first),
                     _ptr(lr), _ptr(wd), _ptr(vr), _ptr(lr_bias), _ptr(wd_bias), _ptr(vr_bias),
                     _ptr(ka), _ptr(kk), B * T, H, C // H, _code(key.dtype),
                     _code(ctx.out_dtype), *[_ptr(t) for t in g], _ptr(dkey), _ptr(dvalue),
                     _ptr(dvf), _ptr(dlr), _ptr(dwd), _ptr(dvr), _ptr(dlr_b), _ptr(dwd_b),
                     _ptr(dvr_b), _ptr(dka), _ptr(dkk), _ptr(ws), nbytes, _stream(dev))
        return (dkey, dvalue, dvf, dlr, dwd, dvr, dlr_b, dwd_b, dvr_b, dka, dkk, None, None)


def weight_prepare_end(key_precursor: torch.Tensor, value_precursor: torch.Tensor,
                       value_from_first_cell: Optional[torch.Tensor],
                       learning_rate_lora: torch.Tensor, weight_decay_lora: torch.Tensor,
                       value_residual_lora: Optional[torch.Tensor],
                       learning_rate_bias: torch.Tensor, weight_decay_bias: torch.Tensor,
                       value_residual_bias: Optional[torch.Tensor],
                       key_replacement: torch.Tensor, key_removal: torch.Tensor,
                       num_heads: int, out_dtype: Optional[torch.dtype] = None):
    """The tail of WeightPrepare::forward (weight_prepare.rs:282-317) on one
    kernel: returns ``(weight_decay, replacement_key, value,
    removal_key_normalized, replacement)`` as [B, T, C] in ``out_dtype``
    (default: the inputs' dtype).

    The [B, T, C] inputs share one dtype: the key and value projections and
    the three LoRA products before their bias (``LoRA.product``). The biases
    and ``key_replacement`` / ``key_removal`` are fp32 with C elements (any
    shape). The value residual (``value_from_first_cell``,
    ``value_residual_lora`` and its bias) is given for every cell but the
    first, or not at all."""
    key = _gpu(key_precursor, "key_precursor")
    if key.dim() != 3:
        raise ValueError("key_precursor must be [B, T, C]")
    B, T, C = key.shape
    if num_heads <= 0 or C != num_heads * 64:
        raise ValueError("C must be num_heads * 64")
    res = (value_from_first_cell, value_residual_lora, value_residual_bias)
    if any(t is None for t in res) and not all(t is None for t in res):
        raise ValueError("the value residual needs value_from_first_cell, value_residual_lora "
                         "and value_residual_bias together")
    acts = [key] + [None if t is None else _gpu(t, "activation") for t in
                    (value_precursor, value_from_first_cell, learning_rate_lora,
                     weight_decay_lora, value_residual_lora)]
    for t in acts:
        if t is not None and (t.shape != key.shape or t.dtype != key.dtype):
            raise ValueError("the [B, T, C] inputs must share one shape and dtype")
    params = []
    for t in (learning_rate_bias, weight_decay_bias, value_residual_bias, key_replacement,
              key_removal):
        if t is None:
            params.append(None)
            continue
        t = _gpu(t, "parameter")
        if t.dtype != torch.float32 or t.numel() != C:
            raise ValueError("biases and key_replacement / key_removal must be fp32 with C elements")
        params.append(t.reshape(C))
    out_dtype = key.dtype if out_dtype is None else out_dtype
    _code(out_dtype)
    return _WeightPrepareEnd.apply(*acts, *params, num_heads, out_dtype)
