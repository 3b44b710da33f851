"""RWKV-7 language-model training step on the host framework (PyTorch-ROCm),
with the WKV7 recurrence on the gfx950 kernels through ``wkv7``.

This is the caller of the operator: every module mirrors an rwkv-nn module
(names, argument meaning, the order of the operations), with torch ops in place
of Burn's, and the WKV7 operator passed in as ``kernel`` the way the reference
passes its ``K: Wkv7Kernel<B>`` type parameter:

* ``LoRA``            -- layers/lora.rs:105-124
* ``token_shift_diff``-- kernels/token_shift_diff/kernel.rs:17-64 (one lane's
  shift buffer is the caller's ``embedded_token_shift`` row, as in training,
  where batch_ids = arange(batch))
* ``addcmul``/``addcmul5`` -- kernels/addcmul/kernel.rs:4-53
* ``WeightPrepare``   -- modules/time_mixer/weight_prepare.rs:210-332
* ``GatedReadout``    -- modules/time_mixer/gated_readout.rs:110-148
* ``TimeMixer``       -- modules/time_mixer/mod.rs:153-217 (LoRA ranks :23-84)
* ``ChannelMixer``    -- modules/channel_mixer/mod.rs:83-121
* ``CausalCell`` / ``MultiCausalCells`` -- cells/causal.rs:67-149,226-268
* ``AutoRegressiveModel`` -- examples/rwkv-lm/src/model.rs:56-176, with
  ``l2wrap`` (kernels/l2wrap/mod.rs) before the mean cross entropy
* ``train_step``      -- the pretrain ``TrainStep::step`` (model.rs:316-324)
  followed by the optimizer update (Adam betas (0.9, 0.99), eps 1e-16,
  training.rs:164-177)

The ops on either side of the operator run, by default
(``neighbor_ops="hip"``), as the fused kernels of ``neighbors``: the token
shift with the five mixes and the readout gate's mix in one pass, the
GroupNorm + bonus + gate readout in another (the gate's mix, x + diff *
param_gate, moves from GatedReadout into that first pass). With
``neighbor_ops="torch"`` they are the plain torch formulations below, kept as
the readable mirror of the reference and as the reference the fused kernels
are tested against.

Weights are random N(0, 0.02) (normalisation layers start at one and zero);
the reference's shape-aware initialiser is not needed to time or check a step.
Matrix products run in bfloat16 under autocast with float32 master weights;
the six WKV7 operands are handed to the operator in ``wkv7_dtype`` (bfloat16
by default: bf16 inputs, float32 state and accumulation in the kernels).
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import List, Optional

import torch
import torch.nn as nn
import torch.nn.functional as F

from . import lm_loss as _loss
from . import neighbors as _nb
from . import wkv7 as _wkv7

CHUNK_LEN = 16                 # time_mixer/mod.rs:190
GROUP_NORM_EPS = 64e-5         # gated_readout.rs:48-50
MIN_LORA_RANK = 32             # time_mixer/mod.rs:20-21
LORA_RANK_GRANULARITY = 32


# ------------------------------------------------------------------ LoRA ranks
@dataclass(frozen=True)
class LoRARanks:
    """layers/lora.rs:157-163"""
    weight_decay_lora: int
    learning_rate_lora: int
    value_residual_lora: int
    output_gate_lora: int


def infer_lora_rank_from_formula(value: float) -> int:
    """time_mixer/mod.rs:39-44: nearest multiple of 32 (ties to even), at
    least 32. Python's ``round`` rounds halves to even, like ``round_ties_even``."""
    return max(int(round(value / LORA_RANK_GRANULARITY)) * LORA_RANK_GRANULARITY, MIN_LORA_RANK)


_OVERRIDE_RANKS = {                 # time_mixer/mod.rs:65-75
    (12, 768): (64, 64, 32, 128),
    (24, 1024): (64, 64, 32, 128),
    (24, 2048): (96, 96, 64, 256),
    (32, 2560): (96, 96, 64, 320),
    (32, 4096): (128, 128, 96, 480),
    (61, 4096): (192, 192, 128, 384),
}


def infer_time_mixer_lora_ranks(num_cells: int, embedded_dim: int, head_size: int) -> LoRARanks:
    """time_mixer/mod.rs:46-84: the published table for known model shapes,
    else the sqrt(C) formula scaled by head_size / 64."""
    if (num_cells, embedded_dim) in _OVERRIDE_RANKS:
        return LoRARanks(*_OVERRIDE_RANKS[(num_cells, embedded_dim)])
    root = float(embedded_dim) ** 0.5
    factor = head_size / 64.0
    return LoRARanks(
        infer_lora_rank_from_formula(2.5 * root * factor),
        infer_lora_rank_from_formula(2.5 * root * factor),
        infer_lora_rank_from_formula(1.7 * root * factor),
        infer_lora_rank_from_formula(5.0 * root),
    )


NEIGHBOR_OPS = ("hip", "torch")


def _check_neighbor_ops(neighbor_ops: str) -> str:
    if neighbor_ops not in NEIGHBOR_OPS:
        raise ValueError(f"neighbor_ops must be one of {NEIGHBOR_OPS}, got {neighbor_ops!r}")
    return neighbor_ops


def _matmul_dtype(x: torch.Tensor) -> torch.dtype:
    """The dtype a matrix product reading x computes in: autocast's, else x's."""
    dt = x.device.type
    if torch.is_autocast_enabled(dt):
        return torch.get_autocast_dtype(dt)
    return x.dtype


# ------------------------------------------------------------- element-wise ops
def apply_context_mask(x: torch.Tensor, context_mask: Optional[torch.Tensor]) -> torch.Tensor:
    """functions/context_mask.rs:8-26: masked steps become exact zeros."""
    if context_mask is None:
        return x
    return x * context_mask.to(x.dtype).unsqueeze(2)


def token_shift_diff(embedded_context: torch.Tensor,
                     embedded_token_shift: Optional[torch.Tensor] = None,
                     context_mask: Optional[torch.Tensor] = None,
                     batch_ids: Optional[torch.Tensor] = None):
    """token_shift_diff/kernel.rs:17-64.

    ``diff[t] = prev[t] - x[t]`` where ``prev[t]`` is ``x[t-1]`` when step t-1
    is valid and the external shift otherwise (also at t = 0); masked steps
    give zero. The next shift is ``x`` at the last valid step, or the external
    shift when no step is valid. With ``batch_ids`` the external shift is a
    [full_batch, C] buffer whose row ``batch_ids[b]`` belongs to row b, and
    the next shift is that buffer with those rows replaced. Returns
    ``(token_shifted_diff, next_token_shift)``."""
    B, T, C = embedded_context.shape
    if batch_ids is not None and embedded_token_shift is not None:
        ids = batch_ids.to(device=embedded_token_shift.device, dtype=torch.long)
        diff, rows = token_shift_diff(embedded_context, embedded_token_shift[ids], context_mask)
        full = embedded_token_shift.clone()
        full[ids] = rows.to(full.dtype)
        return diff, full
    ext = (embedded_token_shift if embedded_token_shift is not None
           else embedded_context.new_zeros(B, C))
    if T == 0:
        return embedded_context, ext
    prev = torch.cat([ext.unsqueeze(1), embedded_context[:, :-1]], dim=1)
    if context_mask is None:
        return prev - embedded_context, embedded_context[:, -1]
    m = context_mask.to(embedded_context.dtype)
    prev_valid = torch.cat([m.new_zeros(B, 1), m[:, :-1]], dim=1).unsqueeze(2)
    prev = prev_valid * prev + (1.0 - prev_valid) * ext.unsqueeze(1)
    diff = m.unsqueeze(2) * (prev - embedded_context)
    steps = torch.arange(1, T + 1, device=m.device, dtype=m.dtype)
    last = (m * steps).max(dim=1).values.long()            # 0 = no valid step
    picked = embedded_context[torch.arange(B, device=m.device), (last - 1).clamp(min=0)]
    next_shift = torch.where((last > 0).unsqueeze(1), picked, ext)
    return diff, next_shift


def addcmul(base: torch.Tensor, diff: torch.Tensor, scale: torch.Tensor) -> torch.Tensor:
    """addcmul/kernel.rs:4-19: base + diff * scale[channel]."""
    return base + diff * scale


def addcmul5(base, diff, receptance_scale, weight_decay_scale, key_scale, value_scale,
             learning_rate_scale):
    """addcmul/kernel.rs:21-53: the five token-shift mixes of one input."""
    return tuple(base + diff * s for s in (receptance_scale, weight_decay_scale, key_scale,
                                           value_scale, learning_rate_scale))


class _L2Wrap(torch.autograd.Function):
    """kernels/l2wrap/mod.rs: identity forward; the backward adds
    1e-4 / num_tokens * max(logits) at each row's argmax."""

    @staticmethod
    def forward(ctx, logits, num_tokens_per_batch):
        ctx.save_for_backward(logits)
        ctx.num_tokens = num_tokens_per_batch
        return logits.view_as(logits)

    @staticmethod
    def backward(ctx, grad):
        (logits,) = ctx.saved_tensors
        if ctx.num_tokens == 0:
            return grad, None
        max_vals, max_ids = logits.max(dim=-1, keepdim=True)
        grad = grad.clone()
        grad.scatter_add_(-1, max_ids, (max_vals * (1e-4 / ctx.num_tokens)).to(grad.dtype))
        return grad, None


def l2wrap(logits: torch.Tensor, num_tokens_per_batch: int) -> torch.Tensor:
    return _L2Wrap.apply(logits, num_tokens_per_batch)


# --------------------------------------------------------------------- modules
def _param(*shape) -> nn.Parameter:
    return nn.Parameter(torch.empty(*shape))


def _linear(d_in: int, d_out: int) -> nn.Linear:
    return nn.Linear(d_in, d_out, bias=False)


class LoRA(nn.Module):
    """layers/lora.rs:52-124: ``bias + act(x @ w_a) @ w_b``."""

    def __init__(self, embedded_dim: int, hidden_dim: int, has_bias: bool, activation: str):
        super().__init__()
        if activation not in ("sigmoid", "tanh", "none"):
            raise ValueError(f"unknown LoRA activation {activation!r}")
        self.w_a = _param(embedded_dim, hidden_dim)
        self.w_b = _param(hidden_dim, embedded_dim)
        self.bias = _param(1, 1, embedded_dim) if has_bias else None
        self.activation = activation

    def product(self, x: torch.Tensor) -> torch.Tensor:
        """``act(x @ w_a) @ w_b``: the LoRA without its bias."""
        h = x @ self.w_a
        if self.activation == "sigmoid":
            h = torch.sigmoid(h)
        elif self.activation == "tanh":
            h = torch.tanh(h)
        return h @ self.w_b

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = self.product(x)
        return h + self.bias if self.bias is not None else h


@dataclass
class WeightPrepareOutput:
    """weight_prepare.rs:333-344"""
    token_shifted_diff: torch.Tensor
    next_token_shift: torch.Tensor
    value_from_first_cell: torch.Tensor
    receptance: torch.Tensor
    weight_decay: torch.Tensor
    replacement_key: torch.Tensor
    value: torch.Tensor
    removal_key_normalized: torch.Tensor
    replacement: torch.Tensor
    gate_input: Optional[torch.Tensor] = None   # the readout gate's mix, when fused here

    def reshape_to_wkv7_input(self, shape, dtype: Optional[torch.dtype] = None):
        """weight_prepare.rs:346-356, plus the cast to the operator's dtype."""
        def f(t):
            t = t.reshape(shape)
            return t.to(dtype) if dtype is not None else t
        return _wkv7.Wkv7ForwardInput(
            receptance=f(self.receptance), weight_decay=f(self.weight_decay),
            replacement_key=f(self.replacement_key), value=f(self.value),
            removal_key_normalized=f(self.removal_key_normalized),
            replacement=f(self.replacement))


class WeightPrepare(nn.Module):
    """modules/time_mixer/weight_prepare.rs:28-131"""

    def __init__(self, num_cells, embedded_dim, num_heads, head_size, ranks: LoRARanks,
                 cell_id: int, neighbor_ops: str = "hip"):
        super().__init__()
        C = embedded_dim
        self.param_receptance = _param(1, 1, C)
        self.param_weight_decay = _param(1, 1, C)
        self.param_key = _param(1, 1, C)
        self.param_value = _param(1, 1, C)
        self.param_learning_rate = _param(1, 1, C)
        self.projection_receptance = _linear(C, C)
        self.projection_key = _linear(C, C)
        self.projection_value = _linear(C, C)
        self.param_weight_decay_lora = LoRA(C, ranks.weight_decay_lora, True, "tanh")
        self.param_learning_rate_lora = LoRA(C, ranks.learning_rate_lora, True, "none")
        self.param_value_residual_lora = (LoRA(C, ranks.value_residual_lora, True, "none")
                                          if cell_id > 0 else None)
        self.param_key_removal = _param(1, 1, C)
        self.param_key_replacement = _param(1, 1, C)
        self.num_heads, self.head_size, self.cell_id = num_heads, head_size, cell_id
        self.neighbor_ops = _check_neighbor_ops(neighbor_ops)

    def forward(self, embedded_context, value_from_first_cell, embedded_token_shift=None,
                context_mask=None, gate_scale: Optional[torch.Tensor] = None,
                operand_dtype: Optional[torch.dtype] = None,
                batch_ids: Optional[torch.Tensor] = None) -> WeightPrepareOutput:
        """weight_prepare.rs:210-330. With the HIP neighbour ops the token shift
        and the five mixes are one kernel, which also forms the readout gate's
        mix x + diff * ``gate_scale`` (gated_readout.rs:122) when it is given;
        the difference itself is then not materialised. ``batch_ids`` maps
        rows to the slots of a full-batch ``embedded_token_shift``
        (weight_prepare.rs:224-229). Everything after the
        projections and the LoRA products is a second kernel, which writes
        the five WKV7 operands it forms in ``operand_dtype`` (default: the
        products' dtype)."""
        B, T, C = embedded_context.shape
        scales = [self.param_receptance, self.param_weight_decay, self.param_key,
                  self.param_value, self.param_learning_rate]
        gate_input = None
        if self.neighbor_ops == "hip":
            want_next = embedded_token_shift is not None
            res = _nb.token_shift_mix(
                embedded_context, scales + ([gate_scale] if gate_scale is not None else []),
                embedded_token_shift, batch_ids, context_mask, _matmul_dtype(embedded_context),
                return_next_token_shift=want_next)
            mixes, next_shift = res if want_next else (res, None)
            xr, xw, xk, xv, xa = mixes[:5]
            if gate_scale is not None:
                gate_input = mixes[5]
            diff = None
        else:
            diff, next_shift = token_shift_diff(embedded_context, embedded_token_shift,
                                                context_mask, batch_ids)
            xr, xw, xk, xv, xa = addcmul5(embedded_context, diff, *scales)
        receptance = self.projection_receptance(xr)
        key_precursor = self.projection_key(xk)
        value_precursor = self.projection_value(xv)
        if self.cell_id == 0:
            value_from_first_cell = value_precursor
        if self.neighbor_ops == "hip":
            first = self.cell_id == 0
            vr_lora = self.param_value_residual_lora
            weight_decay, replacement_key, value, removal_key_normalized, replacement = \
                _nb.weight_prepare_end(
                    key_precursor, value_precursor, None if first else value_from_first_cell,
                    self.param_learning_rate_lora.product(xa),
                    self.param_weight_decay_lora.product(xw),
                    None if first else vr_lora.product(xv),
                    self.param_learning_rate_lora.bias, self.param_weight_decay_lora.bias,
                    None if first else vr_lora.bias, self.param_key_replacement,
                    self.param_key_removal, self.num_heads, operand_dtype)
            return WeightPrepareOutput(diff, next_shift, value_from_first_cell, receptance,
                                       weight_decay, replacement_key, value,
                                       removal_key_normalized, replacement, gate_input)
        learning_rate = torch.sigmoid(self.param_learning_rate_lora(xa))
        alpha_modulated = self.param_key_replacement * (learning_rate - 1.0) + 1.0
        replacement_key = key_precursor * alpha_modulated
        if self.cell_id != 0:
            nu = torch.sigmoid(self.param_value_residual_lora(xv))
            value = value_precursor + (value_from_first_cell - value_precursor) * nu   # lerp
        else:
            value = value_precursor
        weight_decay = -F.softplus(-self.param_weight_decay_lora(xw)) - 0.5
        removal_key = key_precursor * self.param_key_removal
        removal_key_normalized = -F.normalize(
            removal_key.reshape(B, T, self.num_heads, self.head_size), p=2.0, dim=-1,
            eps=1e-12).reshape(B, T, C)
        replacement = -removal_key_normalized * learning_rate
        return WeightPrepareOutput(diff, next_shift, value_from_first_cell, receptance,
                                   weight_decay, replacement_key, value,
                                   removal_key_normalized, replacement, gate_input)


class GatedReadout(nn.Module):
    """modules/time_mixer/gated_readout.rs:13-80"""

    def __init__(self, num_cells, embedded_dim, num_heads, head_size, ranks: LoRARanks,
                 cell_id: int, neighbor_ops: str = "hip"):
        super().__init__()
        C = embedded_dim
        self.param_gate = _param(1, 1, C)
        self.param_output_gate_lora = LoRA(C, ranks.output_gate_lora, False, "sigmoid")
        self.param_receptance_key_bonus = _param(num_heads, C // num_heads)
        self.group_norm = nn.GroupNorm(num_heads, C, eps=GROUP_NORM_EPS)
        self.projection_output = _linear(C, C)
        self.neighbor_ops = _check_neighbor_ops(neighbor_ops)

    def forward(self, embedded_context, token_shifted_diff, wkv7_forward_output,
                receptance, replacement_key, value,
                gate_input: Optional[torch.Tensor] = None) -> torch.Tensor:
        """gated_readout.rs:110-148; the operator's output and operands are
        [B, T, H, N]. ``gate_input`` is x + diff * param_gate when the token
        shift kernel already formed it."""
        B, T, C = embedded_context.shape
        if gate_input is None:
            gate_input = embedded_context + token_shifted_diff * self.param_gate
        gate = self.param_output_gate_lora(gate_input)
        if self.neighbor_ops == "hip":
            out = _nb.gated_readout(wkv7_forward_output, receptance, replacement_key, value,
                                    gate, self.param_receptance_key_bonus,
                                    self.group_norm.weight, self.group_norm.bias, GROUP_NORM_EPS)
            return self.projection_output(out)
        # the operator's output comes back in its operand dtype; the norm runs
        # in the residual stream's
        y = wkv7_forward_output.to(embedded_context.dtype).reshape(B * T, C)
        y = self.group_norm(y).reshape(B, T, C)
        bonus = ((receptance * replacement_key * self.param_receptance_key_bonus)
                 .sum(dim=3, keepdim=True) * value).reshape(B, T, C)
        return self.projection_output((y + bonus) * gate)


@dataclass
class TimeMixerIO:
    """time_mixer/mod.rs:220-228"""
    embedded_context: torch.Tensor
    batch_ids: torch.Tensor
    elapsed_t: Optional[torch.Tensor]
    context_mask: Optional[torch.Tensor]
    value_from_first_cell: torch.Tensor
    embedded_token_shift: Optional[torch.Tensor]
    state: Optional[torch.Tensor]


class TimeMixer(nn.Module):
    """modules/time_mixer/mod.rs:86-141"""

    def __init__(self, num_cells, embedded_dim, num_heads, head_size, cell_id: int,
                 wkv7_dtype: torch.dtype = torch.bfloat16, neighbor_ops: str = "hip"):
        super().__init__()
        ranks = infer_time_mixer_lora_ranks(num_cells, embedded_dim, head_size)
        self.weight_prepare = WeightPrepare(num_cells, embedded_dim, num_heads, head_size, ranks,
                                            cell_id, neighbor_ops)
        self.gated_readout = GatedReadout(num_cells, embedded_dim, num_heads, head_size, ranks,
                                          cell_id, neighbor_ops)
        self.neighbor_ops = _check_neighbor_ops(neighbor_ops)
        self.num_heads, self.head_size, self.cell_id = num_heads, head_size, cell_id
        self.wkv7_dtype = wkv7_dtype

    def forward(self, io: TimeMixerIO, kernel) -> TimeMixerIO:
        """time_mixer/mod.rs:153-217; ``kernel`` has the ``forward`` of the
        ``Wkv7Kernel`` implementations in ``wkv7`` (KernelPretrain, ...)."""
        return_shift = io.embedded_token_shift is not None
        B, T, _ = io.embedded_context.shape
        x = apply_context_mask(io.embedded_context, io.context_mask)
        v_first = apply_context_mask(io.value_from_first_cell, io.context_mask)
        gate_scale = self.gated_readout.param_gate if self.neighbor_ops == "hip" else None
        wp = self.weight_prepare(x, v_first, io.embedded_token_shift, io.context_mask, gate_scale,
                                 self.wkv7_dtype, io.batch_ids)
        shape = (B, T, self.num_heads, self.head_size)
        wkv_in = wp.reshape_to_wkv7_input(shape, self.wkv7_dtype)
        out = kernel.forward(wkv_in, io.state, io.batch_ids, io.elapsed_t, CHUNK_LEN,
                             io.context_mask)
        y = self.gated_readout(x, wp.token_shifted_diff, out.output, wkv_in.receptance,
                               wkv_in.replacement_key, wkv_in.value, wp.gate_input)
        return TimeMixerIO(
            embedded_context=apply_context_mask(y, io.context_mask),
            batch_ids=io.batch_ids, elapsed_t=io.elapsed_t, context_mask=io.context_mask,
            value_from_first_cell=apply_context_mask(wp.value_from_first_cell, io.context_mask),
            embedded_token_shift=wp.next_token_shift if return_shift else None,
            state=out.next_state)


class ChannelMixer(nn.Module):
    """modules/channel_mixer/mod.rs:20-121"""

    def __init__(self, num_cells, embedded_dim, cell_id: int, neighbor_ops: str = "hip"):
        super().__init__()
        self.key = _linear(embedded_dim, embedded_dim * 4)
        self.value = _linear(embedded_dim * 4, embedded_dim)
        self.token_shift_diff_scale = _param(1, 1, embedded_dim)
        self.neighbor_ops = _check_neighbor_ops(neighbor_ops)

    def forward(self, embedded_context, embedded_token_shift=None, context_mask=None,
                batch_ids=None):
        """channel_mixer/mod.rs:83-121 (the token shift by slot, :84-88); returns
        (output, next_token_shift or None)."""
        return_shift = embedded_token_shift is not None
        x = apply_context_mask(embedded_context, context_mask)
        if self.neighbor_ops == "hip":
            res = _nb.token_shift_mix(x, [self.token_shift_diff_scale], embedded_token_shift,
                                      batch_ids, context_mask, _matmul_dtype(x),
                                      return_next_token_shift=return_shift)
            (mixed,), next_shift = res if return_shift else (res, None)
        else:
            diff, next_shift = token_shift_diff(x, embedded_token_shift, context_mask, batch_ids)
            mixed = addcmul(x, diff, self.token_shift_diff_scale)
        # relu(.)^2 (channel_mixer/mod.rs:108) as a product: autocast runs pow
        # in fp32 (a cast up, then one back for the value projection, and the
        # same in the backward), a product stays in the matmul dtype; the
        # square of a bf16 value is exact in fp32, so both round it once
        r = torch.relu(self.key(mixed))
        k = r * r
        out = apply_context_mask(self.value(k), context_mask)
        return out, (next_shift if return_shift else None)


class CausalCell(nn.Module):
    """cells/causal.rs:166-268: pre-norm time mixer and channel mixer, each
    added to the residual stream."""

    def __init__(self, num_cells, embedded_dim, num_heads, head_size, cell_id: int,
                 wkv7_dtype: torch.dtype = torch.bfloat16, neighbor_ops: str = "hip"):
        super().__init__()
        self.pre_layer_norm_for_time_mix = nn.LayerNorm(embedded_dim)
        self.pre_layer_norm_for_channel_mix = nn.LayerNorm(embedded_dim)
        self.time_mixer = TimeMixer(num_cells, embedded_dim, num_heads, head_size, cell_id,
                                    wkv7_dtype, neighbor_ops)
        self.channel_mixer = ChannelMixer(num_cells, embedded_dim, cell_id, neighbor_ops)

    def forward(self, x, batch_ids, elapsed_t, value_from_first_cell, state, shift_time,
                shift_channel, context_mask, kernel):
        tm = self.time_mixer(TimeMixerIO(self.pre_layer_norm_for_time_mix(x), batch_ids,
                                         elapsed_t, context_mask, value_from_first_cell,
                                         shift_time, state), kernel)
        x = x + tm.embedded_context
        cm, next_shift_channel = self.channel_mixer(self.pre_layer_norm_for_channel_mix(x),
                                                    shift_channel, context_mask, batch_ids)
        x = x + cm
        return x, tm.value_from_first_cell, tm.state, tm.embedded_token_shift, next_shift_channel


class MultiCausalCells(nn.Module):
    """cells/causal.rs:21-158: the cells in order; the first cell's value
    precursor feeds every later cell's value residual."""

    def __init__(self, num_cells, embedded_dim, num_heads, head_size,
                 wkv7_dtype: torch.dtype = torch.bfloat16, neighbor_ops: str = "hip"):
        super().__init__()
        self.cells = nn.ModuleList(
            CausalCell(num_cells, embedded_dim, num_heads, head_size, i, wkv7_dtype, neighbor_ops)
            for i in range(num_cells))

    def forward(self, x, batch_ids, kernel, elapsed_t=None, context_mask=None,
                shift_time: Optional[List[torch.Tensor]] = None,
                state: Optional[List[torch.Tensor]] = None,
                shift_channel: Optional[List[torch.Tensor]] = None):
        x = apply_context_mask(x, context_mask)
        v_first = torch.zeros_like(x)
        shift_time = list(shift_time) if shift_time is not None else None
        state = list(state) if state is not None else None
        shift_channel = list(shift_channel) if shift_channel is not None else None
        for i, cell in enumerate(self.cells):
            x, v_first, s, st, sc = cell(
                x, batch_ids, elapsed_t, v_first,
                state[i] if state is not None else None,
                shift_time[i] if shift_time is not None else None,
                shift_channel[i] if shift_channel is not None else None,
                context_mask, kernel)
            if shift_time is not None:
                shift_time[i] = st
            if state is not None:
                state[i] = s
            if shift_channel is not None:
                shift_channel[i] = sc
        return x, shift_time, state, shift_channel


class AutoRegressiveModel(nn.Module):
    """examples/rwkv-lm/src/model.rs:50-176: embedding, layer norm, the
    cells, layer norm, unembedding, l2wrap and mean cross entropy."""

    def __init__(self, vocab_size: int, num_cells: int, embedded_dim: int, num_heads: int,
                 head_size: int = 64, wkv7_dtype: torch.dtype = torch.bfloat16,
                 neighbor_ops: str = "hip"):
        super().__init__()
        if embedded_dim != num_heads * head_size:
            raise ValueError("embedded_dim must equal num_heads * head_size")
        self.embed = nn.Embedding(vocab_size, embedded_dim)
        self.layer_norm_for_first_cell = nn.LayerNorm(embedded_dim)
        self.cells = MultiCausalCells(num_cells, embedded_dim, num_heads, head_size, wkv7_dtype,
                                      neighbor_ops)
        self.layer_norm_for_unembed = nn.LayerNorm(embedded_dim)
        self.unembed = _linear(embedded_dim, vocab_size)
        self.vocab_size = vocab_size
        self.neighbor_ops = _check_neighbor_ops(neighbor_ops)

    def init_random(self, std: float = 0.02, generator: Optional[torch.Generator] = None):
        """Every weight N(0, std); LayerNorm and GroupNorm weights one and biases zero."""
        norms = (nn.LayerNorm, nn.GroupNorm)
        with torch.no_grad():
            norm_params = set()
            for m in self.modules():
                if isinstance(m, norms):
                    m.weight.fill_(1.0)
                    m.bias.zero_()
                    norm_params.update((id(m.weight), id(m.bias)))
            for p in self.parameters():
                if id(p) not in norm_params:
                    p.normal_(0.0, std, generator=generator)
        return self

    def new_infer_state(self, full_batch_size: int, device=None,
                        state_dtype: Optional[torch.dtype] = None) -> "InferState":
        """Zeroed per-slot buffers for ``full_batch_size`` slots.

        By default the WKV7 state has the operator's element type, as the
        reference keeps it in its backend's float type
        (wkv7_infer/kernel.rs:35-42): a bfloat16 model decodes with the
        reference's bf16 arithmetic and its dither. ``state_dtype=
        torch.float32`` keeps a bfloat16 model's states in fp32 instead: the
        decode then runs the reference's f32 kernel on the bf16 operands
        (exact fp32 values), without the dither, as the training path's fp32
        state does."""
        device = device if device is not None else self.embed.weight.device
        C = self.embed.weight.shape[1]
        H = self.cells.cells[0].time_mixer.num_heads
        N = self.cells.cells[0].time_mixer.head_size
        n = len(self.cells.cells)
        op_dtype = self.cells.cells[0].time_mixer.wkv7_dtype
        if state_dtype is None:
            state_dtype = op_dtype
        if state_dtype not in (torch.float32, torch.bfloat16):
            raise ValueError("state_dtype must be torch.float32 or torch.bfloat16")
        if state_dtype == torch.bfloat16 and op_dtype != torch.bfloat16:
            raise ValueError("a bfloat16 state needs the model's bfloat16 operator")

        def z(*shape, dtype=torch.float32):
            return torch.zeros(*shape, dtype=dtype, device=device)
        return InferState([z(full_batch_size, C) for _ in range(n)],
                          [z(full_batch_size, H, N, N, dtype=state_dtype) for _ in range(n)],
                          [z(full_batch_size, C) for _ in range(n)],
                          torch.zeros(full_batch_size, dtype=torch.int32, device=device))

    @torch.no_grad()
    def infer(self, contexts: torch.Tensor, batch_ids: torch.Tensor, infer_state: "InferState",
              context_mask: Optional[torch.Tensor] = None, unembed_mode: str = "last"):
        """model.rs:184-300: run ``contexts`` ([batch, T] token ids) through
        the cells on the decode kernel, reading and updating the slots
        ``batch_ids`` of ``infer_state`` in place (state, both token shifts),
        with ``infer_state.elapsed_t`` as the dither's step count (the
        caller advances it afterwards, ``InferState.advance``, as
        inferring.rs:276 does). ``context_mask`` ([batch, T], 0/1) marks
        valid steps; a masked step leaves its slot's state alone. Returns
        the logits of the last step ([batch, 1, vocab], "last"), of every
        step ("full") or None ("skip")."""
        if unembed_mode not in UNEMBED_MODES:
            raise ValueError(f"unembed_mode must be one of {UNEMBED_MODES}")
        B, T = contexts.shape
        if T == 0:
            raise ValueError("contexts must be non-empty")
        kernel = _wkv7.KernelInfer
        x = self.layer_norm_for_first_cell(self.embed(contexts))
        x, st, state, sc = self.cells(x, batch_ids, kernel, infer_state.elapsed_t, context_mask,
                                      infer_state.shift_time, infer_state.state,
                                      infer_state.shift_channel)
        infer_state.shift_time[:] = st
        infer_state.state[:] = state
        infer_state.shift_channel[:] = sc
        if unembed_mode == "skip":
            return None
        if unembed_mode == "last":
            x = x[:, T - 1:]
        return self.unembed(self.layer_norm_for_unembed(x))

    def forward(self, inputs: torch.Tensor, targets: torch.Tensor, kernel=None):
        """model.rs:121-176 with the pretrain kernel by default; returns the loss."""
        kernel = kernel if kernel is not None else _wkv7.KernelPretrain
        B, T = inputs.shape
        batch_ids = torch.arange(B, device=inputs.device)
        x = self.layer_norm_for_first_cell(self.embed(inputs))
        x, _, _, _ = self.cells(x, batch_ids, kernel)
        logits = self.unembed(self.layer_norm_for_unembed(x))
        n = B * T
        if self.neighbor_ops == "hip":
            return _loss.cross_entropy_l2wrap(logits.reshape(n, self.vocab_size), targets.reshape(n))
        logits = l2wrap(logits.reshape(n, self.vocab_size), n)
        return F.cross_entropy(logits.float(), targets.reshape(n))


# ------------------------------------------------------------------ inference
@dataclass
class InferState:
    """The per-slot buffers of a serving loop (examples/rwkv-lm/src/
    inferring.rs:100-180): for each cell the time- and channel-mix token
    shifts ([full_batch, C], fp32) and the WKV7 state ([full_batch, H, 64,
    64], in the operator's element type: bf16 for bf16 operands, where the
    decode kernel runs the reference's bf16 arithmetic and its dither), and
    each slot's elapsed_t (int32), the dither seed's step count."""
    shift_time: List[torch.Tensor]
    state: List[torch.Tensor]
    shift_channel: List[torch.Tensor]
    elapsed_t: torch.Tensor

    def advance(self, batch_ids: torch.Tensor, context_len: int,
                context_mask: Optional[torch.Tensor] = None) -> None:
        """inferring.rs:61-83: each slot's elapsed_t advances by its valid
        (unmasked) steps, saturating at the int32 maximum, so a left-padded
        prefill uses the dither seeds of the same prefill unpadded."""
        ids = batch_ids.to(device=self.elapsed_t.device, dtype=torch.long)
        if context_mask is None:
            valid = torch.full((ids.numel(),), context_len, dtype=torch.int64,
                               device=self.elapsed_t.device)
        else:
            valid = (context_mask != 0).sum(dim=1).to(self.elapsed_t.device)
        total = (self.elapsed_t[ids].to(torch.int64) + valid).clamp(max=2 ** 31 - 1)
        self.elapsed_t[ids] = total.to(torch.int32)

    def reset_slot(self, slot: int) -> None:
        """A new sequence in ``slot``: zero state and shifts, elapsed_t 0
        (inferring.rs:455-465)."""
        for t in self.shift_time + self.state + self.shift_channel:
            t[slot].zero_()
        self.elapsed_t[slot] = 0


UNEMBED_MODES = ("skip", "last", "full")


def make_optimizer(model: nn.Module, lr: float = 6e-4, weight_decay: float = 0.1):
    """Adam with betas (0.9, 0.99) and eps 1e-16 (training.rs:164-177); decoupled
    weight decay on the matrices only."""
    decay = [p for p in model.parameters() if p.dim() >= 2]
    other = [p for p in model.parameters() if p.dim() < 2]
    groups = [{"params": decay, "weight_decay": weight_decay},
              {"params": other, "weight_decay": 0.0}]
    fused = all(p.is_cuda for p in model.parameters())
    return torch.optim.AdamW(groups, lr=lr, betas=(0.9, 0.99), eps=1e-16, fused=fused or None)


def train_step(model: AutoRegressiveModel, optimizer, inputs, targets, kernel=None,
               autocast: bool = True, check_faults: bool = False) -> torch.Tensor:
    """One pretrain step: forward, loss, backward, optimizer update
    (model.rs:316-324). Returns the detached loss. With ``check_faults`` the
    step ends by waiting for the device and raising ``Wkv7Error`` if a
    chunked forward of the step gave up a hand-over wait (its outputs, and so
    the loss, are then NaN); without it the step stays asynchronous and the
    caller polls ``wkv7.check_faults`` where it synchronises anyway."""
    device_type = inputs.device.type
    with torch.autocast(device_type, dtype=torch.bfloat16, enabled=autocast):
        loss = model(inputs, targets, kernel)
    loss.backward()
    optimizer.step()
    optimizer.zero_grad(set_to_none=True)
    if check_faults and inputs.is_cuda:
        _wkv7.check_faults(inputs.device)
    return loss.detach()
