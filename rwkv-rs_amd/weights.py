"""RWKV-7 checkpoints in the PyTorch ``.pth`` format of the public RWKV-7
releases, loaded into ``model.AutoRegressiveModel``.

Mirrors examples/rwkv-lm/src/pth2bpk.rs:57-264 (key remapping, the expected
missing and unused tensors, the error report) and the file-name parsing and
model-size table of examples/rwkv-lm/examples/rwkv-lm-pth2bpk.rs:59-136. The
model's parameter paths are the reference's module paths (``cells.cells.3.
time_mixer.weight_prepare.param_key`` ...), so the reference's remapping
table applies as is; the one difference is that Burn names norm parameters
``gamma``/``beta`` and torch ``weight``/``bias``. Linear weights are
[out, in] in both the checkpoint and torch, so nothing is transposed. Where
the reference writes a Burn ``.bpk``, ``convert_pth`` writes the remapped
tensors as safetensors.

Files are read with ``torch.load(..., weights_only=True)``, which executes
nothing from the file.
"""

from __future__ import annotations

import os
import re
from dataclasses import dataclass, field
from typing import Dict, List, Optional, Tuple

import torch

HEAD_SIZE = 64
VOCAB_SIZE = 65536

# (num_cells, embedded_dim) per released size, rwkv-lm-pth2bpk.rs:59-87
MODEL_SIZES = {
    "0.1b": (12, 768),
    "0.4b": (24, 1024),
    "1.5b": (24, 2048),
    "2.9b": (32, 2560),
    "7.2b": (32, 4096),
    "13.3b": (61, 4096),
}

_CELL = "cells.cells.{}."
_TM = _CELL + "time_mixer."
_WP = _TM + "weight_prepare."
_GR = _TM + "gated_readout."

# checkpoint key -> model parameter path, pth2bpk.rs:66-210 ("{}" = block index)
_GLOBAL_KEYS = {
    "emb.weight": "embed.weight",
    "blocks.0.ln0.weight": "layer_norm_for_first_cell.weight",
    "blocks.0.ln0.bias": "layer_norm_for_first_cell.bias",
    "ln_out.weight": "layer_norm_for_unembed.weight",
    "ln_out.bias": "layer_norm_for_unembed.bias",
    "head.weight": "unembed.weight",
}
_BLOCK_KEYS = {
    "ln1.weight": _CELL + "pre_layer_norm_for_time_mix.weight",
    "ln1.bias": _CELL + "pre_layer_norm_for_time_mix.bias",
    "ln2.weight": _CELL + "pre_layer_norm_for_channel_mix.weight",
    "ln2.bias": _CELL + "pre_layer_norm_for_channel_mix.bias",
    "att.receptance.weight": _WP + "projection_receptance.weight",
    "att.key.weight": _WP + "projection_key.weight",
    "att.value.weight": _WP + "projection_value.weight",
    "att.output.weight": _GR + "projection_output.weight",
    "att.ln_x.weight": _GR + "group_norm.weight",
    "att.ln_x.bias": _GR + "group_norm.bias",
    "att.k_k": _WP + "param_key_removal",
    "att.r_k": _GR + "param_receptance_key_bonus",
    "att.k_a": _WP + "param_key_replacement",
    "att.w0": _WP + "param_weight_decay_lora.bias",
    "att.w1": _WP + "param_weight_decay_lora.w_a",
    "att.w2": _WP + "param_weight_decay_lora.w_b",
    "att.a0": _WP + "param_learning_rate_lora.bias",
    "att.a1": _WP + "param_learning_rate_lora.w_a",
    "att.a2": _WP + "param_learning_rate_lora.w_b",
    "att.g1": _GR + "param_output_gate_lora.w_a",
    "att.g2": _GR + "param_output_gate_lora.w_b",
    "att.v0": _WP + "param_value_residual_lora.bias",
    "att.v1": _WP + "param_value_residual_lora.w_a",
    "att.v2": _WP + "param_value_residual_lora.w_b",
    "att.x_r": _WP + "param_receptance",
    "att.x_w": _WP + "param_weight_decay",
    "att.x_k": _WP + "param_key",
    "att.x_v": _WP + "param_value",
    "att.x_a": _WP + "param_learning_rate",
    "att.x_g": _GR + "param_gate",
    "ffn.key.weight": _CELL + "channel_mixer.key.weight",
    "ffn.value.weight": _CELL + "channel_mixer.value.weight",
    "ffn.x_k": _CELL + "channel_mixer.token_shift_diff_scale",
}
_BLOCK_RE = re.compile(r"^blocks\.([0-9]+)\.(.+)$")


def remap_key(key: str) -> Optional[str]:
    """The model parameter path of a checkpoint key, or None when the
    reference's table has no entry for it."""
    if key in _GLOBAL_KEYS:
        return _GLOBAL_KEYS[key]
    m = _BLOCK_RE.match(key)
    if m and m.group(2) in _BLOCK_KEYS:
        return _BLOCK_KEYS[m.group(2)].format(int(m.group(1)))
    return None


def is_expected_missing_tensor(path: str) -> bool:
    """pth2bpk.rs:58-60: the state-tuning state is not in a pretrained file."""
    return path.startswith("state.state.")


def is_expected_unused_tensor(path: str) -> bool:
    """pth2bpk.rs:62-64: the first cell has no value residual, but the
    released checkpoints carry one."""
    return path.startswith("cells.cells.0.time_mixer.weight_prepare.param_value_residual_lora.")


@dataclass
class LoadResult:
    """What ``load_pth`` applied, and what it left (model paths)."""
    applied: List[str] = field(default_factory=list)
    missing: List[str] = field(default_factory=list)   # model parameters with no tensor
    unused: List[str] = field(default_factory=list)    # checkpoint tensors with no parameter
    errors: List[str] = field(default_factory=list)    # shape mismatches


class CheckpointMappingError(ValueError):
    pass


def _report(result: LoadResult) -> str:
    """The message of pth2bpk.rs:235-264."""
    missing = [p for p in result.missing if not is_expected_missing_tensor(p)]
    unused = [p for p in result.unused if not is_expected_unused_tensor(p)]
    if not result.errors and not missing and not unused:
        return ""
    msg = "pth2bpk found unexpected tensor mapping issues:\n"
    if result.errors:
        msg += f"  - errors: {len(result.errors)}\n"
        for e in result.errors[:10]:
            msg += f"    * {e}\n"
    if missing:
        msg += f"  - unexpected missing tensors ({len(missing)}), first 10:\n"
        for p in missing[:10]:
            msg += f"    * {p}\n"
    if unused:
        msg += f"  - unexpected unused tensors ({len(unused)}), first 10:\n"
        for p in unused[:10]:
            msg += f"    * {p}\n"
    return msg


def read_pth(path: str) -> Dict[str, torch.Tensor]:
    """The checkpoint's tensors, read without executing anything from the file."""
    sd = torch.load(path, map_location="cpu", weights_only=True)
    if not isinstance(sd, dict) or not all(isinstance(v, torch.Tensor) for v in sd.values()):
        raise CheckpointMappingError(f"{path} does not hold a flat dict of tensors")
    return sd


def remap_state_dict(checkpoint: Dict[str, torch.Tensor]) -> Tuple[Dict[str, torch.Tensor], List[str]]:
    """Checkpoint keys -> model paths; keys the table does not know are
    returned by their own name as unmapped."""
    mapped, unmapped = {}, []
    for key, value in checkpoint.items():
        path = remap_key(key)
        if path is None:
            unmapped.append(key)
        else:
            mapped[path] = value
    return mapped, unmapped


def _match(checkpoint: Dict[str, torch.Tensor], params: Dict[str, torch.Tensor]):
    """Remaps the checkpoint and sorts its tensors against the model's
    parameters: the tensors that fit, and what is missing, unused or misshapen."""
    mapped, unmapped = remap_state_dict(checkpoint)
    result = LoadResult()
    result.unused = sorted(unmapped + [p for p in mapped if p not in params])
    result.missing = sorted(p for p in params if p not in mapped)
    fits = {}
    for path, value in mapped.items():
        if path not in params:
            continue
        if tuple(value.shape) != tuple(params[path].shape):
            result.errors.append(f"{path}: checkpoint {tuple(value.shape)}, "
                                 f"model {tuple(params[path].shape)}")
            continue
        fits[path] = value
    return result, fits


def load_pth(model: torch.nn.Module, checkpoint, strict: bool = True) -> LoadResult:
    """Copies the tensors of ``checkpoint`` (a path or a state dict in the
    release format) into ``model``'s parameters, converting the dtype.
    With ``strict`` (the reference's behaviour) unexpected missing or unused
    tensors and shape mismatches raise ``CheckpointMappingError``, and
    nothing is copied."""
    sd = read_pth(checkpoint) if isinstance(checkpoint, (str, os.PathLike)) else checkpoint
    params = dict(model.named_parameters())
    result, fits = _match(sd, params)
    msg = _report(result)
    if strict and msg:
        raise CheckpointMappingError(msg)
    with torch.no_grad():
        for path, value in fits.items():
            params[path].copy_(value.to(params[path].dtype))
    result.applied = sorted(fits)
    return result


# ------------------------------------------------------- file names and config
@dataclass(frozen=True)
class ParsedCheckpoint:
    """rwkv-lm-pth2bpk.rs:89-136: rwkv7-<data version>-<size>-<yyyymmdd>[-...]"""
    file_stem: str
    data_version: str
    model_size: str
    date: str


def parse_rwkv7_checkpoint(file_stem: str) -> Optional[ParsedCheckpoint]:
    """None for another architecture; ValueError for a malformed rwkv7 name."""
    parts = file_stem.split("-")
    if parts[0] != "rwkv7":
        return None
    if len(parts) < 4:
        raise ValueError(f"invalid rwkv7 checkpoint name: {file_stem}")
    data_version, model_size, date = parts[1], parts[2], parts[3]
    if len(date) != 8 or not date.isdigit():
        raise ValueError(f"invalid rwkv7 checkpoint date: {file_stem}")
    return ParsedCheckpoint(file_stem, data_version, model_size, date)


def infer_model_config(model_size: str) -> dict:
    """rwkv-lm-pth2bpk.rs:59-87: keyword arguments of AutoRegressiveModel."""
    if model_size not in MODEL_SIZES:
        raise ValueError(f"unsupported model size in file name: {model_size}")
    num_cells, embedded_dim = MODEL_SIZES[model_size]
    return dict(vocab_size=VOCAB_SIZE, num_cells=num_cells, embedded_dim=embedded_dim,
                num_heads=embedded_dim // HEAD_SIZE, head_size=HEAD_SIZE)


def convert_pth(model_path: str, output_path: str, model_config: Optional[dict] = None) -> LoadResult:
    """pth2bpk: checks a release checkpoint against the model its name (or
    ``model_config``) implies and writes the remapped tensors, in the
    checkpoint's dtype, as safetensors."""
    from safetensors.torch import save_file

    from .model import AutoRegressiveModel
    if model_config is None:
        stem = os.path.splitext(os.path.basename(model_path))[0]
        parsed = parse_rwkv7_checkpoint(stem)
        if parsed is None:
            raise ValueError(f"{stem}: arch_version is not rwkv7")
        model_config = infer_model_config(parsed.model_size)
    sd = read_pth(model_path)
    with torch.device("meta"):      # shapes only: the model holds no data
        model = AutoRegressiveModel(**model_config, neighbor_ops="torch")
    result, fits = _match(sd, dict(model.named_parameters()))
    msg = _report(result)
    if msg:
        raise CheckpointMappingError(msg)
    save_file({p: v.contiguous() for p, v in fits.items()}, output_path)
    result.applied = sorted(fits)
    return result


def load_converted(model: torch.nn.Module, path: str) -> None:
    """Loads a file written by ``convert_pth``; every parameter must be in
    it with its shape."""
    from safetensors.torch import load_file
    sd = load_file(path)
    params = dict(model.named_parameters())
    missing = sorted(set(params) - set(sd))
    extra = sorted(set(sd) - set(params))
    bad = [p for p in sd if p in params and tuple(sd[p].shape) != tuple(params[p].shape)]
    if missing or extra or bad:
        raise CheckpointMappingError(f"{path}: missing {missing[:10]}, unexpected {extra[:10]}, "
                                     f"shape mismatches {bad[:10]}")
    with torch.no_grad():
        for p, v in sd.items():
            params[p].copy_(v.to(params[p].dtype))
