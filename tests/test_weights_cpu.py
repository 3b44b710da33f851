"""CPU tests of the release-checkpoint loader (rwkv-rs_amd/weights.py), the
mirror of examples/rwkv-lm/src/pth2bpk.rs.

No release checkpoint ships with the reference and there is no network, so
the checkpoint here is synthetic (``model_helpers.release_checkpoint``): the
release format's key names and shapes, written out there and not taken from
the loader's table, filled with distinct random values, so that every tensor
can be traced to the parameter it lands in. Where tensors are traced only by
identity, a key mapped to the wrong one of two same-shaped parameters would
still pass; ``test_loaded_model_computes_the_release_forward`` closes that by
comparing the loaded model's logits with a float64 forward that reads the
checkpoint by its release key names (``model_helpers.release_forward_f64``)."""

import importlib

import pytest
import torch

from model_helpers import TorchKernel, _model_mod, model_logits, release_checkpoint as _release
from model_helpers import release_forward_f64


def _w():
    return importlib.import_module("rwkv-rs_amd.weights")


L, C, H, V = 2, 128, 2, 97
# the rank formula at C = 128: 2.5 sqrt(C) = 28 -> 32; 1.7 sqrt(C) = 19 -> 32; 5 sqrt(C) = 57 -> 64
RW, RA, RV, RG = 32, 32, 32, 64


def release_checkpoint(seed=0, dtype=torch.bfloat16, scaled=False):
    return _release(L, C, H, V, (RW, RA, RV, RG), seed, dtype, scaled)


def tiny(wkv7_dtype=torch.bfloat16):
    return _model_mod().AutoRegressiveModel(V, L, C, H, 64, wkv7_dtype=wkv7_dtype,
                                            neighbor_ops="torch")


CELL0_VALUE_RESIDUAL = {"blocks.0.att.v0", "blocks.0.att.v1", "blocks.0.att.v2"}


def test_every_release_tensor_lands_in_its_parameter(tmp_path):
    w = _w()
    sd = release_checkpoint()
    path = tmp_path / "tiny.pth"
    torch.save(sd, path)
    model = tiny()
    res = w.load_pth(model, str(path))
    assert res.missing == []
    assert set(res.unused) == {
        "cells.cells.0.time_mixer.weight_prepare.param_value_residual_lora." + n
        for n in ("bias", "w_a", "w_b")}
    params = dict(model.named_parameters())
    # a few correspondences written out in full
    expect = {
        "blocks.1.att.w1": "cells.cells.1.time_mixer.weight_prepare.param_weight_decay_lora.w_a",
        "blocks.1.att.a0": "cells.cells.1.time_mixer.weight_prepare.param_learning_rate_lora.bias",
        "blocks.1.att.v2": "cells.cells.1.time_mixer.weight_prepare.param_value_residual_lora.w_b",
        "blocks.0.att.g1": "cells.cells.0.time_mixer.gated_readout.param_output_gate_lora.w_a",
        "blocks.0.att.r_k": "cells.cells.0.time_mixer.gated_readout.param_receptance_key_bonus",
        "blocks.1.att.k_k": "cells.cells.1.time_mixer.weight_prepare.param_key_removal",
        "blocks.1.att.k_a": "cells.cells.1.time_mixer.weight_prepare.param_key_replacement",
        "blocks.0.att.x_g": "cells.cells.0.time_mixer.gated_readout.param_gate",
        "blocks.1.att.ln_x.bias": "cells.cells.1.time_mixer.gated_readout.group_norm.bias",
        "blocks.0.ffn.x_k": "cells.cells.0.channel_mixer.token_shift_diff_scale",
        "blocks.0.ln0.weight": "layer_norm_for_first_cell.weight",
        "ln_out.bias": "layer_norm_for_unembed.bias",
        "head.weight": "unembed.weight",
        "emb.weight": "embed.weight",
    }
    for key, path_ in expect.items():
        assert torch.equal(params[path_].detach(), sd[key].float()), key
    # and every release tensor (but cell 0's value residual) is in exactly one parameter
    used = [k for k in sd if k not in CELL0_VALUE_RESIDUAL]
    assert len(used) == len(params)
    for k in used:
        hits = [p for p, v in params.items()
                if tuple(v.shape) == tuple(sd[k].shape) and torch.equal(v.detach(), sd[k].float())]
        assert len(hits) == 1, (k, hits)


def test_missing_unknown_and_misshapen_tensors_are_refused():
    w = _w()
    sd = release_checkpoint()
    bad = dict(sd)
    del bad["blocks.1.att.k_a"]
    with pytest.raises(w.CheckpointMappingError, match="param_key_replacement"):
        w.load_pth(tiny(), bad)
    bad = dict(sd, **{"blocks.1.att.bogus": torch.zeros(3)})
    with pytest.raises(w.CheckpointMappingError, match="bogus"):
        w.load_pth(tiny(), bad)
    bad = dict(sd, **{"blocks.1.att.w1": torch.zeros(C, RW + 32)})
    with pytest.raises(w.CheckpointMappingError, match="errors: 1"):
        w.load_pth(tiny(), bad)
    # nothing was copied by a refused load; a lenient one applies what fits
    model = tiny()
    before = model.embed.weight.detach().clone()
    with pytest.raises(w.CheckpointMappingError):
        w.load_pth(model, bad)
    assert torch.equal(model.embed.weight.detach(), before)
    res = w.load_pth(model, bad, strict=False)
    assert res.errors and torch.equal(model.embed.weight.detach(), sd["emb.weight"].float())


def test_convert_then_load_equals_direct_load(tmp_path):
    w = _w()
    sd = release_checkpoint(seed=3)
    src, dst = tmp_path / "tiny.pth", tmp_path / "tiny.safetensors"
    torch.save(sd, src)
    cfg = dict(vocab_size=V, num_cells=L, embedded_dim=C, num_heads=H, head_size=64)
    w.convert_pth(str(src), str(dst), cfg)
    a, b = tiny(), tiny()
    w.load_pth(a, str(src))
    w.load_converted(b, str(dst))
    for (n, p), (_, q) in zip(a.named_parameters(), b.named_parameters()):
        assert torch.equal(p, q), n


def test_checkpoint_names_and_sizes():
    w = _w()
    p = w.parse_rwkv7_checkpoint("rwkv7-g1-0.1b-20250307-ctx4096")
    assert (p.data_version, p.model_size, p.date) == ("g1", "0.1b", "20250307")
    assert w.parse_rwkv7_checkpoint("rwkv6-world-1.6b-20240101") is None
    with pytest.raises(ValueError):
        w.parse_rwkv7_checkpoint("rwkv7-g1-0.1b-2025")
    with pytest.raises(ValueError):
        w.parse_rwkv7_checkpoint("rwkv7-g1")
    cfg = w.infer_model_config("0.1b")
    assert (cfg["num_cells"], cfg["embedded_dim"], cfg["num_heads"], cfg["vocab_size"]) == \
        (12, 768, 12, 65536)
    assert w.infer_model_config("7.2b")["num_heads"] == 64
    with pytest.raises(ValueError):
        w.infer_model_config("0.2b")


def test_release_lora_shapes_of_the_0_1b_model():
    """The 0.1B release stores w1/a1 as [768, 64], v1 as [768, 32] and g1 as
    [768, 128]; the model built from the size table must have those shapes."""
    w = _w()
    with torch.device("meta"):
        model = _model_mod().AutoRegressiveModel(**w.infer_model_config("0.1b"),
                                                 neighbor_ops="torch")
    tm = model.cells.cells[1].time_mixer
    assert tuple(tm.weight_prepare.param_weight_decay_lora.w_a.shape) == (768, 64)
    assert tuple(tm.weight_prepare.param_learning_rate_lora.w_a.shape) == (768, 64)
    assert tuple(tm.weight_prepare.param_value_residual_lora.w_a.shape) == (768, 32)
    assert tuple(tm.gated_readout.param_output_gate_lora.w_a.shape) == (768, 128)
    assert tuple(model.unembed.weight.shape) == (65536, 768)


def _logits_cpu(model, tokens):
    with torch.no_grad():
        return model_logits(model, tokens, TorchKernel).double()


def _rel(a, b):
    return float((a - b).norm() / b.norm())


def test_loaded_model_computes_the_release_forward():
    """The loaded model (torch neighbour ops, the float64 recurrence as the
    operator, fp32 weights) gives the logits of the release-key forward; the
    same model loaded from a checkpoint with two same-shaped LoRA factors
    swapped, or a square projection transposed, does not (a planted mapping
    mistake moves the logits by far more than the bar)."""
    w = _w()
    sd = release_checkpoint(seed=5, dtype=torch.float32, scaled=True)
    g = torch.Generator().manual_seed(9)
    toks = torch.randint(0, V, (2, 24), generator=g)
    want = release_forward_f64(sd, toks, H)
    model = tiny(torch.float32)
    w.load_pth(model, sd)
    err = _rel(_logits_cpu(model, toks), want)
    assert err <= 1e-5, err
    planted = {
        "lora factors swapped": dict(sd, **{"blocks.1.att.w1": sd["blocks.1.att.a1"],
                                            "blocks.1.att.a1": sd["blocks.1.att.w1"]}),
        "projection transposed": dict(sd, **{"blocks.0.att.key.weight":
                                             sd["blocks.0.att.key.weight"].T.contiguous()}),
        "mixes swapped": dict(sd, **{"blocks.0.att.x_r": sd["blocks.0.att.x_g"],
                                     "blocks.0.att.x_g": sd["blocks.0.att.x_r"]}),
    }
    for label, bad in planted.items():
        m = tiny(torch.float32)
        w.load_pth(m, bad)
        assert _rel(_logits_cpu(m, toks), want) > 1e-2, label
