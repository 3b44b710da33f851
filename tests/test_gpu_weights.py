"""GPU tests of a release-format RWKV-7 checkpoint driving the WKV7 operator:
``weights.load_pth`` (the mirror of examples/rwkv-lm/src/pth2bpk.rs:57-264)
loads a ``.pth`` file in the release format into ``model.AutoRegressiveModel``
(examples/rwkv-lm/src/model.rs:122-178), whose cells then run the HIP kernels
through the C ABI and the fused neighbour ops.

No release checkpoint ships with the reference and there is no network, so the
file is synthetic (``model_helpers.release_checkpoint``: the release key names
and shapes, values at well-conditioned scales), saved with ``torch.save`` in
bfloat16 as the releases are, and read back by ``load_pth`` from disk.

* The loaded model's logits equal a float64 forward that reads the checkpoint
  by its release key names with no key table (``release_forward_f64``), so a
  key mapped to the wrong one of two same-shaped parameters, or a transposed
  projection, fails here even where the shapes agree: fp32 operands (the fp32
  chunked kernels) within 1e-5 relative L2; bf16 operands under autocast (the
  bf16 chunked kernels) within 1e-2.
* Loss and every parameter gradient through ``KernelPretrain`` equal those of
  the same loaded model with a plain PyTorch recurrence as the operator: fp32
  loss 1e-5 and gradients 1e-4, bf16 loss 1e-3 and gradients 1e-2.
* ``infer`` on the loaded model (the decode kernel) gives the training path's
  logits for a whole prompt, and prefill plus token-by-token decode gives the
  same last logits (fp32 state, 1e-5).
"""

import importlib

import pytest
import torch

from conftest import announce, rel_l2
from model_helpers import (TorchKernel, _model_mod, _wkv7_mod, loss_and_grads, model_logits,
                           release_checkpoint, release_forward_f64)

pytestmark = pytest.mark.gpu
DEV = torch.device("cuda:0")

L, C, H, V = 2, 256, 4, 211
# the rank formula at C = 256: 2.5 sqrt(C) = 40 -> 32; 1.7 sqrt(C) = 27 -> 32; 5 sqrt(C) = 80 -> 64
RANKS = (32, 32, 32, 64)


def _weights():
    return importlib.import_module("rwkv-rs_amd.weights")


@pytest.fixture(scope="module")
def release_file(tmp_path_factory):
    sd = release_checkpoint(L, C, H, V, RANKS, seed=11, dtype=torch.bfloat16, scaled=True)
    path = tmp_path_factory.mktemp("release") / "rwkv7-synthetic-tiny.pth"
    torch.save(sd, path)
    return str(path), sd


def _loaded(path, wkv7_dtype, neighbor_ops="hip"):
    model = _model_mod().AutoRegressiveModel(V, L, C, H, 64, wkv7_dtype=wkv7_dtype,
                                             neighbor_ops=neighbor_ops)
    res = _weights().load_pth(model, path)
    assert res.missing == [] and len(res.unused) == 3     # cell 0's value residual
    return model.to(DEV)


def _tokens(B, T, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, V, (B, T + 1), generator=g).to(DEV)


def _err(a, b):
    return rel_l2(a.double().cpu().numpy(), b.double().cpu().numpy())


@pytest.mark.parametrize("wkv7_dtype,tol", [(torch.float32, 1e-5), (torch.bfloat16, 1e-2)],
                         ids=["fp32", "bf16"])
@pytest.mark.parametrize("neighbor_ops", ["hip", "torch"])
@torch.no_grad()
def test_release_checkpoint_logits_match_release_forward(release_file, wkv7_dtype, tol,
                                                        neighbor_ops):
    path, sd = release_file
    model = _loaded(path, wkv7_dtype, neighbor_ops)
    toks = _tokens(2, 64, 21)[:, :-1].contiguous()
    want = release_forward_f64(sd, toks, H)
    announce("release ckpt logits", str(wkv7_dtype), neighbor_ops)
    with torch.autocast("cuda", dtype=torch.bfloat16, enabled=wkv7_dtype == torch.bfloat16):
        got = model_logits(model, toks, _wkv7_mod().KernelPretrain)
    torch.cuda.synchronize()
    err = _err(got, want)
    print(f"[release ckpt {wkv7_dtype} {neighbor_ops}] logits rel-L2 vs release forward {err:.2e}")
    assert err <= tol, err


@pytest.mark.parametrize("wkv7_dtype,loss_tol,grad_tol",
                         [(torch.float32, 1e-5, 1e-4), (torch.bfloat16, 1e-3, 1e-2)],
                         ids=["fp32", "bf16"])
def test_release_checkpoint_train_step_matches_torch_recurrence(release_file, wkv7_dtype,
                                                                loss_tol, grad_tol):
    path, _ = release_file
    model = _loaded(path, wkv7_dtype)
    tok = _tokens(2, 64, 22)
    inputs, targets = tok[:, :-1].contiguous(), tok[:, 1:].contiguous()
    announce("release ckpt train step", str(wkv7_dtype), "torch recurrence")
    l0, g0 = loss_and_grads(model, TorchKernel, inputs, targets)
    announce("release ckpt train step", str(wkv7_dtype), "KernelPretrain")
    l1, g1 = loss_and_grads(model, _wkv7_mod().KernelPretrain, inputs, targets)
    torch.cuda.synchronize()
    assert abs(l1 - l0) <= loss_tol * abs(l0), (l0, l1)
    assert g0.keys() == g1.keys() and len(g0) == len(list(model.parameters()))
    errs = {n: _err(g1[n], g0[n]) for n in g0}
    worst = max(errs, key=errs.get)
    print(f"[release ckpt {wkv7_dtype}] loss {l0:.6f} vs {l1:.6f}; "
          f"worst grad {worst} {errs[worst]:.3e}")
    assert errs[worst] <= grad_tol, (worst, errs[worst])


@torch.no_grad()
def test_release_checkpoint_infer_matches_training_logits(release_file):
    path, _ = release_file
    model = _loaded(path, torch.float32)
    toks = _tokens(2, 48, 23)[:, :-1].contiguous()
    ids = torch.arange(2, device=DEV)
    announce("release ckpt infer", "whole prompt")
    st = model.new_infer_state(2)
    got = model.infer(toks, ids, st, unembed_mode="full")
    want = model_logits(model, toks, _wkv7_mod().KernelPretrain)
    torch.cuda.synchronize()
    assert _err(got, want) <= 1e-5
    announce("release ckpt infer", "prefill + decode")
    st2 = model.new_infer_state(2)
    model.infer(toks[:, :32], ids, st2, unembed_mode="skip")
    st2.advance(ids, 32)
    last = None
    for t in range(32, 48):
        last = model.infer(toks[:, t:t + 1], ids, st2, unembed_mode="last")
        st2.advance(ids, 1)
    torch.cuda.synchronize()
    assert _err(last[:, 0], want[:, -1]) <= 1e-5
    for a, b in zip(st.state, st2.state):
        assert _err(b, a) <= 1e-5
