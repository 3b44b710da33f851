"""GPU parity of the fused loss (include/rwkv_lm_loss.h) against float64
PyTorch on the CPU: l2wrap as the model's torch Function (kernels/l2wrap/
mod.rs:38-66) followed by ``F.cross_entropy`` (the mean over rows, as
examples/rwkv-lm/src/model.rs:161-169), forward and backward.

Every row gets a unique maximum, so the argmax that l2wrap's term lands on
is the same in both. Bars: the loss and the per-row statistics within 1e-5
relative (both read the same logits and compute in fp32 / fp64); the
logits' gradient within 1e-5 relative L2 in fp32 and 8e-3 in bf16 (its
rounding).
"""

import pytest
import torch
import torch.nn.functional as F

from conftest import announce, load_pkg, rel_l2
from model_helpers import _model_mod

pytestmark = pytest.mark.gpu

CASES = [
    dict(rows=6, V=97, dt="f32"),          # element path (vocab not a multiple of 8)
    dict(rows=33, V=512, dt="f32"),        # vector path
    dict(rows=17, V=50, dt="bf16"),
    dict(rows=40, V=1000, dt="bf16"),
    dict(rows=64, V=65536, dt="bf16"),     # config[4]'s vocabulary
    dict(rows=3, V=8, dt="f32"),           # fewer logits than threads
]
DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _case_id(c):
    return "rows{rows}_V{V}_{dt}".format(**c)


def _inputs(rows, V, dt, seed):
    g = torch.Generator().manual_seed(seed)
    logits = 3.0 * torch.randn(rows, V, generator=g)
    peak = torch.randint(0, V, (rows,), generator=g)
    logits[torch.arange(rows), peak] = logits.max(dim=1).values + 1.0   # unique maximum
    logits = logits.to(DT[dt])
    targets = torch.randint(0, V, (rows,), generator=g)
    return logits, targets, peak


@pytest.mark.parametrize("case", CASES, ids=_case_id)
def test_cross_entropy_l2wrap_matches_torch(case):
    ll = load_pkg().lm_loss
    m = _model_mod()
    rows, V, dt = case["rows"], case["V"], case["dt"]
    logits, targets, peak = _inputs(rows, V, dt, rows * 7 + V)

    x64 = logits.double().requires_grad_(True)
    want = F.cross_entropy(m.l2wrap(x64, rows), targets)
    want.backward()

    dev = torch.device("cuda:0")
    x = logits.to(dev).requires_grad_(True)
    announce("cross_entropy_l2wrap", _case_id(case))
    got = ll.cross_entropy_l2wrap(x, targets.to(dev))
    got.backward()
    torch.cuda.synchronize()
    assert abs(got.item() - want.item()) <= 1e-5 * abs(want.item()), (got.item(), want.item())
    tol = 8e-3 if dt == "bf16" else 1e-5
    assert x.grad.dtype == logits.dtype
    assert rel_l2(x.grad.double().cpu().numpy(), x64.grad.numpy()) <= tol


def test_row_statistics_and_out_of_range_target():
    ll = load_pkg().lm_loss
    rows, V = 5, 300
    logits, targets, peak = _inputs(rows, V, "f32", 11)
    targets[2] = V + 4                          # out of range: NaN loss, no target term
    dev = torch.device("cuda:0")
    x = logits.to(dev).requires_grad_(True)
    announce("cross_entropy_l2wrap", "rows5_V300_bad_target")
    per_row = ll.cross_entropy_l2wrap_rows(x, targets.to(dev), rows)
    w = torch.arange(1, rows + 1, dtype=torch.float32, device=dev)   # uneven row weights
    per_row.backward(w)
    torch.cuda.synchronize()
    got = per_row.double().cpu()
    lse = torch.logsumexp(logits.double(), dim=1)
    ok = torch.arange(rows) != 2
    want = lse - logits.double()[torch.arange(rows), targets.clamp(max=V - 1)]
    assert torch.isnan(got[2])
    assert torch.allclose(got[ok], want[ok], rtol=1e-5, atol=0)
    # gradient: w_r (softmax - onehot) + 1e-4 / rows * max at the argmax
    sm = torch.softmax(logits.double(), dim=1)
    onehot = torch.zeros(rows, V, dtype=torch.float64)
    onehot[ok, targets[ok]] = 1.0
    ref = w.double().cpu()[:, None] * (sm - onehot)
    ref[torch.arange(rows), peak] += 1e-4 / rows * logits.double().max(dim=1).values
    assert rel_l2(x.grad.double().cpu().numpy(), ref.numpy()) <= 1e-5
