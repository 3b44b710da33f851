"""CPU tests of the RWKV-7 language-model step (rwkv-rs_amd/model.py), the
host-framework caller of the WKV7 operator.

The operator is swapped for CPU stand-ins the way the reference swaps its
``K: Wkv7Kernel`` type parameter: a plain PyTorch recurrence differentiated
by autograd, and the oracle's reference-order forward/backward wrapped in an
autograd Function. Both must give the same loss and parameter gradients,
which checks that the model hands the six operands and takes the six
gradients in the operator's order. The product kernel is compared against
the plain recurrence on the GPU (tests/test_gpu_model.py).
"""

import math

import numpy as np
import pytest
import torch

from conftest import rel_l2
from model_helpers import (TorchKernel, W_SCALE, _model_mod, _wkv7_mod, loss_and_grads,
                           tiny_model, tokens, torch_recurrence)


def oracle_kernel(oracle):
    class _F(torch.autograd.Function):
        @staticmethod
        def forward(ctx, w, r, k, v, a, b, chunk_len):
            arrs = [x.detach().float().numpy() for x in (w, r, k, v, a, b)]
            out = oracle.forward_f32(*arrs, chunk_len=chunk_len, return_final_state=False)
            ctx.saved = (arrs, out["state"], out["removal_state"], chunk_len, w.dtype)
            return torch.from_numpy(out["output"]).to(w.dtype)

        @staticmethod
        def backward(ctx, dy):
            arrs, ckpt, sa, chunk_len, dt = ctx.saved
            g = oracle.backward_f32(*arrs, ckpt, sa, dy.float().numpy(), chunk_len=chunk_len,
                                    write_initial_state_grad=False)
            names = ("weight_decay_grad", "receptance_grad", "key_grad", "value_grad",
                     "removal_grad", "replacement_grad")
            return (*(torch.from_numpy(g[n]).to(dt) for n in names), None)

    class _K:
        @staticmethod
        def forward(input, state, batch_ids, elapsed_t, chunk_len, context_mask):
            wk = _wkv7_mod()
            y = _F.apply(input.weight_decay, input.receptance, input.replacement_key,
                         input.value, input.removal_key_normalized, input.replacement,
                         chunk_len)
            return wk.KernelOutput(output=y, next_state=state)

    return _K


# ----------------------------------------------------------------- LoRA ranks
def test_lora_ranks_table_and_formula():
    m = _model_mod()
    r = m.infer_time_mixer_lora_ranks(12, 768, 64)           # the 0.1B model
    assert (r.weight_decay_lora, r.learning_rate_lora, r.value_residual_lora,
            r.output_gate_lora) == (64, 64, 32, 128)
    # sqrt(512) = 22.63: 2.5x -> 56.6 -> 64; 1.7x -> 38.5 -> 32; 5x -> 113.1 -> 128
    r = m.infer_time_mixer_lora_ranks(8, 512, 64)
    assert (r.weight_decay_lora, r.value_residual_lora, r.output_gate_lora) == (64, 32, 128)
    # head_size scales all but the output gate: 2.5 * 22.63 * 2 = 113.1 -> 128,
    # 1.7 * 22.63 * 2 = 76.9 -> 64
    r = m.infer_time_mixer_lora_ranks(8, 512, 128)
    assert (r.weight_decay_lora, r.value_residual_lora, r.output_gate_lora) == (128, 64, 128)
    # halves round to even multiples of 32, and nothing goes below 32
    assert m.infer_lora_rank_from_formula(80.0) == 64
    assert m.infer_lora_rank_from_formula(112.0) == 128
    assert m.infer_lora_rank_from_formula(3.0) == 32


# ------------------------------------------------------------ token shift diff
def _token_shift_loop(x, shift, mask):
    """One lane at a time, as token_shift_diff/kernel.rs:36-63 walks time."""
    B, T, C = x.shape
    diff = np.zeros_like(x)
    nxt = np.zeros((B, C), x.dtype)
    for bi in range(B):
        ext = shift[bi]
        prev, nx = ext.copy(), ext.copy()
        for t in range(T):
            if mask[bi, t] == 0:
                diff[bi, t] = 0.0
                prev = ext.copy()
            else:
                diff[bi, t] = prev - x[bi, t]
                prev = x[bi, t].copy()
                nx = x[bi, t].copy()
        nxt[bi] = nx
    return diff, nxt


@pytest.mark.parametrize("masked", [False, True])
def test_token_shift_diff_matches_lane_walk(masked):
    m = _model_mod()
    rng = np.random.default_rng(3)
    B, T, C = 4, 9, 8
    x = rng.standard_normal((B, T, C)).astype(np.float32)
    shift = rng.standard_normal((B, C)).astype(np.float32)
    mask = (rng.random((B, T)) > 0.4).astype(np.float32) if masked else np.ones((B, T), np.float32)
    if masked:
        mask[0] = 0.0                   # a lane with no valid step keeps its shift
        mask[1, :3] = 0.0               # left padding
    x = x * mask[:, :, None]            # callers zero masked steps first
    want_d, want_n = _token_shift_loop(x, shift, mask)
    d, n = m.token_shift_diff(torch.from_numpy(x), torch.from_numpy(shift),
                              torch.from_numpy(mask) if masked else None)
    np.testing.assert_array_equal(d.numpy(), want_d)
    np.testing.assert_array_equal(n.numpy(), want_n)


def test_token_shift_diff_zero_external_shift_by_default():
    m = _model_mod()
    x = torch.arange(6.0).reshape(1, 3, 2)
    d, n = m.token_shift_diff(x)
    np.testing.assert_array_equal(d.numpy(), [[[0, -1], [-2, -2], [-2, -2]]])
    np.testing.assert_array_equal(n.numpy(), [[4, 5]])


# ---------------------------------------------------------------------- l2wrap
def test_l2wrap_gradient_known_answer():
    m = _model_mod()
    logits = torch.tensor([[1.0, 3.0, -2.0], [0.5, -1.0, 0.25]], requires_grad=True)
    out = m.l2wrap(logits, 2)
    np.testing.assert_array_equal(out.detach().numpy(), logits.detach().numpy())
    out.backward(torch.ones_like(out))
    want = np.ones((2, 3))
    want[0, 1] += 1e-4 / 2 * 3.0
    want[1, 0] += 1e-4 / 2 * 0.5
    np.testing.assert_allclose(logits.grad.numpy(), want, rtol=0, atol=1e-7)


# ------------------------------------------------------------- model wiring
def test_torch_recurrence_closed_form_decay_only():
    """a = b = 0 makes y_t = sum_{s<=t} (prod_{s<u<=t} w~_u * k_s . r_t) v_s
    (decayed linear attention), computed here directly."""
    rng = np.random.default_rng(5)
    B, T, H, N = 1, 5, 1, 64
    w, r, k, v = (torch.from_numpy(rng.standard_normal((B, T, H, N))) for _ in range(4))
    z = torch.zeros_like(w)
    y = torch_recurrence(w, r, k, v, z, z)
    wt = torch.exp(W_SCALE * torch.sigmoid(w))[0, :, 0]
    for t in range(T):
        acc = torch.zeros(N, dtype=torch.float64)
        for s in range(t + 1):
            dec = torch.prod(wt[s + 1:t + 1], dim=0) if s < t else torch.ones(N, dtype=torch.float64)
            acc += (dec * k[0, s, 0] * r[0, t, 0]).sum() * v[0, s, 0]
        np.testing.assert_allclose(y[0, t, 0].numpy(), acc.numpy(), rtol=1e-12, atol=1e-12)


def test_model_oracle_kernel_matches_torch_recurrence(oracle):
    """The oracle's fp32 forward/backward inside the model gives the loss and
    every parameter gradient of the model differentiated through the plain
    recurrence: the operands and gradients are wired in the operator's order."""
    model = tiny_model(std=0.2)        # large enough that every path carries signal
    inputs, targets = tokens(2, 32, 97)
    l0, g0 = loss_and_grads(model, TorchKernel, inputs, targets)
    l1, g1 = loss_and_grads(model, oracle_kernel(oracle), inputs, targets)
    assert abs(l0 - l1) <= 1e-5 * abs(l0)
    assert g0.keys() == g1.keys()
    worst = max(rel_l2(g1[n].numpy(), g0[n].numpy()) for n in g0)
    assert worst <= 1e-4, worst
    # every trainable tensor receives a gradient (the first cell has no value residual)
    names = {n for n, _ in model.named_parameters()}
    assert names == set(g0)


def test_model_loss_at_init_is_uniform_entropy():
    """N(0, 0.02) weights over the unit-variance layer-normed stream give
    Gaussian logits of variance sigma^2 = C * 0.02^2, and a mean cross entropy
    of ln(vocab) + sigma^2 / 2."""
    model = tiny_model(vocab=211, heads=4)
    inputs, targets = tokens(4, 32, 211)
    with torch.no_grad():
        loss = model(inputs, targets, TorchKernel)
    assert abs(float(loss) - (math.log(211) + 256 * 0.02 ** 2 / 2)) < 0.03


def test_train_step_reduces_loss_on_a_fixed_batch():
    m = _model_mod()
    model = tiny_model(std=0.1)
    opt = m.make_optimizer(model, lr=3e-3)
    inputs, targets = tokens(2, 16, 97)
    losses = [float(m.train_step(model, opt, inputs, targets, TorchKernel, autocast=False))
              for _ in range(6)]
    assert all(math.isfinite(x) for x in losses)
    assert losses[-1] < losses[0] - 0.1, losses


def test_product_kernel_refuses_cpu_tensors():
    """The default operator is the HIP library: CPU operands are an error,
    never a silent CPU fallback."""
    model = tiny_model()
    inputs, targets = tokens(1, 16, 97)
    with pytest.raises((ValueError, RuntimeError)):
        model(inputs, targets)


def test_model_bf16_operands_without_autocast():
    """bf16 operands with float32 weights and no autocast: the operator's
    output is brought back to the residual stream's dtype before the norm."""
    inputs, targets = tokens(2, 32, 97)
    l32, _ = loss_and_grads(tiny_model(std=0.2), TorchKernel, inputs, targets)
    l16, g16 = loss_and_grads(tiny_model(std=0.2, wkv7_dtype=torch.bfloat16), TorchKernel,
                              inputs, targets)
    assert abs(l16 - l32) <= 1e-2 * abs(l32)
    assert all(torch.isfinite(g).all() for g in g16.values())


def test_token_shift_by_slot():
    """token_shift_diff with batch_ids (weight_prepare.rs:224-229,
    channel_mixer/mod.rs:84-99): rows read their slots of the full-batch
    shift, the next shift replaces those slots and keeps the others."""
    m = _model_mod()
    g = torch.Generator().manual_seed(4)
    x = torch.randn(2, 5, 8, generator=g)
    full = torch.randn(4, 8, generator=g)
    ids = torch.tensor([3, 0])
    mask = torch.ones(2, 5)
    mask[1, :2] = 0.0
    diff, nxt = m.token_shift_diff(x, full, mask, ids)
    want_diff, want_rows = m.token_shift_diff(x, full[ids], mask)
    assert torch.equal(diff, want_diff)
    assert torch.equal(nxt[ids], want_rows)
    assert torch.equal(nxt[[1, 2]], full[[1, 2]])
    assert torch.equal(m.token_shift_diff(x, full[:2], mask)[0],
                       m.token_shift_diff(x, full[:2], mask, None)[0])
