"""Stand-ins and fixtures shared by the language-model tests: a plain
PyTorch WKV7 recurrence used as the operator (differentiated by autograd), a
small model and seeded token batches."""

import importlib

import torch


def _model_mod():
    return importlib.import_module("rwkv-rs_amd.model")


def _wkv7_mod():
    return importlib.import_module("rwkv-rs_amd.wkv7")


W_SCALE = -0.6065306597126334


# ------------------------------------------------------------ WKV7 stand-ins
def torch_recurrence(w, r, k, v, a, b):
    """WKV7 per (b, h) in float64 by the reference's step equations
    (wkv7_common/kernel.rs:51-103): S <- S diag(exp(W_SCALE sigmoid(w)))
    + (S a) b^T + v k^T, y = S r, with S[value, key]."""
    B, T, H, N = w.shape
    dt = w.dtype
    w, r, k, v, a, b = (x.double() for x in (w, r, k, v, a, b))
    wt = torch.exp(W_SCALE * torch.sigmoid(w))
    S = w.new_zeros(B, H, N, N)
    ys = []
    for t in range(T):
        sa = (S * a[:, t, :, None, :]).sum(-1)
        S = (S * wt[:, t, :, None, :] + sa[..., None] * b[:, t, :, None, :]
             + v[:, t, :, :, None] * k[:, t, :, None, :])
        ys.append((S * r[:, t, :, None, :]).sum(-1))
    return torch.stack(ys, 1).to(dt)


class TorchKernel:
    """A ``Wkv7Kernel`` whose forward is ``torch_recurrence``."""

    @staticmethod
    def forward(input, state, batch_ids, elapsed_t, chunk_len, context_mask):
        wk = _wkv7_mod()
        y = torch_recurrence(input.weight_decay, input.receptance, input.replacement_key,
                             input.value, input.removal_key_normalized, input.replacement)
        return wk.KernelOutput(output=y, next_state=state)


def tiny_model(seed=0, cells=2, heads=2, vocab=97, std=0.02, wkv7_dtype=torch.float32,
               neighbor_ops="torch"):
    m = _model_mod()
    torch.manual_seed(seed)
    model = m.AutoRegressiveModel(vocab, cells, heads * 64, heads, 64, wkv7_dtype=wkv7_dtype,
                                  neighbor_ops=neighbor_ops)
    g = torch.Generator().manual_seed(seed)
    return model.init_random(std, g)


def tokens(B, T, vocab, seed=1):
    g = torch.Generator().manual_seed(seed)
    t = torch.randint(0, vocab, (B, T + 1), generator=g)
    return t[:, :-1].contiguous(), t[:, 1:].contiguous()


def loss_and_grads(model, kernel, inputs, targets):
    model.zero_grad(set_to_none=True)
    loss = model(inputs, targets, kernel)
    loss.backward()
    return float(loss.detach()), {n: p.grad.detach().clone() for n, p in model.named_parameters()
                         if p.grad is not None}
