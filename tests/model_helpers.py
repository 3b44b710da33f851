"""Stand-ins and fixtures shared by the language-model tests: a plain
PyTorch WKV7 recurrence used as the operator (differentiated by autograd), a
small model, seeded token batches, a synthetic checkpoint in the release
format and a float64 forward that reads such a checkpoint by its own key
names."""

import importlib

import torch
import torch.nn.functional as F


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


# ------------------------------------------------------- release checkpoints
def release_checkpoint(L, C, H, V, ranks, seed=0, dtype=torch.bfloat16, scaled=False):
    """A checkpoint in the format of the public RWKV-7 ``.pth`` releases:
    their key names and shapes, written out here rather than taken from the
    loader's table. ``ranks`` = (w, a, v, g) LoRA ranks. Unscaled, every
    tensor is N(0, 1) (distinct values, so a tensor can be traced to the
    parameter it lands in); ``scaled`` draws each at a scale that keeps a
    forward pass well conditioned (projections ~ 1/sqrt(fan-in), norms near
    one, mixes in (0, 1)), so that its logits can be compared."""
    g = torch.Generator().manual_seed(seed)
    RW, RA, RV, RG = ranks

    def t(*shape, std=1.0, mean=0.0):
        if not scaled:
            std, mean = 1.0, 0.0
        return (torch.randn(*shape, generator=g) * std + mean).to(dtype)

    def u(*shape):          # mixes: uniform in (0, 1)
        if not scaled:
            return t(*shape)
        return torch.rand(*shape, generator=g).to(dtype)

    def lin(o, i):          # [out, in]
        return t(o, i, std=i ** -0.5)

    sd = {"emb.weight": t(V, C), "blocks.0.ln0.weight": t(C, std=0.1, mean=1.0),
          "blocks.0.ln0.bias": t(C, std=0.1), "ln_out.weight": t(C, std=0.1, mean=1.0),
          "ln_out.bias": t(C, std=0.1), "head.weight": lin(V, C)}
    for i in range(L):
        b = f"blocks.{i}."
        for n in ("ln1", "ln2", "att.ln_x"):
            sd[b + n + ".weight"] = t(C, std=0.1, mean=1.0)
            sd[b + n + ".bias"] = t(C, std=0.1)
        for n in ("x_r", "x_w", "x_k", "x_v", "x_a", "x_g"):
            sd[b + "att." + n] = u(1, 1, C)
        sd[b + "att.k_k"] = t(1, 1, C, std=0.2, mean=1.0)
        sd[b + "att.k_a"] = t(1, 1, C, std=0.5, mean=0.5)
        sd[b + "att.w0"] = t(1, 1, C, std=1.0, mean=-1.0)
        sd[b + "att.a0"] = t(1, 1, C, std=0.5)
        sd[b + "att.v0"] = t(1, 1, C, std=0.5)
        sd[b + "att.r_k"] = t(H, 64, std=0.5)
        # LoRA factors are [in, out] (x @ w1 @ w2)
        sd[b + "att.w1"], sd[b + "att.w2"] = t(C, RW, std=C ** -0.5), t(RW, C, std=RW ** -0.5)
        sd[b + "att.a1"], sd[b + "att.a2"] = t(C, RA, std=C ** -0.5), t(RA, C, std=RA ** -0.5)
        sd[b + "att.v1"], sd[b + "att.v2"] = t(C, RV, std=C ** -0.5), t(RV, C, std=RV ** -0.5)
        sd[b + "att.g1"], sd[b + "att.g2"] = t(C, RG, std=C ** -0.5), t(RG, C, std=RG ** -0.5)
        for n in ("receptance", "key", "value", "output"):
            sd[b + f"att.{n}.weight"] = lin(C, C)
        sd[b + "ffn.x_k"] = u(1, 1, C)
        sd[b + "ffn.key.weight"] = lin(4 * C, C)
        sd[b + "ffn.value.weight"] = lin(C, 4 * C)
    return sd


def release_forward_f64(sd, tokens, num_heads, head_size=64):
    """Logits [B, T, V] in float64 of an RWKV-7 checkpoint in the release
    format, computed from its tensors by their release names, with no model
    object and no key table: the release's conventions (linear weights
    [out, in], LoRA factors [in, out], mixes [1, 1, C]) applied to the
    reference's operations:

    * embedding, LayerNorm ln0 (eps 1e-5), the cells, LayerNorm ln_out, head
      (examples/rwkv-lm/src/model.rs:122-178, cells/causal.rs:226-268);
    * time mix (weight_prepare.rs:210-330, gated_readout.rs:110-148): token
      shift diff x[t-1] - x[t]; r, k, v projections; the value residual from
      cell 0's value (sigmoid LoRA v0/v1/v2); learning rate sigmoid(a0 + ..);
      decay logit -softplus(-(w0 + tanh(x w1) w2)) - 0.5; gate
      sigmoid(x g1) g2; kk = L2-normalised k * k_k per head; the operator's
      key k * (1 + (lr - 1) * k_a); WKV7 on (w, r, k~, v, -kk, kk * lr);
      GroupNorm over heads (eps 64e-5), the r k~ r_k bonus times v, gate,
      output projection;
    * channel mix (channel_mixer/mod.rs:83-121): relu(key(x + diff * x_k))^2,
      value.
    """
    f = {k: v.detach().double().cpu() for k, v in sd.items()}
    tokens = tokens.cpu()
    C = f["emb.weight"].shape[1]
    H, N = num_heads, head_size
    B, T = tokens.shape
    L = 1 + max(int(k.split(".")[1]) for k in f if k.startswith("blocks."))
    shape = (B, T, H, N)

    def ln(x, p, eps=1e-5):
        return F.layer_norm(x, (C,), f[p + ".weight"], f[p + ".bias"], eps)

    def shift_diff(x):
        prev = torch.cat([torch.zeros_like(x[:, :1]), x[:, :-1]], dim=1)
        return prev - x

    def vec(p):
        return f[p].reshape(C)

    x = ln(f["emb.weight"][tokens], "blocks.0.ln0")
    v_first = None
    for i in range(L):
        p = f"blocks.{i}.att."
        xt = ln(x, f"blocks.{i}.ln1")
        d = shift_diff(xt)
        xr, xw, xk, xv, xa, xg = (xt + d * vec(p + "x_" + n) for n in "rwkvag")
        r = xr @ f[p + "receptance.weight"].T
        k = xk @ f[p + "key.weight"].T
        v = xv @ f[p + "value.weight"].T
        if i == 0:
            v_first = v
        else:
            nu = torch.sigmoid(vec(p + "v0") + (xv @ f[p + "v1"]) @ f[p + "v2"])
            v = v + (v_first - v) * nu
        lr = torch.sigmoid(vec(p + "a0") + (xa @ f[p + "a1"]) @ f[p + "a2"])
        w = -F.softplus(-(vec(p + "w0") + torch.tanh(xw @ f[p + "w1"]) @ f[p + "w2"])) - 0.5
        g = torch.sigmoid(xg @ f[p + "g1"]) @ f[p + "g2"]
        kk = F.normalize((k * vec(p + "k_k")).reshape(shape), p=2.0, dim=-1, eps=1e-12)
        kt = k * (1.0 + (lr - 1.0) * vec(p + "k_a"))
        y = torch_recurrence(w.reshape(shape), r.reshape(shape), kt.reshape(shape),
                             v.reshape(shape), -kk, kk * lr.reshape(shape))
        y = F.group_norm(y.reshape(B * T, C), H, f[p + "ln_x.weight"], f[p + "ln_x.bias"],
                         64e-5).reshape(B, T, C)
        bonus = ((r.reshape(shape) * kt.reshape(shape) * f[p + "r_k"]).sum(-1, keepdim=True)
                 * v.reshape(shape)).reshape(B, T, C)
        x = x + ((y + bonus) * g) @ f[p + "output.weight"].T
        xc = ln(x, f"blocks.{i}.ln2")
        mixed = xc + shift_diff(xc) * vec(f"blocks.{i}.ffn.x_k")
        h = torch.relu(mixed @ f[f"blocks.{i}.ffn.key.weight"].T) ** 2
        x = x + h @ f[f"blocks.{i}.ffn.value.weight"].T
    return ln(x, "ln_out") @ f["head.weight"].T


def model_logits(model, tokens, kernel):
    """The training path's logits (model.rs:122-156) with ``kernel`` as the
    WKV7 operator."""
    ids = torch.arange(tokens.shape[0], device=tokens.device)
    x = model.layer_norm_for_first_cell(model.embed(tokens))
    x, _, _, _ = model.cells(x, ids, kernel)
    return model.unembed(model.layer_norm_for_unembed(x))
