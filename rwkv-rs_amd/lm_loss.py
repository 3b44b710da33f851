"""The language model's training loss on the gfx950 kernels of
include/rwkv_lm_loss.h: l2wrap followed by the mean cross entropy of the
next-token logits (examples/rwkv-lm/src/model.rs:158-169), as one torch
autograd Function.

The forward reads the logits once (online maximum and log-sum-exp per row)
and keeps four numbers per row; the backward reads them once more and
writes the logits' gradient once, with l2wrap's term (kernels/l2wrap/mod.rs:
38-66: 1e-4 / num_tokens * max(logits) at each row's argmax) folded in. The
logits stay in their dtype (bf16 under autocast) instead of being cast to
fp32. Operands live on the GPU; there is no CPU path.
"""

from __future__ import annotations

import torch

from . import _native
from .neighbors import _code, _ptr, _stream

L2WRAP_FACTOR = 1e-4     # kernels/l2wrap/mod.rs:61-62


class _CrossEntropyL2Wrap(torch.autograd.Function):
    @staticmethod
    def forward(ctx, logits, targets, num_tokens):
        rows, vocab = logits.shape
        dev = logits.device
        loss, lse, mx = (torch.empty(rows, dtype=torch.float32, device=dev) for _ in range(3))
        arg = torch.empty(rows, dtype=torch.int32, device=dev)
        _native.call("rwkv_cross_entropy_l2wrap_forward", _ptr(logits), _ptr(targets), rows,
                     vocab, _code(logits.dtype), _ptr(loss), _ptr(lse), _ptr(mx), _ptr(arg),
                     _stream(dev))
        ctx.save_for_backward(logits, targets, lse, mx, arg)
        ctx.scale = L2WRAP_FACTOR / num_tokens if num_tokens > 0 else 0.0
        return loss

    @staticmethod
    def backward(ctx, dloss):
        logits, targets, lse, mx, arg = ctx.saved_tensors
        rows, vocab = logits.shape
        g = dloss.to(torch.float32).contiguous()
        dlogits = torch.empty_like(logits)
        _native.call("rwkv_cross_entropy_l2wrap_backward", _ptr(logits), _ptr(targets), _ptr(lse),
                     _ptr(mx), _ptr(arg), _ptr(g), float(ctx.scale), rows, vocab,
                     _code(logits.dtype), _ptr(dlogits), _stream(logits.device))
        return dlogits, None, None


def cross_entropy_l2wrap_rows(logits: torch.Tensor, targets: torch.Tensor,
                              num_tokens: int) -> torch.Tensor:
    """Per-row cross entropy of ``logits`` ([rows, vocab], fp32 or bf16) against ``targets`` ([rows] integer), with l2wrap's
    gradient term for ``num_tokens`` tokens in the backward. A target outside
    [0, vocab) gives its row a NaN loss."""
    if not logits.is_cuda or not targets.is_cuda:
        raise ValueError("logits and targets must be GPU tensors")
    if logits.dim() != 2 or targets.shape != (logits.shape[0],):
        raise ValueError("logits must be [rows, vocab] and targets [rows]")
    return _CrossEntropyL2Wrap.apply(logits.contiguous(), targets.to(torch.int64).contiguous(),
                                     int(num_tokens))


def cross_entropy_l2wrap(logits: torch.Tensor, targets: torch.Tensor) -> torch.Tensor:
    """``F.cross_entropy(l2wrap(logits, rows), targets)``: the mean over the
    rows, l2wrap counting every row as a token (model.rs:161-169)."""
    return cross_entropy_l2wrap_rows(logits, targets, logits.shape[0]).mean()
