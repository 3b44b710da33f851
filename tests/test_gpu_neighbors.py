"""GPU parity of the fused neighbour kernels (include/rwkv_neighbors.h)
against float64 PyTorch on the CPU of the same ops, forward and backward:

* token shift + mixes against ``model.token_shift_diff`` + ``addcmul`` (the
  torch mirror of token_shift_diff/kernel.rs:17-64 and addcmul/kernel.rs),
  with and without masks, external shifts and slot-mapped batch ids; fp32
  results within 1e-5 relative L2, bf16 outputs within bf16 rounding (8e-3);
* the gated readout against GroupNorm + bonus + gate written with torch ops
  (gated_readout.rs:126-145), same bars;
* the end of the weight preparation (learning rate, replacement key, value
  residual, decay, normalized removal key, replacement) against the same ops
  in torch (weight_prepare.rs:282-317), with and without the residual, with a
  head whose removal key is zero (the clamped norm), same bars;
* the whole language model with the fused ops against the same model with
  the torch formulations (same weights and tokens): loss and every
  parameter gradient within 1e-4 in fp32.
"""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import announce, load_pkg, rel_l2
from model_helpers import _model_mod, loss_and_grads, tiny_model, tokens

pytestmark = pytest.mark.gpu

F32_TOL = 1e-5
BF16_TOL = 8e-3


def _nb():
    return load_pkg().neighbors


def _err(got, want):
    return rel_l2(got.detach().double().cpu().numpy(), want.detach().double().cpu().numpy())


# ---------------------------------------------------------------- token shift
SHIFT_CASES = [
    dict(B=2, T=33, C=64, K=5, mask=False, shift=False, ids=False, xdt="f32", odt="f32"),
    dict(B=3, T=17, C=192, K=6, mask=True, shift=True, ids=True, xdt="f32", odt="f32"),
    dict(B=2, T=40, C=768, K=6, mask=False, shift=False, ids=False, xdt="f32", odt="bf16"),
    dict(B=2, T=9, C=260, K=5, mask=True, shift=False, ids=False, xdt="f32", odt="f32"),
    dict(B=4, T=1, C=128, K=1, mask=False, shift=True, ids=True, xdt="f32", odt="f32"),
    dict(B=2, T=16, C=128, K=6, mask=True, shift=True, ids=False, xdt="bf16", odt="bf16"),
    dict(B=16, T=512, C=768, K=6, mask=False, shift=False, ids=False, xdt="f32", odt="bf16"),
    # one mix (its own forward and backward walks) over runs of rows within a
    # sequence, ragged (T not a multiple of a wave's 8 rows), with masks
    dict(B=3, T=37, C=192, K=1, mask=True, shift=True, ids=True, xdt="f32", odt="bf16"),
    dict(B=2, T=29, C=256, K=1, mask=False, shift=False, ids=False, xdt="bf16", odt="bf16"),
    # seven and eight mixes (the eight-mix instance)
    dict(B=3, T=21, C=128, K=8, mask=True, shift=False, ids=False, xdt="bf16", odt="f32"),
    dict(B=2, T=13, C=64, K=7, mask=False, shift=True, ids=False, xdt="f32", odt="f32"),
]
DT = {"f32": torch.float32, "bf16": torch.bfloat16}


def _shift_case_id(c):
    return "B{B}T{T}C{C}K{K}{m}{s}{i}_{xdt}_{odt}".format(
        m="_mask" if c["mask"] else "", s="_shift" if c["shift"] else "",
        i="_ids" if c["ids"] else "", **c)


@pytest.mark.parametrize("case", SHIFT_CASES, ids=_shift_case_id)
def test_token_shift_mix_matches_torch(case):
    m = _model_mod()
    nb = _nb()
    B, T, C, K = case["B"], case["T"], case["C"], case["K"]
    xdt, odt = DT[case["xdt"]], DT[case["odt"]]
    g = torch.Generator().manual_seed(B * 1000 + T * 10 + C)
    x = torch.randn(B, T, C, generator=g).to(xdt)
    scales = [torch.rand(1, 1, C, generator=g) for _ in range(K)]
    full = B + 3 if case["ids"] else B
    ids = torch.randperm(full, generator=g)[:B] if case["ids"] else None
    shift = torch.randn(full, C, generator=g).to(xdt) if case["shift"] else None
    mask = None
    if case["mask"]:
        mask = (torch.rand(B, T, generator=g) > 0.3).float()
        mask[0, :3] = 0.0
        if B > 2:
            mask[2] = 0.0                 # a row with no valid step
        x = x * mask.unsqueeze(2).to(xdt)
    grads = [torch.randn(B, T, C, generator=g).to(odt) for _ in range(K)]

    # float64 torch on the CPU
    x64 = x.double().requires_grad_(True)
    sc64 = [s.double().requires_grad_(True) for s in scales]
    sh64 = shift.double().requires_grad_(True) if shift is not None else None
    rows = sh64[ids] if (sh64 is not None and ids is not None) else sh64
    diff, nxt = m.token_shift_diff(x64, rows, mask.double() if mask is not None else None)
    want = [m.addcmul(x64, diff, s) for s in sc64]
    loss = sum((w * gg.double()).sum() for w, gg in zip(want, grads))
    loss.backward()
    want_next = None
    if shift is not None:
        want_next = shift.double().clone()
        if ids is not None:
            want_next[ids] = nxt.detach()
        else:
            want_next = nxt.detach()

    dev = torch.device("cuda:0")
    xg = x.to(dev).requires_grad_(True)
    scg = [s.to(dev).requires_grad_(True) for s in scales]
    shg = shift.to(dev).requires_grad_(True) if shift is not None else None
    announce("token_shift_mix", _shift_case_id(case))
    res = nb.token_shift_mix(xg, scg, shg, ids.to(dev) if ids is not None else None,
                             mask.to(dev) if mask is not None else None, odt,
                             return_next_token_shift=shift is not None)
    mixes, got_next = res if shift is not None else (res, None)
    sum((mx.float() * gg.to(dev).float()).sum() for mx, gg in zip(mixes, grads)).backward()
    torch.cuda.synchronize()

    out_tol = BF16_TOL if odt == torch.bfloat16 else F32_TOL
    for i in range(K):
        assert mixes[i].dtype == odt
        assert _err(mixes[i], want[i]) <= out_tol, ("mix", i)
    grad_tol = BF16_TOL if xdt == torch.bfloat16 else F32_TOL
    assert _err(xg.grad, x64.grad) <= grad_tol
    for i in range(K):
        assert _err(scg[i].grad, sc64[i].grad) <= F32_TOL, ("scale", i)
    if shift is not None:
        assert _err(shg.grad, sh64.grad) <= grad_tol
        assert _err(got_next, want_next) == 0.0        # a copy of x or of the shift


def _reference_shift_backward(x, scales, shift_rows, mask, grads):
    """The token shift + mixes' gradients as the reference's autodiff forms
    them, restated in float64 (token_shift_diff/backward.rs:51-97 for x and
    the external shift, addcmul's backward for the mixes), for any mask
    values: the forward treats a step as valid when its mask is not 0
    (token_shift_diff/kernel.rs:51-60); the backward weights with the mask
    values. Returns dx, dscales (one per scale), dshift_rows."""
    B, T, C = x.shape
    m = mask.double()
    valid = (m != 0).double()
    ext = shift_rows.double()
    prev = torch.cat([ext.unsqueeze(1), x[:, :-1]], 1)
    prev_valid = torch.cat([torch.zeros(B, 1, dtype=torch.float64), valid[:, :-1]], 1)
    prev = prev_valid.unsqueeze(2) * prev + (1 - prev_valid.unsqueeze(2)) * ext.unsqueeze(1)
    diff = valid.unsqueeze(2) * (prev - x)
    dd = sum(g * s.reshape(1, 1, C) for g, s in zip(grads, scales))   # gradient of diff
    gs = sum(grads)                                                    # of x through x + ...
    dscales = [(g * diff).sum(dim=(0, 1)) for g in grads]
    masked = dd * m.unsqueeze(2)
    shifted_next = torch.cat([masked[:, 1:], torch.zeros(B, 1, C, dtype=torch.float64)], 1)
    dx = gs - masked + m.unsqueeze(2) * shifted_next
    prev_m = torch.cat([torch.zeros(B, 1, dtype=torch.float64), m[:, :-1]], 1)
    use_ext = m * (1 - prev_m)
    dshift_rows = (masked * use_ext.unsqueeze(2)).sum(1)
    return dx, dscales, dshift_rows


def test_token_shift_backward_with_fractional_mask_values_and_repeated_slots():
    """Mask values other than 0 and 1 and repeated batch ids, which the
    reference's autodiff handles by weighting with the mask values and by
    adding each row's shift gradient into its slot (select_assign with Add):
    dx, the scale gradients and the external shift's gradient against
    ``_reference_shift_backward`` in float64; the forward mixes are unchanged
    by the values (a step is valid when its mask is not 0)."""
    nb = _nb()
    B, T, C, K = 4, 13, 128, 6
    g = torch.Generator().manual_seed(77)
    x = torch.randn(B, T, C, generator=g, dtype=torch.float64)
    scales = [torch.rand(C, generator=g, dtype=torch.float64) for _ in range(K)]
    mask = torch.tensor([0.0, 0.5, 1.0, 0.25, 2.0, 0.0, 0.0, 1.0, 0.75, 1.0, 0.0, 0.5, 1.0],
                        dtype=torch.float64)
    mask = torch.stack([mask, mask.roll(3), mask.roll(5), torch.ones(T, dtype=torch.float64)])
    full = 3
    ids = torch.tensor([2, 0, 2, 1])          # slot 2 twice
    shift = torch.randn(full, C, generator=g, dtype=torch.float64)
    grads = [torch.randn(B, T, C, generator=g, dtype=torch.float64) for _ in range(K)]
    want_dx, want_dsc, want_rows = _reference_shift_backward(x, scales, shift[ids], mask, grads)
    want_dshift = torch.zeros(full, C, dtype=torch.float64).index_add_(0, ids, want_rows)
    dev = torch.device("cuda:0")
    xg = x.float().to(dev).requires_grad_(True)
    scg = [s.float().to(dev).requires_grad_(True) for s in scales]
    shg = shift.float().to(dev).requires_grad_(True)
    announce("token_shift_mix backward, fractional mask, repeated slots")
    mixes = nb.token_shift_mix(xg, scg, shg, ids.to(dev), mask.float().to(dev), torch.float32)
    sum((mx * gg.float().to(dev)).sum() for mx, gg in zip(mixes, grads)).backward()
    torch.cuda.synchronize()
    assert _err(xg.grad, want_dx) <= F32_TOL
    for i in range(K):
        assert _err(scg[i].grad, want_dsc[i]) <= F32_TOL, i
    assert _err(shg.grad, want_dshift) <= F32_TOL


# --------------------------------------------------------------- gated readout
READOUT_CASES = [
    dict(B=2, T=24, H=3, op="f32", act="f32"),
    dict(B=2, T=16, H=12, op="bf16", act="bf16"),
    dict(B=1, T=70, H=4, op="bf16", act="f32"),
    # the last 16-lane group of rows holds 1 and 3 rows (groups walk 4)
    dict(B=3, T=11, H=2, op="f32", act="bf16"),
    dict(B=1, T=67, H=5, op="bf16", act="bf16"),
    dict(B=16, T=512, H=12, op="bf16", act="bf16"),
]


@pytest.mark.parametrize("case", READOUT_CASES,
                         ids=lambda c: "B{B}T{T}H{H}_{op}_{act}".format(**c))
def test_gated_readout_matches_torch(case):
    nb = _nb()
    B, T, H = case["B"], case["T"], case["H"]
    C = H * 64
    opd, actd = DT[case["op"]], DT[case["act"]]
    g = torch.Generator().manual_seed(B * 100 + T + H)
    y, r, k, v = (torch.randn(B, T, H, 64, generator=g).to(opd) for _ in range(4))
    y = (y.float() * 3.0 + 0.5).to(opd)           # a non-trivial mean and scale per group
    gate = torch.rand(B, T, C, generator=g).to(actd)
    bonus = torch.randn(H, 64, generator=g) * 0.1
    weight = 1.0 + 0.1 * torch.randn(C, generator=g)
    bias = 0.1 * torch.randn(C, generator=g)
    dout = torch.randn(B, T, C, generator=g).to(actd)

    ins64 = [t.double().requires_grad_(True) for t in (y, r, k, v, gate, bonus, weight, bias)]
    y64, r64, k64, v64, g64, bo64, w64, b64 = ins64
    yn = F.group_norm(y64.reshape(B * T, C), H, w64, b64, 64e-5).reshape(B, T, C)
    bon = ((r64 * k64 * bo64).sum(-1, keepdim=True) * v64).reshape(B, T, C)
    want = (yn + bon) * g64
    (want * dout.double()).sum().backward()

    dev = torch.device("cuda:0")
    ins = [t.to(dev).requires_grad_(True) for t in (y, r, k, v, gate, bonus, weight, bias)]
    announce("gated_readout", case)
    out = nb.gated_readout(*ins, eps=64e-5)
    (out.float() * dout.to(dev).float()).sum().backward()
    torch.cuda.synchronize()
    assert out.dtype == actd
    assert _err(out, want) <= (BF16_TOL if actd == torch.bfloat16 else F32_TOL)
    names = ("y", "r", "k", "v", "gate", "bonus", "weight", "bias")
    for n, a, b in zip(names, ins, ins64):
        tol = F32_TOL
        if n in ("y", "r", "k", "v") and opd == torch.bfloat16:
            tol = BF16_TOL
        if n == "gate" and actd == torch.bfloat16:
            tol = BF16_TOL
        assert _err(a.grad, b.grad) <= tol, n


# ------------------------------------------------------- weight preparation end
PREPARE_CASES = [
    dict(B=2, T=24, H=2, res=True, idt="f32", odt="f32", zero_head=False),
    dict(B=1, T=40, H=3, res=False, idt="f32", odt="f32", zero_head=True),
    dict(B=2, T=16, H=12, res=True, idt="bf16", odt="bf16", zero_head=False),
    dict(B=3, T=9, H=4, res=False, idt="bf16", odt="f32", zero_head=False),
    dict(B=2, T=17, H=2, res=True, idt="f32", odt="bf16", zero_head=True),
    dict(B=16, T=512, H=12, res=True, idt="bf16", odt="bf16", zero_head=False),
]


def _prepare_case_id(c):
    return "B{B}T{T}H{H}{r}{z}_{idt}_{odt}".format(
        r="_res" if c["res"] else "", z="_zerohead" if c["zero_head"] else "", **c)


def _torch_prepare_end(k, vp, vf, lr, wd, vr, blr, bwd, bvr, ka, kk, H):
    """weight_prepare.rs:282-317 with the LoRA biases added (lora.rs:118-123),
    as torch ops."""
    B, T, C = k.shape
    learning_rate = torch.sigmoid(lr + blr)
    kt = k * (ka * (learning_rate - 1.0) + 1.0)
    v = vp if vf is None else torch.lerp(vp, vf, torch.sigmoid(vr + bvr))
    w = -F.softplus(-(wd + bwd)) - 0.5
    a = -F.normalize((k * kk).reshape(B, T, H, 64), p=2.0, dim=-1, eps=1e-12).reshape(B, T, C)
    return w, kt, v, a, -a * learning_rate


@pytest.mark.parametrize("case", PREPARE_CASES, ids=_prepare_case_id)
def test_weight_prepare_end_matches_torch(case):
    nb = _nb()
    B, T, H, res = case["B"], case["T"], case["H"], case["res"]
    C = H * 64
    idt, odt = DT[case["idt"]], DT[case["odt"]]
    g = torch.Generator().manual_seed(B * 100 + T + 7 * H)
    acts = [torch.randn(B, T, C, generator=g).to(idt) for _ in range(6)]
    acts[4] = (acts[4].float() * 3.0).to(idt)       # decay LoRA: both softplus regimes
    params = [0.5 * torch.randn(C, generator=g) for _ in range(5)]
    params[1] = params[1] - 25.0 * (torch.rand(C, generator=g) > 0.9)   # softplus's linear part
    if case["zero_head"]:
        params[4][64:128] = 0.0                       # key_removal: head 1's norm is clamped
    if not res:
        acts[2] = acts[5] = params[2] = None
    grads = [torch.randn(B, T, C, generator=g).to(odt) for _ in range(5)]

    ins64 = [None if t is None else t.double().requires_grad_(True) for t in acts + params]
    want = _torch_prepare_end(*ins64, H)
    sum((w * gg.double()).sum() for w, gg in zip(want, grads)).backward()

    dev = torch.device("cuda:0")
    ins = [None if t is None else t.to(dev).requires_grad_(True) for t in acts + params]
    announce("weight_prepare_end", _prepare_case_id(case))
    outs = nb.weight_prepare_end(*ins, H, odt)
    sum((o.float() * gg.to(dev).float()).sum() for o, gg in zip(outs, grads)).backward()
    torch.cuda.synchronize()

    names = ("weight_decay", "replacement_key", "value", "removal", "replacement")
    for n, o, w in zip(names, outs, want):
        assert o.dtype == odt
        assert _err(o, w) <= (BF16_TOL if odt == torch.bfloat16 else F32_TOL), n
    in_names = ("key", "value", "value_first", "lr", "wd", "vr", "lr_bias", "wd_bias",
                "vr_bias", "key_replacement", "key_removal")
    for i, (n, a, b) in enumerate(zip(in_names, ins, ins64)):
        if a is None:
            continue
        # bf16 gradients round once; gradients from bf16 output gradients carry their rounding
        tol = BF16_TOL if (idt == torch.bfloat16 and i < 6) or odt == torch.bfloat16 else F32_TOL
        assert _err(a.grad, b.grad) <= tol, n


# ------------------------------------------------------------ the whole model
def test_model_fused_neighbours_match_torch_ops():
    wk = load_pkg().wkv7
    dev = torch.device("cuda:0")
    fused = tiny_model(std=0.2, neighbor_ops="hip").to(dev)
    plain = tiny_model(std=0.2, neighbor_ops="torch").to(dev)
    plain.load_state_dict(fused.state_dict())
    inputs, targets = (t.to(dev) for t in tokens(2, 64, 97))
    announce("model", "neighbor_ops=torch")
    l0, g0 = loss_and_grads(plain, wk.KernelPretrain, inputs, targets)
    announce("model", "neighbor_ops=hip")
    l1, g1 = loss_and_grads(fused, wk.KernelPretrain, inputs, targets)
    torch.cuda.synchronize()
    assert abs(l1 - l0) <= 1e-5 * abs(l0), (l0, l1)
    assert g0.keys() == g1.keys()
    errs = {n: _err(g1[n], g0[n]) for n in g0}
    worst = max(errs, key=errs.get)
    print(f"[fused neighbours] loss {l0:.6f} vs {l1:.6f}; worst grad {worst} {errs[worst]:.3e}")
    assert errs[worst] <= 1e-4, (worst, errs[worst])


def test_weight_prepare_end_with_no_rows():
    """An empty batch: empty outputs, and parameter gradients that are zero
    (written by the kernels, not left as allocated)."""
    nb = _nb()
    dev = torch.device("cuda:0")
    H, C = 2, 128
    acts = [torch.randn(1, 0, C, device=dev).requires_grad_(True) for _ in range(6)]
    params = [torch.full((C,), float("nan"), device=dev).requires_grad_(True) for _ in range(5)]
    announce("weight_prepare_end", "no rows")
    outs = nb.weight_prepare_end(*acts, *params, H, torch.bfloat16)
    assert all(o.shape == (1, 0, C) and o.dtype == torch.bfloat16 for o in outs)
    sum(o.float().sum() for o in outs).backward()
    torch.cuda.synchronize()
    for p in params:
        assert torch.equal(p.grad, torch.zeros(C, device=dev))


def test_parameter_gradients_are_bitwise_repeatable():
    """The per-channel gradients are reduced without atomics, in a fixed
    order: two runs of each fused backward at config[4]'s size give the same
    bits."""
    nb = _nb()
    ll = load_pkg().lm_loss
    dev = torch.device("cuda:0")
    B, T, H = 16, 512, 12
    C = H * 64
    g = torch.Generator(device=dev).manual_seed(77)

    def rnd(*shape, dtype=torch.float32):
        return torch.randn(*shape, generator=g, device=dev).to(dtype)

    x, y, r, k, v = rnd(B, T, C), *(rnd(B, T, H, 64, dtype=torch.bfloat16) for _ in range(4))
    gate = rnd(B, T, C, dtype=torch.bfloat16)
    acts = [rnd(B, T, C, dtype=torch.bfloat16) for _ in range(6)]
    logits, targets = rnd(512, 65536, dtype=torch.bfloat16), torch.randint(0, 65536, (512,), device=dev)
    grads_mix = [rnd(B, T, C, dtype=torch.bfloat16) for _ in range(6)]
    dro, dpre = rnd(B, T, C, dtype=torch.bfloat16), [rnd(B, T, C, dtype=torch.bfloat16) for _ in range(5)]

    def run():
        scales = [torch.linspace(-1, 1, C, device=dev).requires_grad_(True) for _ in range(6)]
        mixes = nb.token_shift_mix(x, scales, out_dtype=torch.bfloat16)
        sum((m.float() * gm.float()).sum() for m, gm in zip(mixes, grads_mix)).backward()
        params = [torch.full((C,), 0.5, device=dev).requires_grad_(True) for _ in range(3)]
        bonus = torch.full((H, 64), 0.1, device=dev).requires_grad_(True)
        out = nb.gated_readout(y, r, k, v, gate, bonus, params[0], params[1])
        (out.float() * dro.float()).sum().backward()
        pp = [torch.full((C,), 0.3, device=dev).requires_grad_(True) for _ in range(5)]
        outs = nb.weight_prepare_end(*acts, *pp, H, torch.bfloat16)
        sum((o.float() * d.float()).sum() for o, d in zip(outs, dpre)).backward()
        lg = logits.clone().requires_grad_(True)
        ll.cross_entropy_l2wrap(lg, targets).backward()
        torch.cuda.synchronize()
        return [s.grad for s in scales] + [bonus.grad, params[0].grad, params[1].grad] + \
            [p.grad for p in pp] + [lg.grad]

    announce("determinism", "token shift, readout, weight preparation, loss")
    first, second = run(), run()
    for i, (a, b) in enumerate(zip(first, second)):
        assert torch.equal(a, b), i


def test_token_shift_past_2g_elements():
    # x [2048, 2048, 768] fp32 (3.2e9 elements, 12.9 GB), one mix in bf16:
    # mixes and dx of the first and last rows against float64 on the CPU
    # (mix_t = x_t + (x_{t-1} - x_t) s, dx_t = g_t (1 - s) + g_{t+1} s), and
    # the scale gradient sum_t g_t (x_{t-1} - x_t) against float64 sums.
    nb = _nb()
    B, T, C = 2048, 2048, 768
    assert B * T * C > 2 ** 31
    announce("token_shift past 2^31 elements", (B, T, C))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5EED00B3)
    x = torch.randn(B, T, C, generator=gen, device="cuda").requires_grad_(True)
    s = (0.5 * torch.rand(C, generator=gen, device="cuda")).requires_grad_(True)
    g = torch.randn(B, T, C, generator=gen, device="cuda").to(torch.bfloat16)
    (mix,) = nb.token_shift_mix(x, [s], out_dtype=torch.bfloat16)
    mix.backward(g)
    torch.cuda.synchronize()
    s64 = s.detach().double().cpu()
    for b in (0, B - 1):
        xs = x.detach()[b].double().cpu()          # one sequence: [T, C]
        gs = g[b].double().cpu()
        prev = torch.cat([torch.zeros(1, C, dtype=torch.float64), xs[:-1]])
        want_mix = xs + (prev - xs) * s64
        nxt = torch.cat([gs[1:], torch.zeros(1, C, dtype=torch.float64)])
        want_dx = gs * (1 - s64) + nxt * s64
        assert _err(mix[b], want_mix) <= BF16_TOL, ("mix", b)
        assert _err(x.grad[b], want_dx) <= F32_TOL, ("dx", b)
    # the scale gradient over all rows, summed in float64 a batch slice at a time
    want_ds = torch.zeros(C, dtype=torch.float64, device="cuda")
    for b0 in range(0, B, 256):
        xb = x.detach()[b0:b0 + 256].double()
        prev = torch.cat([torch.zeros_like(xb[:, :1]), xb[:, :-1]], 1)
        want_ds += (g[b0:b0 + 256].double() * (prev - xb)).sum(dim=(0, 1))
    assert _err(s.grad, want_ds) <= F32_TOL
    del x, g, mix, xb, prev
    torch.cuda.empty_cache()


def test_gated_readout_past_2g_elements():
    # y, r, k, v [2048, 2048, 12, 64] bf16 (3.2e9 elements each, 6.4 GB): the
    # output and the operand gradients of the first and last rows against
    # float64 GroupNorm + bonus + gate on the CPU.
    nb = _nb()
    B, T, H = 2048, 2048, 12
    C = H * 64
    assert B * T * C > 2 ** 31
    announce("gated_readout past 2^31 elements", (B, T, H))
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5EED00B4)
    bf = torch.bfloat16
    y, r, k, v = (torch.randn(B, T, H, 64, generator=gen, device="cuda").to(bf).requires_grad_(True)
                  for _ in range(4))
    gate = torch.rand(B, T, C, generator=gen, device="cuda").to(bf).requires_grad_(True)
    bonus = (0.1 * torch.randn(H, 64, generator=gen, device="cuda")).requires_grad_(True)
    w = (1.0 + 0.1 * torch.randn(C, generator=gen, device="cuda")).requires_grad_(True)
    bias = (0.1 * torch.randn(C, generator=gen, device="cuda")).requires_grad_(True)
    dout = torch.randn(B, T, C, generator=gen, device="cuda").to(bf)
    out = nb.gated_readout(y, r, k, v, gate, bonus, w, bias, eps=64e-5)
    out.backward(dout)
    torch.cuda.synchronize()
    for b, t0 in ((0, 0), (B - 1, T - 4)):
        sl = lambda z: z.detach()[b, t0:t0 + 4].double().cpu().requires_grad_(True)
        y4, r4, k4, v4, g4 = sl(y), sl(r), sl(k), sl(v), sl(gate)
        bo, w64, b64 = (z.detach().double().cpu() for z in (bonus, w, bias))
        yn = F.group_norm(y4.reshape(4, C), H, w64, b64, 64e-5).reshape(4, C)
        bon = ((r4 * k4 * bo).sum(-1, keepdim=True) * v4).reshape(4, C)
        want = (yn + bon) * g4
        (want * dout[b, t0:t0 + 4].double().cpu()).sum().backward()
        assert _err(out[b, t0:t0 + 4], want) <= BF16_TOL, ("out", b)
        for name, got, ref in (("y", y, y4), ("r", r, r4), ("k", k, k4), ("v", v, v4),
                               ("gate", gate, g4)):
            assert _err(got.grad[b, t0:t0 + 4], ref.grad) <= BF16_TOL, (name, b)
    del y, r, k, v, gate, dout, out
    torch.cuda.empty_cache()
