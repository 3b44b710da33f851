"""GPU parity of the gfx950 kernels (called through the C ABI in
include/wkv7.h via the rwkv-rs_amd.wkv7 mirror) against the CPU oracle, which
restates /root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs.

Tolerances (the target's own): fp32 inputs, relative L2 <= 1e-5 per
tensor; bf16 inputs with fp32 state, relative L2 <= 1e-2 per tensor. For bf16
inputs the fp32 state-family outputs (checkpoints, removal_state, final state,
initial-state gradient) are also held to 1e-4: the chunked matrix-core forward
forms its products from hi/lo bf16 splits (about 16 significant bits) and
measures 2e-6 to 7e-6 against the fp32 oracle."""

import ctypes

import numpy as np
import pytest
import torch

from conftest import GRAD_NAMES, NAMES, announce, load_pkg, rel_l2, to_dev, to_np

pytestmark = pytest.mark.gpu

FP32_TOL = 1e-5
BF16_TOL = 1e-2
BF16_STATE_TOL = 1e-4


@pytest.fixture(scope="module")
def wk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return load_pkg().wkv7


def run_gpu(wk, d, chunk_len, dtype, s0=True, dsT=None):
    ins = [to_dev(d[n], dtype) for n in NAMES]
    s0_t = to_dev(d["s0"]) if (s0 and d["s0"] is not None) else None
    if s0_t is None:
        s0_t = torch.zeros(ins[0].shape[0], ins[0].shape[2], 64, 64, device="cuda")
    fwd = wk.wkv7_statepass_forward(*ins, s0_t, chunk_len)
    dy = to_dev(d["dy"], dtype)
    dsT_t = to_dev(dsT) if dsT is not None else torch.zeros_like(s0_t)
    bwd = wk.wkv7_statepass_backward(*ins, fwd.state, fwd.removal_state, dy, dsT_t, chunk_len)
    torch.cuda.synchronize()
    return fwd, bwd


def run_oracle(oracle, d, chunk_len, dsT=None):
    ins = [d[n] for n in NAMES]
    fwd = oracle.forward_f32(*ins, s0=d["s0"], chunk_len=chunk_len)
    bwd = oracle.backward_f32(*ins, fwd["state"], fwd["removal_state"], d["dy"],
                              ds_T=dsT, chunk_len=chunk_len)
    return fwd, bwd


def compare(fwd, bwd, ofwd, obwd, tok_tol, label, state_tol=FP32_TOL):
    errs = {
        "output": rel_l2(to_np(fwd.output), ofwd["output"]),
        "removal_state": rel_l2(to_np(fwd.removal_state), ofwd["removal_state"]),
        "state": rel_l2(to_np(fwd.state), ofwd["state"]),
        "final_state": rel_l2(to_np(fwd.final_state), ofwd["final_state"]),
        "initial_state_grad": rel_l2(to_np(bwd.initial_state_grad), obwd["initial_state_grad"]),
    }
    for gn in GRAD_NAMES:
        errs[gn] = rel_l2(to_np(getattr(bwd, gn)), obwd[gn])
    print(label, {k: f"{v:.2e}" for k, v in errs.items()}, flush=True)
    tok = ("output",) + GRAD_NAMES
    for key, err in errs.items():
        assert err <= (tok_tol if key in tok else state_tol), (label, key, err)
    return errs


@pytest.mark.parametrize("case", [
    # (B, T, H, chunk_len, s0_std, with_dsT, seed)
    (1, 64, 4, 16, None, False, 0),      # config[0]
    (1, 64, 4, 16, 0.1, True, 1),
    (2, 48, 3, 16, 0.1, True, 2),
    (1, 64, 2, 8, None, True, 3),
    (1, 32, 2, 1, 0.1, True, 4),
    (1, 24, 2, 8, 0.1, False, 5),        # T not a multiple of the 16-step tile
    (1, 20, 1, 4, None, True, 6),
    (3, 1, 5, 1, 0.1, True, 7),          # single step
])
def test_fp32_forward_backward_matches_oracle(wk, oracle, case):
    B, T, H, C, s0_std, with_dsT, seed = case
    announce("fp32 fwd+bwd", case)
    d = load_pkg().synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std)
    dsT = (np.random.default_rng(seed + 50).standard_normal((B, H, 64, 64)).astype(np.float32)
           if with_dsT else None)
    if d["s0"] is None:
        d["s0"] = np.zeros((B, H, 64, 64), np.float32)
    fwd, bwd = run_gpu(wk, d, C, torch.float32, dsT=dsT)
    ofwd, obwd = run_oracle(oracle, d, C, dsT=dsT)
    compare(fwd, bwd, ofwd, obwd, FP32_TOL, f"fp32 {case}")


def test_fp32_gradients_match_fp64(wk, oracle):
    # the kernel against exact (fp64, stored-state) gradients at config[0]
    announce("fp32 vs fp64 grads, config[0]")
    d = load_pkg().synthetic.make_inputs(1, 64, 4, 64, seed=0)
    d["s0"] = np.zeros((1, 4, 64, 64), np.float32)
    fwd, bwd = run_gpu(wk, d, 16, torch.float32)
    ref = oracle.grad_f64(*(d[n] for n in NAMES), d["s0"], d["dy"])
    f64 = oracle.forward_f64(*(d[n] for n in NAMES), s0=d["s0"])
    assert rel_l2(to_np(fwd.output), f64["output"]) < FP32_TOL
    for gn in GRAD_NAMES + ("initial_state_grad",):
        err = rel_l2(to_np(getattr(bwd, gn)), ref[gn])
        assert err < FP32_TOL, (gn, err)


@pytest.mark.parametrize("case", [
    (1, 96, 2, 32, 0.1, 8),   # two 16-step tiles per checkpoint interval
    (1, 48, 2, 24, 0.1, 9),   # a checkpoint in the middle of a forward tile
])
def test_fp32_long_chunks_as_accurate_as_reference(wk, oracle, case):
    # The backward rebuilds S_{t-1} = (S_t - v k^T - sa b^T) / w~ (kernel.rs:239-246),
    # which amplifies rounding roughly 1.35x per step between checkpoints: at
    # chunk_len 24-32 the reference algorithm itself is off the exact gradient by
    # 1e-5 .. 1e-3, and any two fp32 evaluations of it differ by as much. The
    # gradients that use the rebuilt S (dw, dr, da) are therefore held to the
    # reference algorithm's own accuracy against exact fp64 gradients; everything
    # else, which does not pass through the rebuild, to the fp32 tolerance.
    B, T, H, C, s0_std, seed = case
    announce("fp32 long chunk", case)
    d = load_pkg().synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std)
    dsT = np.random.default_rng(seed + 50).standard_normal((B, H, 64, 64)).astype(np.float32)
    fwd, bwd = run_gpu(wk, d, C, torch.float32, dsT=dsT)
    ofwd, obwd = run_oracle(oracle, d, C, dsT=dsT)
    exact = oracle.grad_f64(*(d[n] for n in NAMES), d["s0"], d["dy"], ds_T=dsT)
    for key, got, want in (("output", fwd.output, ofwd["output"]),
                           ("removal_state", fwd.removal_state, ofwd["removal_state"]),
                           ("state", fwd.state, ofwd["state"]),
                           ("final_state", fwd.final_state, ofwd["final_state"])):
        assert rel_l2(to_np(got), want) <= FP32_TOL, key
    rebuilt = ("weight_decay_grad", "receptance_grad", "removal_grad")
    for gn in GRAD_NAMES + ("initial_state_grad",):
        got = to_np(getattr(bwd, gn))
        if gn in rebuilt:
            ref_err = rel_l2(obwd[gn], exact[gn])
            err = rel_l2(got, exact[gn])
            print(case, gn, f"gpu {err:.2e} reference-algorithm {ref_err:.2e}", flush=True)
            assert err <= 5 * ref_err + 1e-6, (gn, err, ref_err)
        else:
            assert rel_l2(got, obwd[gn]) <= FP32_TOL, gn


CRITERION_SHAPES = [   # (B, T, H, chunk_len): crates/rwkv-nn/benches/kernels/mod.rs:108-113
    (1, 128, 8, 32),
    (2, 256, 8, 32),
    (4, 512, 16, 64),
]


@pytest.mark.parametrize("shape", CRITERION_SHAPES)
@pytest.mark.parametrize("conditioned", [True, False], ids=["w_near_1", "synthetic"])
def test_fp32_at_the_criterion_shapes(wk, oracle, shape, conditioned):
    # The reference's Criterion bench shapes with fp32 operands: at chunk_len
    # 32 the forward and the backward run on the fp32 chunked matrix-core
    # kernels; at 64 with 64 (batch, head) pairs both run on the step
    # kernels (test_forward_kernel_choice and test_fp32_backward_kernel_choice
    # below).
    # The benches draw every input N(0, 1), under which
    # the state grows without bound (timing inputs, not a parity case), so
    # the inputs here are the synthetic distributions. With the decay logits
    # shifted by -6 (w~ within 0.2% of one) the reversal between checkpoints
    # (kernel.rs:239-246) amplifies nothing and every tensor, the rebuilt-
    # state gradients dw, dr, da included, is held to 1e-5 against the
    # oracle; a wrong rebuild of the start states, or a wrong hand-over of
    # them between the kernel's wave groups, moves those by O(1). Unshifted,
    # the reference algorithm itself is off the exact gradients by 4e-4 at
    # chunk_len 32 and by more than the gradients' size at 64 (measured), so
    # there dw, dr, da are held to five times its own error against fp64.
    B, T, H, C = shape
    announce("fp32 chunked, Criterion shape", shape, "w~ near 1" if conditioned else "synthetic")
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(B, T, H, 64, seed=40 + C + B, s0_std=0.1)
    if conditioned:
        d["w"] = (d["w"] - 6.0).astype(np.float32)
    dsT = np.random.default_rng(B + T).standard_normal((B, H, 64, 64)).astype(np.float32)
    fwd, bwd = run_gpu(wk, d, C, torch.float32, dsT=dsT)
    ofwd, obwd = run_oracle(oracle, d, C, dsT=dsT)
    exact = oracle.grad_f64(*(d[n] for n in NAMES), d["s0"], d["dy"], ds_T=dsT)
    rebuilt = ("weight_decay_grad", "receptance_grad", "removal_grad")
    if conditioned:
        for gn in rebuilt:
            assert rel_l2(obwd[gn], exact[gn]) <= 1e-5, gn   # the case is well conditioned
        compare(fwd, bwd, ofwd, obwd, FP32_TOL, f"fp32 chunked {shape} w~1")
        return
    for key in ("output", "removal_state", "state", "final_state"):
        assert rel_l2(to_np(getattr(fwd, key)), ofwd[key]) <= FP32_TOL, key
    for gn in GRAD_NAMES + ("initial_state_grad",):
        got = to_np(getattr(bwd, gn))
        if gn in rebuilt:
            ref_err = rel_l2(obwd[gn], exact[gn])
            err = rel_l2(got, exact[gn])
            print(shape, gn, f"gpu {err:.2e} reference-algorithm {ref_err:.2e}", flush=True)
            assert err <= 5 * ref_err + 1e-6, (gn, err, ref_err)
        else:
            assert rel_l2(got, obwd[gn]) <= FP32_TOL, gn


@pytest.mark.parametrize("case", [
    # (B, T, H, chunk_len, s0_std, seed)
    (3, 32, 100, 16, 0.1, 60),   # 300 (batch, head) pairs: more workgroups than CUs
    (1, 144, 2, 48, 0.1, 61),    # three 16-step chunks per checkpoint (step kernels)
    (2, 64, 5, 32, None, 62),    # zero initial state, an odd head count
    (1, 16, 3, 16, 0.1, 63),     # one chunk: the start state by the reversal alone
    (2, 96, 128, 48, 0.1, 64),   # 256 pairs: the chunked backward at chunk_len 48
    (1, 64, 256, 64, None, 65),  # 256 pairs: the chunked backward at chunk_len 64
])
def test_fp32_chunked_kernels_more_shapes(wk, oracle, case):
    # More shapes on the fp32 chunked kernels, with the decay logits shifted
    # by -6 as above, so that every tensor, dw, dr and da included, is held
    # to 1e-5 against the oracle at any chunk_len. Past chunk_len 32 the
    # forward runs the step kernel, and the backward the chunked kernel from
    # 256 (batch, head) pairs up, the step kernel below.
    B, T, H, C, s0_std, seed = case
    announce("fp32 chunked, w~ near 1", case)
    d = load_pkg().synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std)
    d["w"] = (d["w"] - 6.0).astype(np.float32)
    if d["s0"] is None:
        d["s0"] = np.zeros((B, H, 64, 64), np.float32)
    dsT = np.random.default_rng(seed).standard_normal((B, H, 64, 64)).astype(np.float32)
    fwd, bwd = run_gpu(wk, d, C, torch.float32, dsT=dsT)
    ofwd, obwd = run_oracle(oracle, d, C, dsT=dsT)
    compare(fwd, bwd, ofwd, obwd, FP32_TOL, f"fp32 chunked w~1 {case}")


@pytest.mark.parametrize("case", [
    # (dtype, B, T, H, chunk_len, expected kernel of the forward)
    ("f32", 2, 64, 4, 16, "chunked"),
    ("f32", 2, 64, 4, 32, "chunked"),
    ("f32", 1, 96, 4, 48, "step"),
    ("f32", 1, 128, 4, 64, "step"),
    ("bf16", 2, 64, 4, 16, "chunked"),
    ("bf16", 2, 64, 4, 32, "chunked"),
    ("bf16", 1, 128, 4, 64, "step"),
])
def test_forward_kernel_choice(wk, case):
    # The forward's kernel choice (chunk_forward_supported in
    # wkv7_chunk_forward.hip, chunk_f32_forward_supported in
    # wkv7_f32_chunk.hip): past chunk_len 32 the default call gives the step
    # kernel's outputs and checkpoints bit for bit (their reference-order
    # checkpoints keep the rebuilt-state gradients at the reference
    # algorithm's accuracy); at 16 and 32 a chunked kernel's.
    dtype, B, T, H, C, expected = case
    announce("forward kernel choice", case)
    bf16 = dtype == "bf16"
    dt = torch.bfloat16 if bf16 else torch.float32
    d = load_pkg().synthetic.make_inputs(B, T, H, 64, seed=67, s0_std=0.1, bf16=bf16)
    ins = [to_dev(d[n], dt) for n in NAMES]
    s0 = to_dev(d["s0"])
    auto = wk.wkv7_statepass_forward(*ins, s0, C)
    step = wk.wkv7_forward_ex(*ins, s0, C, kernels="step")
    torch.cuda.synchronize()
    same = torch.equal(auto.state, step.state) and torch.equal(auto.output, step.output)
    assert same == (expected == "step"), (case, same)
    assert rel_l2(to_np(auto.state), to_np(step.state)) < (1e-4 if bf16 else 1e-5)


@pytest.mark.parametrize("case", [
    # (B, T, H, chunk_len, expected kernel of the backward)
    (4, 128, 16, 64, "step"),      # 64 pairs, chunk_len 64: the step kernel
    (4, 64, 16, 32, "chunked"),    # 64 pairs, chunk_len 32: the chunked kernel
    (1, 64, 256, 64, "chunked"),   # 256 pairs (one per CU), chunk_len 64: chunked
    (1, 32, 8, 16, "chunked"),     # chunk_len 16: chunked at any size
])
def test_fp32_backward_kernel_choice(wk, case):
    # The fp32 backward's kernel choice (chunk_f32_backward_preferred in
    # wkv7_f32_chunk.hip): the default call gives the step kernels' result bit
    # for bit where they are picked, and another result (the chunked kernel's
    # different summation order) where the chunked kernel is. Decay logits
    # shifted by -6 (w~ near 1), so that the reversal between checkpoints
    # keeps the two kernels' results close at chunk_len 64.
    B, T, H, C, expected = case
    announce("fp32 backward kernel choice", case)
    d = load_pkg().synthetic.make_inputs(B, T, H, 64, seed=66, s0_std=0.1)
    d["w"] = (d["w"] - 6.0).astype(np.float32)
    ins = [to_dev(d[n], torch.float32) for n in NAMES]
    s0 = to_dev(d["s0"])
    fwd = wk.wkv7_statepass_forward(*ins, s0, C)
    dy = to_dev(d["dy"], torch.float32)
    dsT = torch.zeros_like(s0)
    auto = wk.wkv7_statepass_backward(*ins, fwd.state, fwd.removal_state, dy, dsT, C)
    step = wk.wkv7_backward_ex(*ins, fwd.state, fwd.removal_state, dy, dsT, C, kernels="step")
    torch.cuda.synchronize()
    same = all(torch.equal(getattr(auto, gn), getattr(step, gn)) for gn in GRAD_NAMES)
    assert same == (expected == "step"), (case, same)
    for gn in GRAD_NAMES:   # either way both are the reference's gradients
        assert rel_l2(to_np(getattr(auto, gn)), to_np(getattr(step, gn))) < 1e-3, gn


@pytest.mark.parametrize("case", [
    (2, 128, 4, 16, 0.1, 11),   # 16-step checkpoints, 32-step forward tiles (two per tile)
    (1, 64, 4, 16, None, 12),
    (1, 48, 3, 16, 0.1, 13),    # T not a multiple of 32: partial last forward tile
    (1, 40, 2, 8, 0.1, 14),     # backward reloads inside a 16-step tile, partial first tile
    (1, 64, 2, 32, 0.1, 15),    # one checkpoint every 32-step forward tile
    (3, 32, 100, 16, 0.1, 16),  # 300 (batch, head) pairs: more workgroups than CUs
])
def test_bf16_inputs_fp32_state(wk, oracle, case):
    B, T, H, C, s0_std, seed = case
    announce("bf16 fwd+bwd", case)
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std, bf16=True)
    if d["s0"] is None:
        d["s0"] = np.zeros((B, H, 64, 64), np.float32)
    fwd, bwd = run_gpu(wk, d, C, torch.bfloat16)
    assert fwd.output.dtype == torch.bfloat16 and fwd.state.dtype == torch.float32
    assert bwd.key_grad.dtype == torch.bfloat16 and bwd.initial_state_grad.dtype == torch.float32
    ofwd, obwd = run_oracle(oracle, d, C)
    # the reference casts y and the six gradients back to bf16 (host.rs:58-62, 221-228)
    ofwd["output"] = pkg.synthetic.bf16_round(ofwd["output"])
    for gn in GRAD_NAMES:
        obwd[gn] = pkg.synthetic.bf16_round(obwd[gn])
    compare(fwd, bwd, ofwd, obwd, BF16_TOL, f"bf16 {case}", BF16_STATE_TOL)


@pytest.mark.parametrize("case", [
    (2, 128, 4, 32, 0.1, 21),   # two 16-step chunks per checkpoint
    (1, 96, 3, 48, None, 22),   # three
    (1, 192, 2, 64, 0.1, 23),   # four: start states rebuilt over up to 48 steps
])
def test_bf16_long_chunks_on_the_chunked_kernels(wk, oracle, case):
    # chunk_len > 16 with bf16 operands: the forward in fp32 (at 32 the fp32
    # chunked kernel, the bf16 rows widened as the reference casts them; past
    # 32 the step kernel), fp32 checkpoints every chunk_len steps, and the
    # chunked backward, which
    # rebuilds the start states of the 16-step chunks between checkpoints by
    # the reference's reversal (kernel.rs:239-246). The forward's fp32 state
    # family is held to the fp32 bar, y and the gradients that do not read a
    # rebuilt state to the bf16 bars against the oracle; dw, dr and da, which
    # do, to the reference algorithm's own accuracy (the oracle in fp32
    # against exact fp64 gradients, which is what grows with chunk_len) plus
    # bf16 rounding.
    B, T, H, C, s0_std, seed = case
    announce("bf16 long chunk", case)
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std, bf16=True)
    if d["s0"] is None:
        d["s0"] = np.zeros((B, H, 64, 64), np.float32)
    fwd, bwd = run_gpu(wk, d, C, torch.bfloat16)
    ofwd, obwd = run_oracle(oracle, d, C)
    exact = oracle.grad_f64(*(d[n] for n in NAMES), d["s0"], d["dy"])
    assert rel_l2(to_np(fwd.output), pkg.synthetic.bf16_round(ofwd["output"])) <= BF16_TOL
    for key in ("removal_state", "state", "final_state"):
        assert rel_l2(to_np(getattr(fwd, key)), ofwd[key]) <= FP32_TOL, key
    assert fwd.state.shape[2] == T // C
    rebuilt = ("weight_decay_grad", "receptance_grad", "removal_grad")
    for gn in GRAD_NAMES + ("initial_state_grad",):
        got = to_np(getattr(bwd, gn))
        if gn in rebuilt:
            ref_err = rel_l2(obwd[gn], exact[gn])
            err = rel_l2(got, exact[gn])
            print(case, gn, f"gpu {err:.2e} reference-algorithm {ref_err:.2e}", flush=True)
            assert err <= 5 * ref_err + BF16_TOL, (gn, err, ref_err)
        elif gn == "initial_state_grad":
            assert rel_l2(got, obwd[gn]) <= BF16_STATE_TOL, gn
        else:
            assert rel_l2(got, pkg.synthetic.bf16_round(obwd[gn])) <= BF16_TOL, gn


@pytest.mark.parametrize("case", [
    (1, 96, 3, 48, 0.1, 25),
    (1, 192, 2, 64, 0.1, 26),
    (2, 128, 2, 32, None, 27),
])
def test_bf16_long_chunks_well_conditioned(wk, oracle, case):
    # The long-chunk test above can only hold dw, dr and da to the reference
    # algorithm's own (large) error, because its decays amplify the reversal's
    # rounding by 1/w~ ~ 1.35 per step. Here the decay logits are shifted by
    # -6, so w~ = exp(-e^{-1/2} sigmoid(x - 6)) is within 0.2% of one and the
    # reversal (kernel.rs:239-246) amplifies nothing: every tensor, the rebuilt-
    # state gradients included, is held to the bf16 bars against the oracle.
    # A wrong rebuild of the start states between checkpoints in the chunked
    # backward (template instance kLong) moves dw, dr and da by O(1).
    B, T, H, C, s0_std, seed = case
    announce("bf16 long chunk, w~ near 1", case)
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std, bf16=True)
    d["w"] = pkg.synthetic.bf16_round(d["w"] - 6.0)
    if d["s0"] is None:
        d["s0"] = np.zeros((B, H, 64, 64), np.float32)
    fwd, bwd = run_gpu(wk, d, C, torch.bfloat16)
    ofwd, obwd = run_oracle(oracle, d, C)
    exact = oracle.grad_f64(*(d[n] for n in NAMES), d["s0"], d["dy"])
    for gn in ("weight_decay_grad", "receptance_grad", "removal_grad"):
        print(case, gn, f"reference algorithm vs exact {rel_l2(obwd[gn], exact[gn]):.2e}",
              flush=True)
        assert rel_l2(obwd[gn], exact[gn]) <= 1e-4, gn   # the case is well conditioned
    ofwd["output"] = pkg.synthetic.bf16_round(ofwd["output"])
    for gn in GRAD_NAMES:
        obwd[gn] = pkg.synthetic.bf16_round(obwd[gn])
    compare(fwd, bwd, ofwd, obwd, BF16_TOL, f"bf16 long chunk w~1 {case}", BF16_STATE_TOL)


def test_bf16_statetune_on_the_chunked_kernels(wk, oracle):
    # the statetune flags (s0 in, no s_T; no ds_T, ds0 out:
    # wkv7_statetune/forward.rs:19-76) with bf16 operands, i.e. on the chunked
    # kernels, against the oracle with the same flags
    announce("bf16 statetune", (2, 64, 3, 16))
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(2, 64, 3, 64, seed=28, s0_std=0.1, bf16=True)
    ins = [to_dev(d[n], torch.bfloat16) for n in NAMES]
    s0 = to_dev(d["s0"])
    f = wk.wkv7_statetune_forward(*ins, s0, 16)
    g = wk.wkv7_statetune_backward(*ins, f.state, f.removal_state,
                                   to_dev(d["dy"], torch.bfloat16), 16)
    torch.cuda.synchronize()
    ofwd, obwd = run_oracle(oracle, d, 16)
    assert rel_l2(to_np(f.output), pkg.synthetic.bf16_round(ofwd["output"])) <= BF16_TOL
    for key in ("state", "removal_state"):
        assert rel_l2(to_np(getattr(f, key)), ofwd[key]) <= BF16_STATE_TOL, key
    for gn in GRAD_NAMES:
        err = rel_l2(to_np(getattr(g, gn)), pkg.synthetic.bf16_round(obwd[gn]))
        assert err <= BF16_TOL, (gn, err)
    err = rel_l2(to_np(g.initial_state_grad), obwd["initial_state_grad"])
    assert err <= BF16_STATE_TOL, err


def test_long_chunk_bf16_backward_matches_step_backward(wk):
    # chunk_len 32 with bf16 operands: the forward runs the fp32 chunked
    # kernel (its fp32 checkpoints are what the rebuild between checkpoints
    # needs) and the backward the chunked kernels; on the same checkpoints
    # the step backward gives the same gradients to bf16 rounding
    announce("bf16 chunk_len 32 chunked vs step backward", (1, 64, 2, 32))
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(1, 64, 2, 64, seed=24, s0_std=0.1, bf16=True)
    dev = torch.device("cuda:0")
    ins = [torch.from_numpy(d[n]).to(dev).to(torch.bfloat16) for n in NAMES]
    s0 = torch.from_numpy(d["s0"]).to(dev)
    dy = torch.from_numpy(d["dy"]).to(dev).to(torch.bfloat16)
    f = wk.wkv7_forward_ex(*ins, s0, 32)
    a = wk.wkv7_backward_ex(*ins, f.state, f.removal_state, dy, torch.zeros_like(s0), 32)
    b = wk.wkv7_backward_ex(*ins, f.state, f.removal_state, dy, torch.zeros_like(s0), 32,
                            kernels="step")
    torch.cuda.synchronize()
    for gn in GRAD_NAMES:
        assert rel_l2(to_np(getattr(a, gn)), to_np(getattr(b, gn))) <= BF16_TOL, gn
    assert rel_l2(to_np(a.initial_state_grad), to_np(b.initial_state_grad)) <= BF16_STATE_TOL


def test_variants_agree(wk):
    # pretrain == statepass(s0 = 0) == statetune(s0 = 0) on y and the six gradients
    announce("variant equivalence")
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(2, 32, 3, 64, seed=21)
    ins = [to_dev(d[n]) for n in NAMES]
    dy = to_dev(d["dy"])
    z = torch.zeros(2, 3, 64, 64, device="cuda")
    inp = wk.Wkv7ForwardInput(receptance=ins[1], weight_decay=ins[0], replacement_key=ins[2],
                              value=ins[3], removal_key_normalized=ins[4], replacement=ins[5])
    pre = wk.wkv7_pretrain_forward(inp, 16)
    sp = wk.wkv7_statepass_forward(*ins, z, 16)
    st = wk.wkv7_statetune_forward(*ins, z, 16)
    for o in (sp, st):
        assert torch.equal(o.output, pre.output) and torch.equal(o.state, pre.state)
        assert torch.equal(o.removal_state, pre.removal_state)
    gp = wk.wkv7_pretrain_backward(*ins, pre.state, pre.removal_state, dy, 16)
    gs = wk.wkv7_statepass_backward(*ins, sp.state, sp.removal_state, dy, z, 16)
    gt = wk.wkv7_statetune_backward(*ins, st.state, st.removal_state, dy, 16)
    for gn in GRAD_NAMES:
        assert torch.equal(getattr(gs, gn), getattr(gp, gn)), gn
        assert torch.equal(getattr(gt, gn), getattr(gp, gn)), gn
    assert torch.equal(gs.initial_state_grad, gt.initial_state_grad)


def test_sequence_split_is_exact(wk):
    # statepass contract (model.rs:368-409): two halves with s_T -> s0 equal one run
    announce("split invariance")
    d = load_pkg().synthetic.make_inputs(2, 64, 2, 64, seed=22, s0_std=0.1)
    ins = [to_dev(d[n]) for n in NAMES]
    s0 = to_dev(d["s0"])
    full = wk.wkv7_statepass_forward(*ins, s0, 16)
    a = wk.wkv7_statepass_forward(*(x[:, :32] for x in ins), s0, 16)
    b = wk.wkv7_statepass_forward(*(x[:, 32:] for x in ins), a.final_state, 16)
    assert torch.equal(torch.cat([a.output, b.output], 1), full.output)
    assert torch.equal(b.final_state, full.final_state)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16], ids=["fp32", "bf16"])
@pytest.mark.parametrize("chunk_len", [16, 32])
def test_empty_sequence(wk, dtype, chunk_len):
    # T = 0: final state = initial state, initial-state grad = final-state grad.
    # Both chunked forwards run with no chunks (bf16 at chunk_len 16 the
    # split-bf16 one, fp32 and bf16 at 32 the fp32 one).
    announce("T=0", str(dtype), chunk_len)
    B, H = 2, 3
    e = torch.empty(B, 0, H, 64, device="cuda", dtype=dtype)
    s0 = torch.randn(B, H, 64, 64, device="cuda")
    out = wk.wkv7_statepass_forward(e, e, e, e, e, e, s0, chunk_len)
    assert out.output.shape == (B, 0, H, 64) and out.state.shape == (B, H, 0, 64, 64)
    assert torch.equal(out.final_state, s0)
    dsT = torch.randn(B, H, 64, 64, device="cuda")
    g = wk.wkv7_statepass_backward(e, e, e, e, e, e, out.state, out.removal_state, e, dsT,
                                   chunk_len)
    assert torch.equal(g.initial_state_grad, dsT)


def test_two_streams_match_one(wk):
    # The C ABI enqueues on the caller's stream and keeps no state between
    # calls (include/wkv7.h): two workloads launched alternately on two
    # streams -- bf16 and fp32 operands, each on its chunked kernels --
    # give each workload's one-stream results bit for bit.
    announce("two streams")
    syn = load_pkg().synthetic
    work = []
    for seed, dtype in ((31, torch.bfloat16), (32, torch.float32)):
        d = syn.make_inputs(2, 128, 4, 64, seed=seed, s0_std=0.1)
        ins = [to_dev(d[n], dtype) for n in NAMES]
        work.append((ins, to_dev(d["s0"]), to_dev(d["dy"], dtype)))

    def run(ins, s0, dy):
        f = wk.wkv7_statepass_forward(*ins, s0, 16)
        g = wk.wkv7_statepass_backward(*ins, f.state, f.removal_state, dy,
                                       torch.zeros_like(s0), 16)
        return f, g

    one = [run(*w) for w in work]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    fwd = [None, None]
    for i, (s, (ins, s0, dy)) in enumerate(zip(streams, work)):
        with torch.cuda.stream(s):
            fwd[i] = wk.wkv7_statepass_forward(*ins, s0, 16)
    two = []
    for i, (s, (ins, s0, dy)) in enumerate(zip(streams, work)):
        with torch.cuda.stream(s):
            f = fwd[i]
            two.append((f, wk.wkv7_statepass_backward(*ins, f.state, f.removal_state, dy,
                                                      torch.zeros_like(s0), 16)))
    torch.cuda.synchronize()
    for (f1, g1), (f2, g2) in zip(one, two):
        for name in ("output", "state", "removal_state", "final_state"):
            assert torch.equal(getattr(f1, name), getattr(f2, name)), name
        for gn in GRAD_NAMES + ("initial_state_grad",):
            assert torch.equal(getattr(g1, gn), getattr(g2, gn)), gn


@pytest.mark.parametrize("dtype,chunk_len", [("bf16", 16), ("f32", 16), ("bf16", 32)])
def test_graph_replays_match_eager(wk, dtype, chunk_len):
    # The forward and backward launch kernels only (no memsets, copies or
    # allocations inside the library), so a caller can capture them in a HIP
    # graph: each of several replays, with eager work between them, gives
    # the eager results bit for bit (bf16 and fp32 operands: the chunked
    # kernels of each, bf16 at chunk_len 32 on the fp32 chunked forward and
    # the long-chunk bf16 backward; the fp32 forward looks up its fault
    # counter's address at every launch, captured ones included).
    announce("graph replay", dtype, chunk_len)
    bf16 = dtype == "bf16"
    dt = torch.bfloat16 if bf16 else torch.float32
    d = load_pkg().synthetic.make_inputs(2, 128, 4, 64, seed=41, s0_std=0.1, bf16=bf16)
    ins = [to_dev(d[n], dt) for n in NAMES]
    s0, dy = to_dev(d["s0"]), to_dev(d["dy"], dt)
    zero = torch.zeros_like(s0)

    def run():
        f = wk.wkv7_statepass_forward(*ins, s0, chunk_len)
        return f, wk.wkv7_statepass_backward(*ins, f.state, f.removal_state, dy, zero, chunk_len)

    ef, eg = run()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        run()                                  # warm-up off the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        gf, gg = run()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for name in ("output", "state", "removal_state", "final_state"):
            assert torch.equal(getattr(gf, name), getattr(ef, name)), name
        for gn in GRAD_NAMES + ("initial_state_grad",):
            assert torch.equal(getattr(gg, gn), getattr(eg, gn)), gn
        run()                                  # eager work between replays
        torch.cuda.synchronize()


def test_autograd_matches_direct_backward(wk):
    announce("autograd")
    d = load_pkg().synthetic.make_inputs(1, 32, 2, 64, seed=23, s0_std=0.1)
    ins = [to_dev(d[n]).requires_grad_(True) for n in NAMES]
    s0 = to_dev(d["s0"]).requires_grad_(True)
    dy = to_dev(d["dy"])
    y, sT = wk.Wkv7StatePassFunction.apply(*ins, s0, 16)
    y.backward(dy)
    direct_f = wk.wkv7_statepass_forward(*(x.detach() for x in ins), s0.detach(), 16)
    direct = wk.wkv7_statepass_backward(*(x.detach() for x in ins), direct_f.state,
                                        direct_f.removal_state, dy, torch.zeros_like(s0), 16)
    for x, gn in zip(ins, GRAD_NAMES):
        assert torch.equal(x.grad, getattr(direct, gn)), gn
    assert torch.equal(s0.grad, direct.initial_state_grad)
    assert torch.equal(sT, direct_f.final_state)


def check_every_pair(pkg, fwd, bwd, ins, s0, dy, oracle, label, state_family=True):
    """Every (b, h) pair of a full-size run against the oracle over all steps:
    output and the six gradients (bf16, rounded like the reference's cast back,
    wkv7_common/host.rs:58-62, 221-228) within 1e-2 per pair, the fp32 state
    family within 1e-4 per pair."""
    ins_np = [to_np(x) for x in ins]
    of = oracle.forward_f32(*ins_np, s0=None if s0 is None else to_np(s0), chunk_len=16)
    ob = oracle.backward_f32(*ins_np, of["state"], of["removal_state"], to_np(dy), chunk_len=16,
                             write_initial_state_grad=state_family)
    worst = {}
    checks = [("output", fwd.output, pkg.synthetic.bf16_round(of["output"]), BF16_TOL)]
    for gn in GRAD_NAMES:
        checks.append((gn, getattr(bwd, gn), pkg.synthetic.bf16_round(ob[gn]), BF16_TOL))
    checks.append(("removal_state", fwd.removal_state, of["removal_state"], BF16_STATE_TOL))
    checks.append(("state", fwd.state, of["state"], BF16_STATE_TOL))
    if state_family:
        checks.append(("final_state", fwd.final_state, of["final_state"], BF16_STATE_TOL))
        checks.append(("initial_state_grad", bwd.initial_state_grad, ob["initial_state_grad"],
                       BF16_STATE_TOL))
    for name, got, want, tol in checks:
        e = pair_rel_l2(to_np(got), want, per_token=got.dim() == 4 and name not in (
            "final_state", "initial_state_grad"))
        worst[name] = float(e.max())
        bad = np.argwhere(~(e <= tol))
        assert bad.size == 0, (label, name, bad[:4].tolist(), float(e.max()))
    print(label, "worst pair", {k: f"{v:.2e}" for k, v in worst.items()}, flush=True)


def pair_rel_l2(got, want, per_token):
    """Relative L2 error of every (b, h) pair, as a [B, H] array: per-token
    tensors are [B, T, H, N], state-family tensors [B, H, ...]."""
    B = got.shape[0]
    H = got.shape[2] if per_token else got.shape[1]
    out = np.empty((B, H), np.float64)
    for bi in range(B):
        g = got[bi].astype(np.float64)
        w = want[bi].astype(np.float64)
        axes = (0, 2) if per_token else tuple(range(1, g.ndim))
        num = np.sqrt(((g - w) ** 2).sum(axis=axes))
        den = np.sqrt((w ** 2).sum(axis=axes))
        out[bi] = num / np.where(den == 0.0, 1.0, den)
    return out


def test_full_size_config1_every_pair(wk, oracle):
    # the headline workload at full size (B=8, T=4096, H=32, bf16, s0 ~ N(0, 0.1)):
    # all 256 (b, h) pairs against the oracle over all 4096 steps, and the
    # checkpoint of the last chunk equals the transposed final state.
    announce("config[1] full size, every (b, h)")
    pkg = load_pkg()
    B, T, H = 8, 4096, 32
    t = pkg.synthetic.make_inputs_torch(B, T, H, seed=0x5EED0001, s0_std=0.1, dtype=torch.bfloat16)
    ins = [t[n] for n in NAMES]
    fwd = wk.wkv7_statepass_forward(*ins, t["s0"], 16)
    bwd = wk.wkv7_statepass_backward(*ins, fwd.state, fwd.removal_state, t["dy"],
                                     torch.zeros_like(t["s0"]), 16)
    torch.cuda.synchronize()
    assert torch.equal(fwd.state[:, :, -1], fwd.final_state.transpose(-1, -2))
    check_every_pair(pkg, fwd, bwd, ins, t["s0"], t["dy"], oracle, "config[1]")


def test_full_size_config2_every_pair(wk, oracle):
    # the 7B-class workload at full size (B=4, T=4096, H=64, bf16, zero initial
    # state) on the pretrain operator: all 256 (b, h) pairs against the oracle
    # over all 4096 steps; and the statepass operator from an all-zero state
    # gives the same outputs and gradients bit for bit.
    announce("config[2] full size, every (b, h)")
    pkg = load_pkg()
    B, T, H = 4, 4096, 64
    t = pkg.synthetic.make_inputs_torch(B, T, H, seed=0x5EED0002, s0_std=None, dtype=torch.bfloat16)
    ins = [t[n] for n in NAMES]
    fwd = wk.wkv7_pretrain_forward(wk.Wkv7ForwardInput(
        receptance=ins[1], weight_decay=ins[0], replacement_key=ins[2], value=ins[3],
        removal_key_normalized=ins[4], replacement=ins[5]), 16)
    bwd = wk.wkv7_pretrain_backward(*ins, fwd.state, fwd.removal_state, t["dy"], 16)
    zero = torch.zeros(B, H, 64, 64, device=ins[0].device)
    sp_f = wk.wkv7_statepass_forward(*ins, zero, 16)
    sp_b = wk.wkv7_statepass_backward(*ins, sp_f.state, sp_f.removal_state, t["dy"], zero, 16)
    torch.cuda.synchronize()
    assert torch.equal(sp_f.output, fwd.output)
    assert torch.equal(sp_f.state, fwd.state)
    for gn in GRAD_NAMES:
        assert torch.equal(getattr(sp_b, gn), getattr(bwd, gn)), gn
    del sp_f, sp_b
    check_every_pair(pkg, fwd, bwd, ins, None, t["dy"], oracle, "config[2]", state_family=False)


@pytest.mark.parametrize("case", [
    (1, 16, 1, None, 31),    # one chunk from a zero state
    (2, 64, 3, 0.1, 32),     # one full batch of four chunks
    (1, 80, 2, 0.1, 33),     # a partial last batch (one chunk)
    (3, 48, 2, None, 34),    # three chunks, no initial state
])
def test_bf16_chunked_forward_matches_step_forward(wk, case):
    # bf16, chunk_len 16 runs the chunked matrix-core forward; kernels="step"
    # (wkv7_forward_ex) runs the step-by-step fp32 kernel on the same call.
    # Outputs within bf16 rounding, fp32 state family within 1e-4.
    B, T, H, s0_std, seed = case
    announce("bf16 chunked vs step forward", case)
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std, bf16=True)
    ins = [to_dev(d[n], torch.bfloat16) for n in NAMES]
    s0 = to_dev(d["s0"]) if d["s0"] is not None else torch.zeros(B, H, 64, 64, device="cuda")
    ch = wk.wkv7_statepass_forward(*ins, s0, 16)
    st = wk.wkv7_forward_ex(*ins, s0, 16, kernels="step")
    torch.cuda.synchronize()
    assert rel_l2(to_np(ch.output), to_np(st.output)) < 1e-3
    for name in ("removal_state", "state", "final_state"):
        err = rel_l2(to_np(getattr(ch, name)), to_np(getattr(st, name)))
        assert err < BF16_STATE_TOL, (name, err)
    assert torch.equal(ch.state[:, :, -1], ch.final_state.transpose(-1, -2))


@pytest.mark.parametrize("case", [
    (1, 16, 1, None, 41),    # one chunk: the start state is rebuilt by reversal
    (1, 16, 2, 0.1, 42),
    (2, 64, 3, 0.1, 43),     # carried state gradient across chunks
    (1, 80, 2, None, 44),
])
def test_bf16_chunked_backward_matches_step_backward(wk, case):
    # bf16, chunk_len 16 runs the chunked matrix-core backward; kernels="step"
    # the step-by-step fp32 kernel. Both get the same forward outputs and a
    # nonzero final-state gradient; gradients agree within bf16 rounding, the
    # fp32 initial-state gradient within 1e-4.
    B, T, H, s0_std, seed = case
    announce("bf16 chunked vs step backward", case)
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(B, T, H, 64, seed=seed, s0_std=s0_std, bf16=True)
    ins = [to_dev(d[n], torch.bfloat16) for n in NAMES]
    s0 = to_dev(d["s0"]) if d["s0"] is not None else torch.zeros(B, H, 64, 64, device="cuda")
    dy = to_dev(d["dy"], torch.bfloat16)
    dsT = 0.1 * torch.randn(B, H, 64, 64, device="cuda", generator=torch.Generator("cuda").manual_seed(seed))
    f = wk.wkv7_forward_ex(*ins, s0, 16, kernels="step")
    st = wk.wkv7_backward_ex(*ins, f.state, f.removal_state, dy, dsT, 16, kernels="step")
    ch = wk.wkv7_statepass_backward(*ins, f.state, f.removal_state, dy, dsT, 16)
    torch.cuda.synchronize()
    for gn in GRAD_NAMES:
        err = rel_l2(to_np(getattr(ch, gn)), to_np(getattr(st, gn)))
        assert err < 2e-3, (gn, err)
    err = rel_l2(to_np(ch.initial_state_grad), to_np(st.initial_state_grad))
    assert err < BF16_STATE_TOL, err


@pytest.mark.parametrize("dtype,chunk_len", [("bf16", 16), ("f32", 16), ("bf16", 32)])
def test_handover_fault_poisons_outputs_and_is_reported(wk, dtype, chunk_len):
    """The chunked forwards' waves (bf16 operands at chunk_len 16, fp32
    operands, and bf16 operands past 16 on the fp32 kernel) hand chunks over
    through LDS flags with bounded waits. With the bound forced down to a
    single poll (the handover_spin_limit option) waves give up waits, which a
    correct run never does: every (batch, head) whose launch saw that must
    come back entirely NaN (output, removal_state, checkpoints, final state),
    the count of such launches must be reported by wkv7_take_faults as
    WKV7_ERR_HANDOVER, and every other (batch, head) must equal the normal run
    bit for bit. A normal run afterwards reports no fault."""
    announce("hand-over fault path (forced from the host)", dtype, chunk_len)
    pkg = load_pkg()
    B, T, H = 2, 256, 8
    bf16 = dtype == "bf16"
    d = pkg.synthetic.make_inputs(B, T, H, 64, seed=51, s0_std=0.1, bf16=bf16)
    ins = [to_dev(d[n], torch.bfloat16 if bf16 else torch.float32) for n in NAMES]
    s0 = to_dev(d["s0"])
    assert wk.take_faults() == 0
    good = wk.wkv7_statepass_forward(*ins, s0, chunk_len)
    assert wk.take_faults() == 0
    bad = wk.wkv7_forward_ex(*ins, s0, chunk_len, handover_spin_limit=1)
    faults = wk.take_faults()
    poisoned = 0
    for b in range(B):
        for h in range(H):
            parts = (bad.output[b, :, h], bad.removal_state[b, :, h], bad.state[b, h],
                     bad.final_state[b, h])
            if torch.isnan(bad.final_state[b, h]).any():
                assert all(torch.isnan(x.float()).all() for x in parts), (b, h)
                poisoned += 1
            else:
                assert torch.equal(bad.output[b, :, h], good.output[b, :, h]), (b, h)
                assert torch.equal(bad.state[b, h], good.state[b, h]), (b, h)
                assert torch.equal(bad.final_state[b, h], good.final_state[b, h]), (b, h)
    print("forced hand-over faults:", faults, "poisoned pairs:", poisoned, flush=True)
    assert faults == poisoned and faults > 0
    again = wk.wkv7_statepass_forward(*ins, s0, chunk_len)
    assert wk.take_faults() == 0
    assert torch.equal(again.output, good.output)
    # the C ABI's own status for the same event
    native = load_pkg()._native
    wk.wkv7_forward_ex(*ins, s0, chunk_len, handover_spin_limit=1)
    n = ctypes.c_uint32(0)
    rc = native.lib().wkv7_take_faults(torch.cuda.current_stream().cuda_stream, ctypes.byref(n))
    assert rc == native.WKV7_ERR_HANDOVER and n.value > 0, (rc, n.value)
    assert wk.take_faults() == 0
    # and the Python side raises it where the caller polls
    wk.wkv7_forward_ex(*ins, s0, chunk_len, handover_spin_limit=1)
    with pytest.raises(native.Wkv7Error, match="hand-over"):
        wk.check_faults()
    wk.check_faults()      # the counter was reset


@pytest.mark.parametrize("dtype", ["bf16", "f32"])
def test_tensors_past_2g_elements(wk, oracle, dtype):
    # Inputs past 2^31 elements each: bf16 [136, 4096, 64, 64] on the chunked
    # kernels (2.28e9 elements, 4.6 GB each; about 110 GB on the device with
    # the checkpoints and gradients), fp32 [129, 4096, 64, 64] on the fp32
    # chunked kernels (2.16e9 elements, 8.7 GB each; about 165 GB). The first and the
    # last (b, h) pairs -- the last one's elements lie past 2^31 elements and
    # 2^32 bytes from every tensor's start -- against the oracle run on that
    # pair alone, at the dtype's bars.
    announce("tensors past 2^31 elements", dtype)
    pkg = load_pkg()
    bf16 = dtype == "bf16"
    B, T, H = (136 if bf16 else 129), 4096, 64
    dt = torch.bfloat16 if bf16 else torch.float32
    tok_tol, st_tol = (BF16_TOL, BF16_STATE_TOL) if bf16 else (FP32_TOL, FP32_TOL)
    rnd_out = pkg.synthetic.bf16_round if bf16 else (lambda a: a)
    assert B * T * H * 64 > 2 ** 31
    gen = torch.Generator(device="cuda")
    gen.manual_seed(0x5EED00B1)

    def randn(*shape):
        return torch.randn(*shape, generator=gen, device="cuda")

    x = {n: randn(B, T, H, 64).to(dt) for n in ("w", "r", "k", "v")}
    kk = torch.nn.functional.normalize(randn(B, T, H, 64), dim=-1)
    x["a"] = (-kk).to(dt)
    x["b"] = (kk * torch.sigmoid(randn(B, T, H, 64))).to(dt)
    del kk
    dy = randn(B, T, H, 64).to(dt)
    s0 = randn(B, H, 64, 64) * 0.1
    ins = [x[n] for n in NAMES]
    fwd = wk.wkv7_statepass_forward(*ins, s0, 16)
    bwd = wk.wkv7_statepass_backward(*ins, fwd.state, fwd.removal_state, dy,
                                     torch.zeros_like(s0), 16)
    torch.cuda.synchronize()
    for bi, h in ((0, 0), (B - 1, H - 1)):
        tok = lambda t: to_np(t[bi:bi + 1, :, h:h + 1])      # [1, T, 1, 64]
        st = lambda t: to_np(t[bi:bi + 1, h:h + 1])          # [1, 1, ...]
        pin = [tok(t) for t in ins]
        of = oracle.forward_f32(*pin, s0=st(s0), chunk_len=16)
        ob = oracle.backward_f32(*pin, of["state"], of["removal_state"], tok(dy), chunk_len=16)
        errs = {"output": (rel_l2(tok(fwd.output), rnd_out(of["output"])), tok_tol),
                "removal_state": (rel_l2(tok(fwd.removal_state), of["removal_state"]), st_tol),
                "state": (rel_l2(st(fwd.state), of["state"]), st_tol),
                "final_state": (rel_l2(st(fwd.final_state), of["final_state"]), st_tol),
                "initial_state_grad": (rel_l2(st(bwd.initial_state_grad), ob["initial_state_grad"]),
                                       st_tol)}
        for gn in GRAD_NAMES:
            errs[gn] = (rel_l2(tok(getattr(bwd, gn)), rnd_out(ob[gn])), tok_tol)
        print(dtype, "pair", (bi, h), {k: f"{e:.2e}" for k, (e, _) in errs.items()}, flush=True)
        for k, (e, tol) in errs.items():
            assert e <= tol, ((bi, h), k, e)
    # give the device memory back to the tests that follow in this process
    del x, ins, dy, s0, fwd, bwd
    torch.cuda.empty_cache()
