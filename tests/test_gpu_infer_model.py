"""GPU tests of the model's serving path (``AutoRegressiveModel.infer``, the
mirror of examples/rwkv-lm/src/model.rs:184-300 with the buffers and
elapsed_t bookkeeping of inferring.rs:61-87, 100-180), on the decode kernel
and the fused neighbour ops, fp32 operands (and one bf16 case):

* a whole prompt through ``infer`` gives the training path's logits (the
  chunked pretrain kernel from a zero state), within 1e-5 relative L2;
* the prompt in one call, or split and then decoded token by token, leaves
  the same state and gives the same last logits (1e-5);
* slot mapping: two sequences in slots 3 and 1 of five, one left-padded,
  match each run alone; untouched slots keep their bytes; elapsed_t advances
  by the valid steps only (with the fused and with the torch neighbour ops).
"""

import pytest
import torch

from conftest import announce, rel_l2
from model_helpers import _wkv7_mod, tiny_model

pytestmark = pytest.mark.gpu
TOL = 1e-5
DEV = torch.device("cuda:0")


def _model(neighbor_ops="hip"):
    return tiny_model(seed=3, std=0.2, neighbor_ops=neighbor_ops).to(DEV)


def _err(a, b):
    return rel_l2(a.double().cpu().numpy(), b.double().cpu().numpy())


def _prompt(B, T, seed):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 97, (B, T), generator=g).to(DEV)


@torch.no_grad()
def test_infer_prompt_matches_training_logits():
    model = _model()
    toks = _prompt(2, 48, 5)
    ids = torch.arange(2, device=DEV)
    st = model.new_infer_state(2)
    announce("model infer", "full prompt vs training path")
    got = model.infer(toks, ids, st, unembed_mode="full")
    x = model.layer_norm_for_first_cell(model.embed(toks))
    x, _, _, _ = model.cells(x, ids, _wkv7_mod().KernelPretrain)
    want = model.unembed(model.layer_norm_for_unembed(x))
    torch.cuda.synchronize()
    assert got.shape == (2, 48, 97)
    assert _err(got, want) <= TOL


@torch.no_grad()
def test_prefill_then_decode_equals_one_call():
    model = _model()
    toks = _prompt(2, 20, 6)
    ids = torch.tensor([1, 0], device=DEV)
    one = model.new_infer_state(2)
    announce("model infer", "one call")
    want = model.infer(toks, ids, one)
    one.advance(ids, 20)
    step = model.new_infer_state(2)
    announce("model infer", "prefill 12 + 8 decode steps")
    model.infer(toks[:, :12], ids, step, unembed_mode="skip")
    step.advance(ids, 12)
    for t in range(12, 20):
        got = model.infer(toks[:, t:t + 1], ids, step)
        step.advance(ids, 1)
    torch.cuda.synchronize()
    assert _err(got, want) <= TOL
    for a, b in zip(step.state + step.shift_time + step.shift_channel,
                    one.state + one.shift_time + one.shift_channel):
        assert _err(a, b) <= TOL
    assert torch.equal(step.elapsed_t, one.elapsed_t)
    assert step.elapsed_t.tolist() == [20, 20]


@pytest.mark.parametrize("neighbor_ops", ["hip", "torch"])
@torch.no_grad()
def test_slot_mapped_batch_with_left_padding(neighbor_ops):
    model = _model(neighbor_ops)
    a, b = _prompt(1, 16, 7), _prompt(1, 11, 8)
    # b left-padded to 16 steps
    batch = torch.cat([a, torch.cat([torch.zeros(1, 5, dtype=a.dtype, device=DEV), b], 1)])
    mask = torch.ones(2, 16, device=DEV)
    mask[1, :5] = 0.0
    ids = torch.tensor([3, 1], device=DEV)
    st = model.new_infer_state(5)
    g = torch.Generator().manual_seed(9)
    for t in st.state + st.shift_time + st.shift_channel:   # other slots hold other sequences
        t.copy_(torch.randn(t.shape, generator=g))
    before = [t.clone() for t in st.state + st.shift_time + st.shift_channel]
    for slot in (3, 1):
        st.reset_slot(slot)
    announce("model infer", "slots 3 and 1 of 5, left padding", neighbor_ops)
    got = model.infer(batch, ids, st, context_mask=mask)
    st.advance(ids, 16, mask)
    torch.cuda.synchronize()
    for slot, toks in ((3, a), (1, b)):
        alone = model.new_infer_state(1)
        want = model.infer(toks, torch.zeros(1, dtype=torch.long, device=DEV), alone)
        row = 0 if slot == 3 else 1
        assert _err(got[row], want[0]) <= TOL, slot
        for x, y in zip(st.state + st.shift_time + st.shift_channel,
                        alone.state + alone.shift_time + alone.shift_channel):
            assert _err(x[slot], y[0]) <= TOL, slot
    for x, y in zip(st.state + st.shift_time + st.shift_channel, before):
        for slot in (0, 2, 4):
            assert torch.equal(x[slot], y[slot])
    assert st.elapsed_t.tolist() == [0, 11, 0, 16, 0]


@torch.no_grad()
def test_bf16_operator_serves_with_a_bf16_state_and_the_dither():
    """With bf16 operands the serving path runs the reference's decode at
    element type bf16 (wkv7_infer/kernel.rs at F = bf16, dither on per
    host.rs:157): the per-slot WKV7 state is bf16; prefill then token-by-token
    decode matches one call to bf16 rounding (the per-token operands are the
    same; only the row count of the matrix products differs); and the dither
    is live: the same prompt from a different elapsed_t leaves another state."""
    model = tiny_model(seed=3, std=0.2, neighbor_ops="hip", wkv7_dtype=torch.bfloat16).to(DEV)
    toks = _prompt(2, 20, 6)
    ids = torch.tensor([1, 0], device=DEV)
    one = model.new_infer_state(2)
    assert all(s.dtype == torch.bfloat16 for s in one.state)
    announce("model infer bf16", "one call")
    want = model.infer(toks, ids, one)
    one.advance(ids, 20)
    step = model.new_infer_state(2)
    announce("model infer bf16", "prefill 12 + 8 decode steps")
    model.infer(toks[:, :12], ids, step, unembed_mode="skip")
    step.advance(ids, 12)
    for t in range(12, 20):
        got = model.infer(toks[:, t:t + 1], ids, step)
        step.advance(ids, 1)
    torch.cuda.synchronize()
    assert _err(got, want) <= 2e-2
    for a, b in zip(step.state, one.state):
        assert _err(a, b) <= 2e-2
    assert step.elapsed_t.tolist() == [20, 20]
    shifted = model.new_infer_state(2)
    shifted.elapsed_t.fill_(1000)
    announce("model infer bf16", "other dither seeds")
    model.infer(toks, ids, shifted)
    torch.cuda.synchronize()
    assert any(not torch.equal(a, b) for a, b in zip(shifted.state, one.state))


@torch.no_grad()
def test_bf16_operator_serves_with_an_fp32_state_on_request():
    """new_infer_state(state_dtype=float32) keeps a bf16 model's WKV7 states in
    fp32: the decode runs the f32 kernel on the bf16 operands with no dither.
    A whole prompt through infer gives the training path's logits (the
    chunked kernels, fp32 state) to the bf16 bar; the same prompt from
    another elapsed_t leaves the same states bit for bit (no dither); prefill
    plus decode matches one call to bf16 rounding (the per-token operands
    are the same; only the row count of the matrix products differs)."""
    model = tiny_model(seed=3, std=0.2, neighbor_ops="hip", wkv7_dtype=torch.bfloat16).to(DEV)
    toks = _prompt(2, 32, 10)
    ids = torch.tensor([0, 1], device=DEV)
    one = model.new_infer_state(2, state_dtype=torch.float32)
    assert all(s.dtype == torch.float32 for s in one.state)
    announce("model infer bf16 operands, fp32 state", "one call")
    got = model.infer(toks, ids, one, unembed_mode="full")
    x = model.layer_norm_for_first_cell(model.embed(toks))
    x, _, _, _ = model.cells(x, ids, _wkv7_mod().KernelPretrain)
    want = model.unembed(model.layer_norm_for_unembed(x))
    torch.cuda.synchronize()
    assert _err(got, want) <= 1e-2
    shifted = model.new_infer_state(2, state_dtype=torch.float32)
    shifted.elapsed_t.fill_(1000)
    announce("model infer bf16 operands, fp32 state", "other elapsed_t")
    model.infer(toks, ids, shifted, unembed_mode="skip")
    torch.cuda.synchronize()
    assert all(torch.equal(a, b) for a, b in zip(shifted.state, one.state))
    step = model.new_infer_state(2, state_dtype=torch.float32)
    announce("model infer bf16 operands, fp32 state", "prefill 16 + 16 decode steps")
    model.infer(toks[:, :16], ids, step, unembed_mode="skip")
    for t in range(16, 32):
        last = model.infer(toks[:, t:t + 1], ids, step)
    torch.cuda.synchronize()
    assert _err(last[:, 0], got[:, -1]) <= 1e-2
    for a, b in zip(step.state, one.state):
        assert _err(a, b) <= 1e-2
    with pytest.raises(ValueError):
        tiny_model(seed=3).new_infer_state(1, state_dtype=torch.bfloat16)
