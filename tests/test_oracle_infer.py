"""Pins the oracle's decode path (wkv7o_infer_f32, restating
/root/reference/crates/rwkv-nn/src/kernels/wkv7_infer/kernel.rs:8-114) with the
reference's own two scalar tests (wkv7_infer/mod.rs:189-269), known answers of
the dither hash and agreement with the forward kernel."""

import numpy as np

from conftest import load_pkg

# ScalarStep values of wkv7_infer/mod.rs:191-222 (weight_decay, receptance, key,
# value, removal, replacement)
PAD = (3.0, 2.0, 4.0, 5.0, 6.0, 7.0)
STEP0 = (-1.2, 0.7, 0.3, 1.1, 0.2, 0.9)
STEP1 = (0.4, 1.2, -0.5, 0.8, -0.3, 1.05)


def scalar_steps(steps):
    cols = list(zip(*steps))
    return [np.array(c, np.float32).reshape(1, len(steps), 1, 1) for c in cols]


def test_dither_known_answers(oracle):
    # (i32)(seed * 2654435769 mod 2^32) * 2^-41
    assert oracle.dither(0) == 0.0
    assert oracle.dither(1) == float(np.float32(-1640531527) * np.float32(2.0 ** -41))
    assert oracle.dither(2) == float(np.float32(1013904242) * np.float32(2.0 ** -41))
    assert oracle.dither(17) == float(np.float32(-2119232183) * np.float32(2.0 ** -41))
    assert abs(oracle.dither(0xFFFFFFFF)) < 2.0 ** -10


def test_masked_dither_seed_matches_unpadded_execution(oracle):
    # wkv7_infer/mod.rs:189-230 at N=1: left padding with a masked step must
    # leave outputs and state equal to the unpadded run, dither on.
    unpadded = scalar_steps([STEP0, STEP1])
    padded = scalar_steps([PAD, STEP0, STEP1])
    s_u = np.zeros((1, 1, 1, 1), np.float32)
    s_p = np.zeros((1, 1, 1, 1), np.float32)
    et = np.array([17], np.uint32)
    y_u = oracle.infer_f32(*unpadded, [0], s_u, np.ones((1, 2), np.float32), et, use_dither=True)
    y_p = oracle.infer_f32(*padded, [0], s_p, np.array([[0, 1, 1]], np.float32), et, use_dither=True)
    assert y_p[0, 0, 0, 0] == 0.0
    np.testing.assert_allclose(y_p[0, 1:, 0, 0], y_u[0, :, 0, 0], atol=1e-7)
    assert abs(float(s_p.ravel()[0] - s_u.ravel()[0])) <= 1e-7


def test_counting_masked_steps_in_seed_shifts_state(oracle):
    # wkv7_infer/mod.rs:232-269: had the masked step consumed a dither position
    # (seed elapsed_t + t instead of elapsed_t + valid_t), the state would differ.
    steps = scalar_steps([STEP0, STEP1])
    s_ok = np.zeros((1, 1, 1, 1), np.float32)
    s_shift = np.zeros((1, 1, 1, 1), np.float32)
    oracle.infer_f32(*steps, [0], s_ok, None, np.array([17], np.uint32), use_dither=True)
    oracle.infer_f32(*steps, [0], s_shift, None, np.array([18], np.uint32), use_dither=True)
    assert abs(float(s_ok.ravel()[0] - s_shift.ravel()[0])) > 1e-9


def test_infer_single_step_equals_forward(oracle):
    d = load_pkg().synthetic.make_inputs(5, 1, 3, 64, seed=2, s0_std=0.1)
    ins = [d[n] for n in ("w", "r", "k", "v", "a", "b")]
    fwd = oracle.forward_f32(*ins, s0=d["s0"], chunk_len=1)
    state = d["s0"].copy()
    y = oracle.infer_f32(*ins, np.arange(5, dtype=np.int32), state)
    np.testing.assert_array_equal(y, fwd["output"])
    np.testing.assert_array_equal(state, fwd["final_state"])


def test_infer_slot_mapping(oracle):
    # active rows map to arbitrary slots; unmapped slots stay untouched.
    d = load_pkg().synthetic.make_inputs(3, 4, 2, 16, seed=8)
    ins = [d[n] for n in ("w", "r", "k", "v", "a", "b")]
    rng = np.random.default_rng(3)
    state = (rng.standard_normal((6, 2, 16, 16)) * 0.1).astype(np.float32)
    before = state.copy()
    ids = np.array([4, 0, 2], np.int32)
    y = oracle.infer_f32(*ins, ids, state)
    for row, slot in enumerate(ids):
        fwd = oracle.forward_f32(*(x[row:row + 1] for x in ins), s0=before[slot:slot + 1], chunk_len=4)
        np.testing.assert_array_equal(y[row:row + 1], fwd["output"])
        np.testing.assert_array_equal(state[slot:slot + 1], fwd["final_state"])
    for slot in (1, 3, 5):
        np.testing.assert_array_equal(state[slot], before[slot])
