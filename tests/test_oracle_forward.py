"""Pins the oracle's forward (oracle/wkv7_oracle.c, wkv7o_forward_*), which
restates /root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:6-114,
against closed forms and invariants that a dropped term, a wrong sign, a
transposed index or an off-by-one in the decay would break."""

import numpy as np
import pytest

from conftest import load_pkg, rel_l2

W_SCALE = -0.6065306597


def decay(x):
    return np.exp(W_SCALE / (1.0 + np.exp(-np.asarray(x, np.float64))))


def scalar_inputs(T, x, r, k, v, a, b):
    shape = (1, T, 1, 1)
    return [np.full(shape, val, np.float64) for val in (x, r, k, v, a, b)]


@pytest.mark.parametrize("s0", [0.0, 0.7])
def test_n1_geometric_series(oracle, s0):
    # N=1: S_t = lam * S_{t-1} + k v with lam = w~ + a b, y_t = r S_t,
    # sa_t = a S_{t-1}. Closed form: S_t = lam^{t+1} s0 + kv (1-lam^{t+1})/(1-lam).
    T = 40
    x, r, k, v, a, b = -0.3, 1.3, 0.8, -1.1, -0.6, 0.45
    lam = decay(x) + a * b
    t = np.arange(T, dtype=np.float64)
    S = lam ** (t + 1) * s0 + k * v * (1 - lam ** (t + 1)) / (1 - lam)
    S_prev = np.concatenate([[s0], S[:-1]])
    ins = scalar_inputs(T, x, r, k, v, a, b)
    s0a = np.full((1, 1, 1, 1), s0)
    f64 = oracle.forward_f64(*ins, s0=s0a)
    np.testing.assert_allclose(f64["output"].ravel(), r * S, rtol=1e-12, atol=1e-14)
    np.testing.assert_allclose(f64["final_state"].ravel(), S[-1:], rtol=1e-12)
    f32 = oracle.forward_f32(*ins, s0=s0a.astype(np.float32), chunk_len=8)
    np.testing.assert_allclose(f32["output"].ravel(), r * S, rtol=2e-6, atol=1e-7)
    np.testing.assert_allclose(f32["removal_state"].ravel(), a * S_prev, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize("x_shift", [0.0, -40.0])
def test_decayed_linear_attention_closed_form(oracle, x_shift):
    # a = b = 0: y_t[j] = sum_{s<=t} v_s[j] sum_i k_s[i] r_t[i] prod_{u=s+1..t} w~_u[i].
    # x_shift=-40 drives w~ -> 1: plain causal linear attention (prefix sums).
    rng = np.random.default_rng(1)
    B, T, H, N = 1, 24, 2, 8
    x = rng.standard_normal((B, T, H, N)) + x_shift
    r, k, v = (rng.standard_normal((B, T, H, N)) for _ in range(3))
    z = np.zeros((B, T, H, N))
    logw = np.log(decay(x))
    D = np.cumsum(logw, axis=1)                     # D[t] = sum_{u<=t} log w~_u
    # weight[t, s, i] = exp(D[t,i] - D[s,i]) for s <= t
    diff = D[:, :, None] - D[:, None, :]            # [B, t, s, H, N]
    mask = np.tril(np.ones((T, T)))[None, :, :, None, None]
    A = np.einsum("btshi,bthi,bshi->btsh", np.exp(np.minimum(diff, 0.0)) * mask, r, k)
    y_ref = np.einsum("btsh,bshj->bthj", A, v)
    f64 = oracle.forward_f64(x, r, k, v, z, z)
    np.testing.assert_allclose(f64["output"], y_ref, rtol=1e-10, atol=1e-11)
    f32 = oracle.forward_f32(x, r, k, v, z, z, chunk_len=4)
    assert rel_l2(f32["output"], y_ref) < 1e-6


def test_dplr_matrix_form(oracle):
    # S_t = S_{t-1} (diag(w~_t) + a_t b_t^T) + v_t k_t^T, y_t = S_t r_t
    # (the diagonal-plus-low-rank transition written as matrix products).
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(2, 20, 3, 16, seed=3, s0_std=0.5)
    B, T, H, N = d["w"].shape
    S = d["s0"].astype(np.float64).copy()
    y = np.zeros((B, T, H, N))
    for t in range(T):
        for bi in range(B):
            for h in range(H):
                g = lambda key: d[key][bi, t, h].astype(np.float64)
                M = np.diag(decay(g("w"))) + np.outer(g("a"), g("b"))
                S[bi, h] = S[bi, h] @ M + np.outer(g("v"), g("k"))
                y[bi, t, h] = S[bi, h] @ g("r")
    f64 = oracle.forward_f64(d["w"], d["r"], d["k"], d["v"], d["a"], d["b"], s0=d["s0"])
    np.testing.assert_allclose(f64["output"], y, rtol=1e-10, atol=1e-11)
    np.testing.assert_allclose(f64["final_state"], S, rtol=1e-10, atol=1e-11)
    f32 = oracle.forward_f32(d["w"], d["r"], d["k"], d["v"], d["a"], d["b"], s0=d["s0"], chunk_len=5)
    assert rel_l2(f32["output"], y) < 2e-6
    assert rel_l2(f32["final_state"], S) < 2e-6


def test_chunk_len_invariance(oracle):
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(1, 32, 2, 16, seed=4, s0_std=0.1)
    ins = [d[k] for k in ("w", "r", "k", "v", "a", "b")]
    ref = oracle.forward_f32(*ins, s0=d["s0"], chunk_len=32)
    for C in (1, 2, 4, 8, 16):
        got = oracle.forward_f32(*ins, s0=d["s0"], chunk_len=C)
        for key in ("output", "removal_state", "final_state"):
            np.testing.assert_array_equal(got[key], ref[key])
        # the last checkpoint of every chunking is the final state, transposed
        np.testing.assert_array_equal(got["state"][:, :, -1], np.swapaxes(ref["final_state"], -1, -2))


def test_sequence_split_invariance(oracle):
    # statepass contract: running [0, T/2) then [T/2, T) with s_T -> s0 equals one run
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(2, 32, 2, 16, seed=5, s0_std=0.1)
    ins = [d[k] for k in ("w", "r", "k", "v", "a", "b")]
    full = oracle.forward_f32(*ins, s0=d["s0"], chunk_len=16)
    first = oracle.forward_f32(*(x[:, :16] for x in ins), s0=d["s0"], chunk_len=16)
    second = oracle.forward_f32(*(x[:, 16:] for x in ins), s0=first["final_state"], chunk_len=16)
    np.testing.assert_array_equal(np.concatenate([first["output"], second["output"]], 1), full["output"])
    np.testing.assert_array_equal(second["final_state"], full["final_state"])


def test_checkpoints_are_transposed_states(oracle):
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(1, 48, 2, 16, seed=6, s0_std=0.3)
    ins = [d[k] for k in ("w", "r", "k", "v", "a", "b")]
    C = 16
    f32 = oracle.forward_f32(*ins, s0=d["s0"], chunk_len=C)
    for c in range(48 // C):
        t_end = C * c + C
        pref = oracle.forward_f64(*(x[:, :t_end] for x in ins), s0=d["s0"])
        want = np.swapaxes(pref["final_state"], -1, -2)     # [K, V] layout
        got = f32["state"][:, :, c]
        assert rel_l2(got, want) < 2e-6
        # an untransposed checkpoint would fail: S is far from symmetric
        assert rel_l2(got, pref["final_state"]) > 1e-2


def test_f32_matches_f64_at_config0(oracle):
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(1, 64, 4, 64, seed=0)
    ins = [d[k] for k in ("w", "r", "k", "v", "a", "b")]
    f64 = oracle.forward_f64(*ins)
    f32 = oracle.forward_f32(*ins, chunk_len=16)
    assert rel_l2(f32["output"], f64["output"]) < 1e-6
    assert rel_l2(f32["final_state"], f64["final_state"]) < 1e-6


def test_bad_chunk_len_rejected(oracle):
    d = load_pkg().synthetic.make_inputs(1, 12, 1, 4, seed=0)
    ins = [d[k] for k in ("w", "r", "k", "v", "a", "b")]
    with pytest.raises(ValueError, match="chunk_len must divide"):
        oracle.forward_f32(*ins, chunk_len=5)
