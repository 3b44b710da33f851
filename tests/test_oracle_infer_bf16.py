"""Pins the oracle's bf16 decode (wkv7o_infer_bf16): the reference's
inference kernel instantiated at element type bf16
(/root/reference/crates/rwkv-nn/src/kernels/wkv7_infer/kernel.rs:15-114, dither
on per wkv7_infer/host.rs:157), where the state, the staged operands and every
product and sum are bf16.

Checks, each chosen so that a plausible slip fails one of them:
* the reference's own scalar padding test (wkv7_infer/mod.rs:189-230) with
  every F operation rounded to bf16, against the scalar model of
  wkv7_infer/mod.rs:143-176 with the same roundings;
* known answers for where the rounding happens: the decay is rounded after
  the dither is added; the two sums over the key index run left to right;
  the update is (s w + sa b) + k v, left to right;
* small-integer inputs, for which bf16 arithmetic is exact: the oracle must
  then equal the recurrence evaluated in exact integer arithmetic, which pins
  the roles and indices (state rows are values, columns keys);
* agreement with the fp32 oracle to bf16 rounding on random inputs;
* a second evaluation of the same rounding points written over whole rows
  at once (numpy, vectorised over the value index), bit for bit.
"""

import numpy as np

from conftest import load_pkg

W_SCALE = np.float32(-0.6065306597)
# ScalarStep values of wkv7_infer/mod.rs:191-222 (weight_decay, receptance, key,
# value, removal, replacement)
PAD = (3.0, 2.0, 4.0, 5.0, 6.0, 7.0)
STEP0 = (-1.2, 0.7, 0.3, 1.1, 0.2, 0.9)
STEP1 = (0.4, 1.2, -0.5, 0.8, -0.3, 1.05)
NAMES = ("w", "r", "k", "v", "a", "b")


def bf(x):
    """Nearest bf16 (ties to even) of float32 values, as float32."""
    x = np.asarray(x, np.float32)
    return load_pkg().synthetic.bf16_round(x).reshape(x.shape)


def bf1(x):
    return np.float32(bf(np.float32(x)).reshape(-1)[0])


def scalar_steps(steps):
    cols = list(zip(*steps))
    return [bf(np.array(c, np.float32)).reshape(1, len(steps), 1, 1) for c in cols]


def dither(seed):
    mixed = (seed * 2654435769) & 0xFFFFFFFF
    if mixed >= 1 << 31:
        mixed -= 1 << 32
    return np.float32(np.float32(mixed) * np.float32(2.0 ** -41))


def scalar_model_bf16(steps, mask, elapsed_t):
    """wkv7_infer/mod.rs:143-176 (run_scalar_forward, seeds from valid steps)
    with every operation the kernel performs in F rounded to bf16."""
    f = np.float32
    state, valid_t, outs = f(0), 0, []
    for (w, r, k, v, a, b), live in zip(steps, mask):
        if not live:
            outs.append(f(0))
            continue
        sig = f(1) / (f(1) + np.exp(-f(w)))
        wd = bf1(f(np.exp(W_SCALE * sig)) + dither(elapsed_t + valid_t))
        sa = bf1(f(0) + bf1(f(a) * state))
        state = bf1(bf1(bf1(state * wd) + bf1(sa * f(b))) + bf1(f(k) * f(v)))
        outs.append(bf1(f(0) + bf1(state * f(r))))
        valid_t += 1
    return outs, state


def test_reference_padding_test_at_bf16(oracle):
    # wkv7_infer/mod.rs:189-230 with element type bf16: a masked left pad must
    # leave the outputs and the state of the unpadded run, bit for bit, and
    # both equal the reference's scalar model with bf16 roundings.
    unpadded = scalar_steps([STEP0, STEP1])
    padded = scalar_steps([PAD, STEP0, STEP1])
    s_u = np.zeros((1, 1, 1, 1), np.float32)
    s_p = np.zeros((1, 1, 1, 1), np.float32)
    et = np.array([17], np.uint32)
    y_u = oracle.infer_bf16(*unpadded, [0], s_u, np.ones((1, 2), np.float32), et)
    y_p = oracle.infer_bf16(*padded, [0], s_p, np.array([[0, 1, 1]], np.float32), et)
    assert y_p[0, 0, 0, 0] == 0.0
    np.testing.assert_array_equal(y_p[0, 1:, 0, 0], y_u[0, :, 0, 0])
    assert s_p.ravel()[0] == s_u.ravel()[0]
    steps = [tuple(float(x.ravel()[t]) for x in unpadded) for t in range(2)]
    outs, state = scalar_model_bf16(steps, [1, 1], 17)
    np.testing.assert_array_equal(y_u[0, :, 0, 0], np.array(outs, np.float32))
    assert s_u.ravel()[0] == state
    # every value stays a bf16
    assert bf(y_u).tobytes() == y_u.tobytes() and bf(s_u).tobytes() == s_u.tobytes()


def _decay_f32(w):
    sig = np.float32(1) / (np.float32(1) + np.exp(-np.float32(w)))
    return np.float32(np.exp(W_SCALE * sig))


def test_dither_is_added_before_the_bf16_rounding(oracle):
    # with state 1, a = b = k = 0 and r = 1 one step outputs the rounded decay
    # itself. For a decay whose fp32 value lies between 2^-12 and 2^-10 from a
    # bf16 rounding midpoint, a dither of the right sign moves it across the
    # midpoint: the output must be the nearest bf16 of (decay + dither), which
    # differs between a positive and a negative dither.
    found = 0
    for w in bf(np.linspace(-4, 4, 4001).astype(np.float32)):
        d = _decay_f32(w)
        lo = np.float32(np.floor(d * 256) / 256)           # bf16 grid of [0.5, 1)
        mid = lo + np.float32(1 / 512)
        gap = float(d - mid)
        if not (2.0 ** -12 < abs(gap) < 2.0 ** -10 * 0.9):
            continue
        # a seed whose dither pushes d across the midpoint, and one that does not
        for seed in range(1, 400):
            dv = float(dither(seed))
            if abs(dv) > abs(gap) and np.sign(dv) != np.sign(gap):
                break
        else:
            continue
        outs = []
        for s_ in (seed, 0):   # dither(0) = 0
            st = np.ones((1, 1, 1, 1), np.float32)
            ops = [np.full((1, 1, 1, 1), v, np.float32) for v in (w, 1.0, 0.0, 0.0, 0.0, 0.0)]
            y = oracle.infer_bf16(*ops, [0], st, None, np.array([s_], np.uint32))
            outs.append(float(y.ravel()[0]))
            assert outs[-1] == float(bf1(np.float32(d) + dither(s_))), (w, s_)
        assert outs[0] != outs[1], w          # the dither moved the rounding
        found += 1
        if found >= 4:
            break
    assert found >= 4


def _step(oracle, S, w, a, b, k, v, r):
    """One bf16 step at N = len(w) from state S (bf16 values); returns (y, S')."""
    N = len(w)
    st = np.ascontiguousarray(S, np.float32).reshape(1, 1, N, N).copy()
    ops = [np.asarray(x, np.float32).reshape(1, 1, 1, N) for x in (w, r, k, v, a, b)]
    y = oracle.infer_bf16(*ops, [0], st, None, np.array([0], np.uint32), use_dither=False)
    return y.reshape(N), st.reshape(N, N)


W_ONE = -30.0   # decay exp(-e^{-1/2} sigmoid(-30)) rounds to exactly 1.0 in fp32


def test_sums_over_the_key_index_run_left_to_right(oracle):
    N = 64
    ones = np.ones((N, N), np.float32)
    w = np.full(N, W_ONE, np.float32)
    tiny = np.float32(2.0 ** -9)             # a quarter ulp of 1 in bf16
    # removal-state sum: 1 + 63 * 2^-9 added left to right in bf16 stays 1
    # (a pairwise or fp32 sum would give 1.125); it reaches the state through
    # b = e_0 and the output through r = e_0: y_j = S'[j, 0] = 1 + sa_j = 2.
    a = np.full(N, tiny, np.float32)
    a[0] = 1.0
    e0 = np.zeros(N, np.float32)
    e0[0] = 1.0
    z = np.zeros(N, np.float32)
    y, S = _step(oracle, ones, w, a, e0, z, z, e0)
    np.testing.assert_array_equal(y, np.full(N, 2.0, np.float32))
    np.testing.assert_array_equal(S[:, 0], np.full(N, 2.0, np.float32))
    np.testing.assert_array_equal(S[:, 1:], ones[:, 1:])
    # output sum: r = (1, 2^-9, ...) over an all-ones state gives 1, not 1.123
    r = np.full(N, tiny, np.float32)
    r[0] = 1.0
    y, _ = _step(oracle, ones, w, z, z, z, z, r)
    np.testing.assert_array_equal(y, np.ones(N, np.float32))
    # the same inputs with the large term last: 63 * 2^-9 accumulates exactly
    # to 0.123046875, whose sum with 1 rounds to 1.125
    r = np.full(N, tiny, np.float32)
    r[-1] = 1.0
    y, _ = _step(oracle, ones, w, z, z, z, z, r)
    np.testing.assert_array_equal(y, np.full(N, 1.125, np.float32))


def test_update_adds_left_to_right(oracle):
    # s' = (s w + sa b) + k v: with s w = 1, sa b = 2^-8 and k v = 2^-8, the
    # first sum is a tie that rounds to even (1.0), and so is the second;
    # s w + (sa b + k v) would give 1 + 2^-7 exactly.
    N = 2
    h = np.float32(2.0 ** -8)
    S = np.array([[1.0, 0.0], [0.0, 0.0]], np.float32)   # row 0 = (1, 0)
    w = np.array([W_ONE, W_ONE], np.float32)
    a = np.array([1.0, 0.0], np.float32)       # sa_0 = S[0,0] = 1
    b = np.array([h, 0.0], np.float32)         # sa_0 b_0 = 2^-8
    k = np.array([h, 0.0], np.float32)
    v = np.array([1.0, 0.0], np.float32)       # k_0 v_0 = 2^-8 on row 0
    r = np.array([1.0, 0.0], np.float32)
    y, S1 = _step(oracle, S, w, a, b, k, v, r)
    assert S1[0, 0] == 1.0 and y[0] == 1.0
    # the value row the key product lands on is v's index: row 1 gets nothing
    assert S1[1, 0] == 0.0 and y[1] == 0.0


def test_small_integers_are_exact(oracle):
    # inputs and states that are small integers, decay 1 (w = -30): every bf16
    # product and partial sum is an integer of magnitude <= 256, so bf16
    # arithmetic is exact and the oracle must equal the recurrence of
    # wkv7_infer/kernel.rs:81-96 in exact integer arithmetic:
    #   sa_j = sum_i a_i S[j,i];  S[j,i] <- S[j,i] + sa_j b_i + k_i v_j;
    #   y_j = sum_i S[j,i] r_i
    rng = np.random.default_rng(5)
    N, T = 16, 3
    for trial in range(20):
        S0 = rng.integers(-2, 3, (N, N))
        a = np.zeros((T, N), np.int64)
        b = np.zeros((T, N), np.int64)
        for t in range(T):     # sparse a, b keep sa b small
            a[t, rng.integers(0, N, 2)] = rng.integers(-1, 2, 2)
            b[t, rng.integers(0, N, 1)] = rng.integers(-1, 2, 1)
        k = rng.integers(-1, 2, (T, N))
        v = rng.integers(-1, 2, (T, N))
        r = rng.integers(-1, 2, (T, N))
        S = S0.copy()
        ys, bound = [], 0
        for t in range(T):
            sa = S @ a[t]
            bound = max(bound, np.abs(S * a[t]).sum(axis=1).max())
            S = S + np.outer(sa, b[t]) + np.outer(v[t], k[t])
            ys.append(S @ r[t])
            bound = max(bound, np.abs(S * r[t]).sum(axis=1).max(), np.abs(S).max())
        assert bound <= 256, bound      # every intermediate fits bf16's 8 bits
        st = S0.astype(np.float32).reshape(1, 1, N, N).copy()
        ops = {"w": np.full((1, T, 1, N), W_ONE, np.float32)}
        for n, x in (("r", r), ("k", k), ("v", v), ("a", a), ("b", b)):
            ops[n] = x.astype(np.float32).reshape(1, T, 1, N)
        y = oracle.infer_bf16(*(ops[n] for n in NAMES), [0], st, None,
                              np.array([0], np.uint32), use_dither=False)
        np.testing.assert_array_equal(y.reshape(T, N), np.array(ys, np.float32))
        np.testing.assert_array_equal(st.reshape(N, N), S.astype(np.float32))


def test_close_to_fp32_to_bf16_rounding(oracle):
    d = load_pkg().synthetic.make_inputs(3, 6, 2, 64, seed=11, bf16=True)
    rng = np.random.default_rng(12)
    state = bf(rng.standard_normal((4, 2, 64, 64)).astype(np.float32) * np.float32(0.1))
    ids = np.array([3, 0, 2], np.int32)
    s16, s32 = state.copy(), state.copy()
    y16 = oracle.infer_bf16(*(d[n] for n in NAMES), ids, s16, None, np.zeros(4, np.uint32),
                            use_dither=False)
    y32 = oracle.infer_f32(*(d[n] for n in NAMES), ids, s32)
    rel = lambda x, y: float(np.linalg.norm(x - y) / np.linalg.norm(y))
    assert 1e-4 < rel(y16, y32) < 2e-2
    assert 1e-4 < rel(s16[ids], s32[ids]) < 2e-2
    np.testing.assert_array_equal(s16[1], state[1])


def _rowwise_bf16(w, r, k, v, a, b, ids, state, mask, elapsed, use_dither):
    """The same rounding points evaluated for all value rows at once."""
    f = np.float32
    Ba, T, H, N = w.shape
    y = np.zeros_like(w)
    for bi in range(Ba):
        slot = ids[bi]
        for h in range(H):
            S = state[slot, h]
            vt = 0
            for t in range(T):
                if mask is not None and mask[bi, t] == 0:
                    continue
                sig = f(1) / (f(1) + np.exp(-w[bi, t, h]))
                wd = np.exp(W_SCALE * sig).astype(f)
                if use_dither:
                    wd = (wd + dither(int(elapsed[slot]) + vt)).astype(f)
                wd = bf(wd)
                sa = np.zeros(N, f)
                for i in range(N):
                    sa = bf(sa + bf(a[bi, t, h, i] * S[:, i]))
                yy = np.zeros(N, f)
                for i in range(N):
                    p0 = bf(S[:, i] * wd[i])
                    p1 = bf(sa * b[bi, t, h, i])
                    p2 = bf(k[bi, t, h, i] * v[bi, t, h])
                    S[:, i] = bf(bf(p0 + p1) + p2)
                    yy = bf(yy + bf(S[:, i] * r[bi, t, h, i]))
                y[bi, t, h] = yy
                vt += 1
    return y


def test_rowwise_restatement_agrees_bitwise(oracle):
    d = load_pkg().synthetic.make_inputs(2, 5, 2, 64, seed=21, bf16=True)
    rng = np.random.default_rng(22)
    state = bf(rng.standard_normal((3, 2, 64, 64)).astype(np.float32) * np.float32(0.1))
    ids = np.array([2, 0], np.int32)
    mask = np.array([[1, 0, 1, 1, 1], [0, 0, 1, 1, 1]], np.float32)
    elapsed = np.array([5, 0, 91], np.uint32)
    s_o, s_r = state.copy(), state.copy()
    y_o = oracle.infer_bf16(*(d[n] for n in NAMES), ids, s_o, mask, elapsed, use_dither=True)
    y_r = _rowwise_bf16(*(d[n] for n in NAMES), ids, s_r, mask, elapsed, True)
    np.testing.assert_array_equal(y_o, y_r)
    np.testing.assert_array_equal(s_o, s_r)


def test_rounding_matches_an_independent_rne(oracle):
    """The oracle's bf16 rounding (wkv7o_round_bf16, used at every rounding
    point of the bf16 decode) against torch's float32 -> bfloat16 conversion,
    an independent round-to-nearest-even, on exact ties (both parities, both
    signs), values just either side of a tie, the bf16 range's ends and
    random values."""
    import torch
    ties = []
    for base in (1.0, 1.5, -3.25, 1e-3, 6.5e4):
        b = np.float32(base)
        ulp = np.float32(np.spacing(np.float32(bf(b)))) * np.float32(2.0 ** 16)   # one bf16 ulp
        half = np.float32(ulp / 2)
        ties += [b + half, b - half, b + 3 * half]
        ties += [np.nextafter(b + half, np.float32(np.inf)), np.nextafter(b + half, np.float32(-np.inf))]
    edge = [np.float32(3.3895314e38), np.float32(-3.3895314e38), np.float32(1.1754944e-38), np.float32(0.0),
            np.float32(-0.0)]
    rng = np.random.default_rng(5)
    rand = list(rng.standard_normal(2000).astype(np.float32) * np.float32(10.0) ** rng.integers(-20, 20, 2000))
    xs = np.array(ties + edge + rand, np.float32)
    got = np.array([oracle.round_bf16(float(x)) for x in xs], np.float32)
    want = torch.from_numpy(xs).to(torch.bfloat16).to(torch.float32).numpy()
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))
    np.testing.assert_array_equal(bf(xs).view(np.uint32), want.view(np.uint32))
