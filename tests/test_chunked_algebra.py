"""Pins, on the CPU, the chunked matrix form that the bf16 matrix-core kernels
(``wkv7_chunk_forward.hip``, ``wkv7_chunk_backward.hip``) compute.

The form regroups the reference's per-step recurrence
(/root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:31-112
forward, :116-308 backward) into 16-step chunks: with the log-decay prefix
g_t and gamma_t = exp(g_t), the steps of one chunk become products of decayed
rows, a unit lower-triangular solve P = (I - A_ab)^-1 and one state product
per chunk. Restated here in float64 numpy and checked against the oracle's
step-by-step ``forward_f64`` / ``grad_f64``:
- exactly (1e-9), which pins the identities themselves (a dropped term, a
  wrong mask diagonal or a missed decay factor shows at the 1e-2 level);
- with every product of two fp32 quantities rounded the way the kernels form
  it (hi/lo bf16 splits, hi*hi + hi*lo + lo*hi), which bounds the precision
  loss of that scheme alone well inside the bf16 parity tolerance.
"""

import numpy as np
import pytest

from conftest import load_pkg, rel_l2

L = 16
# log-decay = W_SCALE * sigmoid(w), W_SCALE = -exp(-0.5) to the reference's
# ten digits (/root/reference/crates/rwkv-nn/src/kernels/wkv7_common/kernel.rs:4,65)
W_SCALE = -0.6065306597
NAMES = ("w", "r", "k", "v", "a", "b")
GRADS = {"dw": "weight_decay_grad", "dr": "receptance_grad", "dk": "key_grad",
         "dv": "value_grad", "da": "removal_grad", "db": "replacement_grad"}


def _sigmoid(x):
    return 1.0 / (1.0 + np.exp(-x))


class Products:
    """Matrix product as the kernels form it: exact, or from bf16 hi/lo
    splits of both operands with the lo*lo term dropped."""

    def __init__(self, split, bf16_round):
        self.split = split
        self.round = bf16_round

    def _halves(self, x):
        x32 = np.asarray(x, np.float32)
        hi = self.round(x32)
        lo = self.round((x32 - hi).astype(np.float32))
        return hi.astype(np.float64), lo.astype(np.float64)

    def __call__(self, a, b):
        if not self.split:
            return a @ b
        ah, al = self._halves(a)
        bh, bl = self._halves(b)
        return ah @ bh + ah @ bl + al @ bh


def _decays(x, ws):
    lw = ws * _sigmoid(x)
    g = np.cumsum(lw, axis=0)
    g_prev = np.vstack([np.zeros((1, x.shape[1])), g[:-1]])
    return np.exp(g), np.exp(g_prev), np.exp(g[-1])


def chunked_forward(mm, ws, x, r, k, v, a, b, s0):
    """One head: inputs [T, N], s0 [N(value), N(key)]. Returns y, removal
    state, the state after each chunk and the final state."""
    T, N = r.shape
    s = s0.copy()
    y = np.zeros((T, N))
    sa = np.zeros((T, N))
    ends = []
    strict = np.tril(np.ones((L, L)), -1)
    incl = np.tril(np.ones((L, L)))
    for c in range(T // L):
        rows = slice(c * L, (c + 1) * L)
        gam, gam_prev, gam_end = _decays(x[rows], ws)
        a_hat, r_hat = a[rows] * gam_prev, r[rows] * gam
        k_til, b_til = k[rows] / gam, b[rows] / gam
        a_ab = mm(a_hat, b_til.T) * strict
        a_ak = mm(a_hat, k_til.T) * strict
        a_rb = mm(r_hat, b_til.T) * incl
        a_rk = mm(r_hat, k_til.T) * incl
        p = np.linalg.inv(np.eye(L) - a_ab)
        chunk_sa = mm(mm(p, a_hat), s.T) + mm(p, mm(a_ak, v[rows]))
        y[rows] = mm(r_hat, s.T) + mm(a_rk, v[rows]) + mm(a_rb, chunk_sa)
        sa[rows] = chunk_sa
        s = (s + mm(v[rows].T, k_til) + mm(chunk_sa.T, b_til)) * gam_end[None, :]
        ends.append(s.copy())
    return y, sa, ends, s


def chunked_backward(mm, ws, x, r, k, v, a, b, s0, ends, sa, dy, ds_end):
    """One head's gradients by the chunked adjoint, last chunk first."""
    T, N = r.shape
    ds = ds_end.copy()
    strict = np.tril(np.ones((L, L)), -1)
    incl = np.tril(np.ones((L, L)))
    out = {n: np.zeros((T, N)) for n in GRADS}
    for c in reversed(range(T // L)):
        rows = slice(c * L, (c + 1) * L)
        gam, gam_prev, gam_end = _decays(x[rows], ws)
        a_hat, r_hat = a[rows] * gam_prev, r[rows] * gam
        k_til, b_til = k[rows] / gam, b[rows] / gam
        k_end, b_end = k_til * gam_end, b_til * gam_end
        s_start = ends[c - 1] if c > 0 else s0
        vc, sac, dyc = v[rows], sa[rows], dy[rows]
        a_ab = mm(a_hat, b_til.T) * strict
        a_ak = mm(a_hat, k_til.T) * strict
        a_rb = mm(r_hat, b_til.T) * incl
        a_rk = mm(r_hat, k_til.T) * incl
        p = np.linalg.inv(np.eye(L) - a_ab)
        dsa = mm(p.T, mm(b_end, ds.T) + mm(a_rb.T, dyc))
        dv = mm(k_end, ds.T) + mm(a_rk.T, dyc) + mm(a_ak.T, dsa)
        dk_end, db_end = mm(vc, ds), mm(sac, ds)
        b_yv = mm(vc, dyc.T) * incl.T
        b_sav = mm(vc, dsa.T) * strict.T
        b_ysa = mm(sac, dyc.T) * incl.T
        b_sasa = mm(sac, dsa.T) * strict.T
        dk = (mm(b_yv, r_hat) + mm(b_sav, a_hat) + dk_end * gam_end[None, :]) / gam
        db = (mm(b_ysa, r_hat) + mm(b_sasa, a_hat) + db_end * gam_end[None, :]) / gam
        dr = gam * (mm(dyc, s_start) + mm(b_yv.T, k_til) + mm(b_ysa.T, b_til))
        da = gam_prev * (mm(dsa, s_start) + mm(b_sav.T, k_til) + mm(b_sasa.T, b_til))
        # dL/dg_t = r dr - k dk - b db + a_{t+1} da_{t+1}; the chunk end also
        # carries the decay applied to the whole state.
        dg = r[rows] * dr - k[rows] * dk - b[rows] * db
        dg[:-1] += a[rows][1:] * da[1:]
        dg[-1] += ((k_end * dk_end).sum(0) + (b_end * db_end).sum(0)
                   + gam_end * (s_start * ds).sum(0))
        dlw = np.cumsum(dg[::-1], axis=0)[::-1]
        sg = _sigmoid(x[rows])
        out["dw"][rows] = dlw * ws * sg * (1.0 - sg)
        out["dr"][rows], out["dk"][rows], out["dv"][rows] = dr, dk, dv
        out["da"][rows], out["db"][rows] = da, db
        ds = ds * gam_end[None, :] + mm(dyc.T, r_hat) + mm(dsa.T, a_hat)
    return out, ds


def _case(oracle, B, T, H, N, seed, s0_std):
    pkg = load_pkg()
    d = pkg.synthetic.make_inputs(B, T, H, N, seed=seed, s0_std=s0_std)
    s0 = d["s0"] if d["s0"] is not None else np.zeros((B, H, N, N), np.float32)
    ds_end = (np.random.default_rng(seed + 1).standard_normal((B, H, N, N))
              .astype(np.float32) * 0.1)
    ins = [d[n] for n in NAMES]
    fwd = oracle.forward_f64(*ins, s0=s0)
    grads = oracle.grad_f64(*ins, s0, d["dy"], ds_end)
    return pkg, d, s0, ds_end, fwd, grads


def _run(oracle, split, B, T, H, N, seed, s0_std):
    pkg, d, s0, ds_end, fwd, grads = _case(oracle, B, T, H, N, seed, s0_std)
    mm = Products(split, pkg.synthetic.bf16_round)
    ws = W_SCALE
    err = {}
    for bi in range(B):
        for h in range(H):
            head = {n: d[n][bi, :, h, :].astype(np.float64) for n in NAMES + ("dy",)}
            args = [head[n] for n in NAMES]
            y, sa, ends, s_fin = chunked_forward(mm, ws, *args, s0[bi, h].astype(np.float64))
            g, ds0 = chunked_backward(mm, ws, *args, s0[bi, h].astype(np.float64), ends, sa,
                                      head["dy"], ds_end[bi, h].astype(np.float64))
            pairs = [("y", y, fwd["output"][bi, :, h]),
                     ("final_state", s_fin, fwd["final_state"][bi, h]),
                     ("ds0", ds0, grads["initial_state_grad"][bi, h])]
            pairs += [(n, g[n], grads[rn][bi, :, h]) for n, rn in GRADS.items()]
            for name, got, want in pairs:
                err[name] = max(err.get(name, 0.0), rel_l2(got, want))
    return err


CASES = [(1, 64, 2, 64, 3, 0.1), (1, 48, 1, 64, 5, None), (2, 32, 1, 16, 7, 0.5)]


@pytest.mark.parametrize("B,T,H,N,seed,s0_std", CASES)
def test_chunked_form_equals_step_recurrence(oracle, B, T, H, N, seed, s0_std):
    err = _run(oracle, False, B, T, H, N, seed, s0_std)
    assert max(err.values()) < 1e-9, err


def test_split_bf16_products_stay_inside_bf16_tolerance(oracle):
    """The hi/lo scheme alone (no bf16 output rounding): state-side results
    near 1e-5, gradients within 5e-4, both far inside the 1e-2 bar."""
    err = _run(oracle, True, 1, 64, 2, 64, 3, 0.1)
    for name in ("y", "final_state", "ds0", "dk", "dv", "db"):
        assert err[name] < 3e-5, (name, err)
    for name in ("dw", "dr", "da"):
        assert err[name] < 1e-3, (name, err)


def test_dropped_term_is_caught(oracle):
    """Planted mistake on the CPU: omitting the chunk-end decay term of the
    decay gradient must fail the exact check."""
    pkg, d, s0, ds_end, fwd, grads = _case(oracle, 1, 32, 1, 16, 9, 0.5)
    mm = Products(False, pkg.synthetic.bf16_round)
    head = {n: d[n][0, :, 0, :].astype(np.float64) for n in NAMES + ("dy",)}
    args = [head[n] for n in NAMES]
    y, sa, ends, _ = chunked_forward(mm, W_SCALE, *args, s0[0, 0].astype(np.float64))
    g, _ = chunked_backward(mm, W_SCALE, *args, s0[0, 0].astype(np.float64), ends, sa,
                            head["dy"], ds_end[0, 0].astype(np.float64))
    want = grads["weight_decay_grad"][0, :, 0]
    assert rel_l2(g["dw"], want) < 1e-9
    # the same sum without the chunk-end term of the last chunk
    broken = g["dw"].copy()
    x_last = head["w"][-L:]
    sg = _sigmoid(x_last)
    gam, _, gam_end = _decays(x_last, W_SCALE)
    k_end = head["k"][-L:] / gam * gam_end
    b_end = head["b"][-L:] / gam * gam_end
    ds = ds_end[0, 0].astype(np.float64)
    term = ((k_end * mm(head["v"][-L:], ds)).sum(0) + (b_end * mm(sa[-L:], ds)).sum(0)
            + gam_end * (ends[-2] * ds).sum(0))
    broken[-L:] -= term[None, :] * W_SCALE * sg * (1.0 - sg)
    assert rel_l2(broken, want) > 1e-3
