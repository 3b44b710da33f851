"""The committed fixture tests/golden/wkv7_small.npz (exact fp64 results of
a seeded case, written by tests/golden/make_golden.py) against the oracle on
the CPU and against the gfx950 kernels (fp32 tolerance of the north star:
relative L2 <= 1e-5 per tensor, the reversal-based gradients included)."""

import os

import numpy as np
import pytest
import torch

from conftest import NAMES, announce, load_pkg, rel_l2, to_dev, to_np

HERE = os.path.dirname(os.path.abspath(__file__))
FIXTURE = os.path.join(HERE, "golden", "wkv7_small.npz")
GRADS = {"dw": "weight_decay_grad", "dr": "receptance_grad", "dk": "key_grad",
         "dv": "value_grad", "da": "removal_grad", "db": "replacement_grad",
         "ds0": "initial_state_grad"}


@pytest.fixture(scope="module")
def golden():
    with np.load(FIXTURE) as z:
        return {k: z[k] for k in z.files}


def test_oracle_reproduces_fixture(oracle, golden):
    g = golden
    ins = [g[n] for n in NAMES]
    f64 = oracle.forward_f64(*ins, s0=g["s0"])
    np.testing.assert_array_equal(f64["output"], g["y"])
    np.testing.assert_array_equal(f64["final_state"], g["s_T"])
    g64 = oracle.grad_f64(*ins, g["s0"], g["dy"], ds_T=g["ds_T"])
    for short, long in GRADS.items():
        np.testing.assert_array_equal(g64[long], g[short])
    # the reference-order fp32 oracle is within the fp32 tolerance of the fixture
    f32 = oracle.forward_f32(*ins, s0=g["s0"], chunk_len=16)
    assert rel_l2(f32["output"], g["y"]) < 1e-5
    b32 = oracle.backward_f32(*ins, f32["state"], f32["removal_state"], g["dy"],
                              ds_T=g["ds_T"], chunk_len=16)
    for short, long in GRADS.items():
        assert rel_l2(b32[long], g[short]) < 1e-5, short


@pytest.mark.gpu
def test_gpu_matches_fixture(golden):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    announce("golden fixture")
    wk = load_pkg().wkv7
    g = golden
    ins = [to_dev(g[n]) for n in NAMES]
    s0 = to_dev(g["s0"])
    fwd = wk.wkv7_statepass_forward(*ins, s0, 16)
    bwd = wk.wkv7_statepass_backward(*ins, fwd.state, fwd.removal_state, to_dev(g["dy"]),
                                     to_dev(g["ds_T"]), 16)
    torch.cuda.synchronize()
    assert rel_l2(to_np(fwd.output), g["y"]) < 1e-5
    assert rel_l2(to_np(fwd.final_state), g["s_T"]) < 1e-5
    for short, long in GRADS.items():
        err = rel_l2(to_np(getattr(bwd, long)), g[short])
        assert err < 1e-5, (short, err)
