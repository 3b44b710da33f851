"""GPU parity of the slot-mapped decode kernel (wkv7_infer_forward in
include/wkv7.h) against the oracle restating
/root/reference/crates/rwkv-nn/src/kernels/wkv7_infer/kernel.rs:15-114."""

import numpy as np
import pytest
import torch

from conftest import NAMES, announce, load_pkg, rel_l2, to_dev, to_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def wk():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return load_pkg().wkv7


def bf16_state_close(got, want):
    """The bf16-state kernel against the bf16 oracle: the same bf16
    operations in the same order. Only the fp32 decay (exp, division) could
    differ, where the GPU's and the host's fp32 exp land on different sides of
    a bf16 rounding point; on these seeded inputs they do not, and the tests
    require bit-identical results. Returns the fraction of identical elements
    and the relative L2 error."""
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    same = float(np.mean(got.view(np.uint32) == want.view(np.uint32)))
    return same, rel_l2(got, want)


@pytest.mark.parametrize("dtype,state_dtype", [(torch.float32, torch.float32),
                                               (torch.bfloat16, torch.float32),
                                               (torch.bfloat16, torch.bfloat16)])
def test_decode_step_slot_mapped(wk, oracle, dtype, state_dtype):
    announce("infer T=1", dtype, state_dtype)
    pkg = load_pkg()
    Ba, H, full = 6, 5, 11
    bf16_state = state_dtype == torch.bfloat16
    d = pkg.synthetic.make_inputs(Ba, 1, H, 64, seed=31, bf16=(dtype == torch.bfloat16))
    rng = np.random.default_rng(32)
    state = (rng.standard_normal((full, H, 64, 64)) * 0.1).astype(np.float32)
    if bf16_state:
        state = pkg.synthetic.bf16_round(state).reshape(state.shape)
    ids = np.array([7, 0, 3, 10, 5, 1], np.int32)
    elapsed = rng.integers(0, 1000, full).astype(np.int32)
    st_gpu = to_dev(state, state_dtype)
    out = wk.wkv7_infer_forward(*(to_dev(d[n], dtype) for n in NAMES), torch.from_numpy(ids).cuda(),
                                st_gpu, None, torch.from_numpy(elapsed).cuda())
    st_ref = state.copy()
    assert out.final_state.data_ptr() == st_gpu.data_ptr()
    untouched = [s for s in range(full) if s not in ids]
    if bf16_state:
        # the reference at element type bf16, dither on (host.rs:157)
        y_ref = oracle.infer_bf16(*(d[n] for n in NAMES), ids, st_ref, None,
                                  elapsed.view(np.uint32))
        same_y, err_y = bf16_state_close(to_np(out.output), y_ref)
        same_s, err_s = bf16_state_close(to_np(st_gpu), st_ref)
        print("bf16 state", same_y, err_y, same_s, err_s, flush=True)
        assert same_y == 1.0 and same_s == 1.0, (err_y, err_s)
    else:
        y_ref = oracle.infer_f32(*(d[n] for n in NAMES), ids, st_ref, None)
        tol = 1e-5 if dtype == torch.float32 else 1e-2
        if dtype == torch.bfloat16:
            y_ref = pkg.synthetic.bf16_round(y_ref)
        assert rel_l2(to_np(out.output), y_ref) < tol
        assert rel_l2(to_np(st_gpu), st_ref) < 1e-5
    np.testing.assert_array_equal(to_np(st_gpu)[untouched], state[untouched])


def test_bf16_state_prefill_with_mask_and_dither(wk, oracle):
    """The reference at element type bf16 over a ragged, left-padded prefill
    (the per-step kernel path with T > 1): bf16 state, decay rounded after the
    dither, seeds elapsed_t + valid steps."""
    announce("infer bf16 state prefill")
    pkg = load_pkg()
    Ba, T, H, full = 3, 37, 2, 5
    d = pkg.synthetic.make_inputs(Ba, T, H, 64, seed=38, bf16=True)
    rng = np.random.default_rng(39)
    mask = (rng.random((Ba, T)) < 0.8).astype(np.float32)
    mask[0, :5] = 0.0
    state = pkg.synthetic.bf16_round(
        (rng.standard_normal((full, H, 64, 64)) * 0.1).astype(np.float32)).reshape(full, H, 64, 64)
    ids = np.array([4, 0, 2], np.int32)
    elapsed = np.array([5, 17, 0, 9, 1 << 30], np.int32)
    st_gpu = to_dev(state, torch.bfloat16)
    out = wk.wkv7_infer_forward(*(to_dev(d[n], torch.bfloat16) for n in NAMES),
                                torch.from_numpy(ids).cuda(), st_gpu, to_dev(mask, torch.bfloat16),
                                torch.from_numpy(elapsed).cuda())
    st_ref = state.copy()
    y_ref = oracle.infer_bf16(*(d[n] for n in NAMES), ids, st_ref, mask, elapsed.view(np.uint32))
    y = to_np(out.output)
    assert np.all(y[mask == 0] == 0.0)
    same_y, err_y = bf16_state_close(y, y_ref)
    same_s, err_s = bf16_state_close(to_np(st_gpu), st_ref)
    print("bf16 state prefill", same_y, err_y, same_s, err_s, flush=True)
    assert same_y == 1.0 and same_s == 1.0, (err_y, err_s)
    np.testing.assert_array_equal(to_np(st_gpu)[[1, 3]], state[[1, 3]])


def test_config3_decode_bf16_state(wk, oracle):
    """config[3]'s shape (256 sequences, one step, H = 40) on the reference's
    bf16 instantiation: bf16 state ~ N(0, 0.1) rounded to bf16, dither on,
    slots a permutation of a 320-slot buffer."""
    announce("config[3] decode, bf16 state")
    pkg = load_pkg()
    Ba, H, full = 256, 40, 320
    d = pkg.synthetic.make_inputs(Ba, 1, H, 64, seed=0x5EED0003, bf16=True, with_grad=False)
    rng = np.random.default_rng(0x5EED0013)
    state = pkg.synthetic.bf16_round(
        rng.standard_normal((full, H, 64, 64), dtype=np.float32) * np.float32(0.1)
    ).reshape(full, H, 64, 64)
    ids = rng.permutation(full)[:Ba].astype(np.int32)
    elapsed = rng.integers(0, 1 << 20, full).astype(np.int32)
    st_gpu = to_dev(state, torch.bfloat16)
    out = wk.wkv7_infer_forward(*(to_dev(d[n], torch.bfloat16) for n in NAMES),
                                torch.from_numpy(ids).cuda(), st_gpu, None,
                                torch.from_numpy(elapsed).cuda())
    torch.cuda.synchronize()
    st_ref = state.copy()
    y_ref = oracle.infer_bf16(*(d[n] for n in NAMES), ids, st_ref, None, elapsed.view(np.uint32))
    got = to_np(st_gpu)
    same_y, err_y = bf16_state_close(to_np(out.output), y_ref)
    same_s, err_s = bf16_state_close(got[ids], st_ref[ids])
    print("config[3] bf16 state", same_y, err_y, same_s, err_s, flush=True)
    assert same_y == 1.0 and same_s == 1.0, (err_y, err_s)
    untouched = np.setdiff1d(np.arange(full), ids)
    np.testing.assert_array_equal(got[untouched], state[untouched])


def test_dither_with_an_fp32_state_is_refused(wk):
    # the reference dithers only when its element type is not f32 (host.rs:157)
    ins = [torch.zeros(1, 1, 1, 64, device="cuda") for _ in NAMES]
    st = torch.zeros(1, 1, 64, 64, device="cuda")
    et = torch.zeros(1, dtype=torch.int32, device="cuda")
    ids = torch.zeros(1, dtype=torch.int32, device="cuda")
    with pytest.raises(ValueError, match="dither"):
        wk.wkv7_infer_forward(*ins, ids, st, None, et, use_dither=True)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_prefill_with_mask_matches_oracle(wk, oracle, dtype):
    # prefill (T > 1, the 16-step tile kernel) with a left-padded, ragged mask
    # in the operand dtype; fp32 state, no dither (the reference's F = f32
    # kernel, wkv7_infer/host.rs:157), bf16 operands carried as their exact
    # fp32 values by the oracle
    announce("infer prefill with mask", dtype)
    pkg = load_pkg()
    Ba, T, H, full = 3, 37, 2, 4
    bf16 = dtype == torch.bfloat16
    d = pkg.synthetic.make_inputs(Ba, T, H, 64, seed=33, bf16=bf16)
    rng = np.random.default_rng(34)
    mask = (rng.random((Ba, T)) < 0.8).astype(np.float32)
    mask[0, :5] = 0.0   # left padding
    state = (rng.standard_normal((full, H, 64, 64)) * 0.1).astype(np.float32)
    ids = np.array([2, 0, 3], np.int32)
    elapsed = np.array([5, 17, 0, 9], np.int32)
    st_gpu = to_dev(state)
    out = wk.wkv7_infer_forward(*(to_dev(d[n], dtype) for n in NAMES), torch.from_numpy(ids).cuda(),
                                st_gpu, to_dev(mask, dtype), torch.from_numpy(elapsed).cuda())
    st_ref = state.copy()
    y_ref = oracle.infer_f32(*(d[n] for n in NAMES), ids, st_ref, mask, elapsed.view(np.uint32))
    y = to_np(out.output)
    assert np.all(y[mask == 0] == 0.0)
    if bf16:
        y_ref = pkg.synthetic.bf16_round(y_ref)
    assert rel_l2(y, y_ref) < (1e-5 if not bf16 else 1e-2)
    assert rel_l2(to_np(st_gpu), st_ref) < 1e-5
    np.testing.assert_array_equal(to_np(st_gpu)[1], state[1])


def test_config3_decode_at_full_size(wk, oracle):
    """config[3] at its size: one decode step of 256 sequences, H = 40, bf16
    operands, fp32 state ~ N(0, 0.1), the reference's F = f32 kernel (no
    dither). The 256 active rows map onto a permutation of slots of a larger
    320-slot buffer; output and every slot are compared with the oracle, and
    the 64 untouched slots must be bit-identical."""
    announce("config[3] decode at full size")
    pkg = load_pkg()
    Ba, H, full = 256, 40, 320
    d = pkg.synthetic.make_inputs(Ba, 1, H, 64, seed=0x5EED0003, bf16=True, with_grad=False)
    rng = np.random.default_rng(0x5EED0003)
    state = (rng.standard_normal((full, H, 64, 64), dtype=np.float32) * np.float32(0.1))
    ids = rng.permutation(full)[:Ba].astype(np.int32)
    elapsed = rng.integers(0, 1 << 20, full).astype(np.int32)
    st_gpu = to_dev(state)
    out = wk.wkv7_infer_forward(*(to_dev(d[n], torch.bfloat16) for n in NAMES),
                                torch.from_numpy(ids).cuda(), st_gpu, None,
                                torch.from_numpy(elapsed).cuda())
    torch.cuda.synchronize()
    st_ref = state.copy()
    y_ref = oracle.infer_f32(*(d[n] for n in NAMES), ids, st_ref, None, elapsed.view(np.uint32))
    y = to_np(out.output)
    got = to_np(st_gpu)
    err_y = rel_l2(y, pkg.synthetic.bf16_round(y_ref))
    # per (row, head) state errors, the fp32 state family's 1e-5 bar
    num = np.sqrt(((got[ids].astype(np.float64) - st_ref[ids]) ** 2).sum(axis=(2, 3)))
    den = np.sqrt((st_ref[ids].astype(np.float64) ** 2).sum(axis=(2, 3)))
    print("config[3]", f"y {err_y:.2e} worst state pair {float((num / den).max()):.2e}", flush=True)
    assert err_y < 1e-2
    assert float((num / den).max()) < 1e-5
    untouched = np.setdiff1d(np.arange(full), ids)
    assert untouched.size == full - Ba
    np.testing.assert_array_equal(got[untouched], state[untouched])


def test_masked_padding_is_a_noop(wk):
    # wkv7_infer/mod.rs:189-230 at N=64 on the reference's bf16 instantiation
    # (dither on): left padding with masked steps gives the unpadded outputs
    # and state bit for bit.
    announce("infer padding no-op")
    pkg = load_pkg()
    H = 3
    d = pkg.synthetic.make_inputs(1, 6, H, 64, seed=35, bf16=True)
    pad = pkg.synthetic.make_inputs(1, 2, H, 64, seed=36, bf16=True)
    padded = {n: np.concatenate([pad[n], d[n]], 1) for n in NAMES}
    mask_p = np.array([[0, 0, 1, 1, 1, 1, 1, 1]], np.float32)
    et = torch.tensor([17], dtype=torch.int32, device="cuda")
    ids = torch.tensor([0], dtype=torch.int32, device="cuda")
    s_u = torch.zeros(1, H, 64, 64, device="cuda", dtype=torch.bfloat16)
    s_p = torch.zeros(1, H, 64, 64, device="cuda", dtype=torch.bfloat16)
    bf = torch.bfloat16
    y_u = wk.wkv7_infer_forward(*(to_dev(d[n], bf) for n in NAMES), ids, s_u, None, et).output
    y_p = wk.wkv7_infer_forward(*(to_dev(padded[n], bf) for n in NAMES), ids, s_p,
                                to_dev(mask_p, bf), et).output
    assert torch.all(y_p[:, :2] == 0)
    assert torch.equal(y_p[:, 2:], y_u)
    assert torch.equal(s_p, s_u)


def test_decode_matches_forward_step(wk):
    # T = 1 infer without dither equals one step of the training forward
    announce("infer == forward step")
    d = load_pkg().synthetic.make_inputs(4, 1, 3, 64, seed=37, s0_std=0.1)
    ins = [to_dev(d[n]) for n in NAMES]
    s0 = to_dev(d["s0"])
    fwd = wk.wkv7_statepass_forward(*ins, s0, 1)
    st = s0.clone()
    out = wk.wkv7_infer_forward(*ins, torch.arange(4, dtype=torch.int32, device="cuda"), st, None,
                                torch.zeros(4, dtype=torch.int32, device="cuda"))
    assert torch.equal(out.output, fwd.output)
    assert torch.equal(st, fwd.final_state)


def test_decode_step_replays_from_a_captured_graph(wk):
    """A serving loop captures its decode step once and replays it (here the
    reference's bf16 instantiation: bf16 state, dither seeded from elapsed_t): the
    entry point enqueues one kernel on the caller's stream and neither
    allocates nor clears memory, so it can sit in a HIP graph. Four replays,
    each after new tokens are copied into the captured inputs, against the
    same step run eagerly on copies of the state; the step also advances
    elapsed_t as a captured torch op (the host bookkeeping of
    inferring.rs:61-87). Results must be identical."""
    announce("infer graph capture")
    pkg = load_pkg()
    Ba, H, full = 4, 3, 6
    dev = torch.device("cuda:0")
    ids = torch.tensor([5, 0, 2, 3], dtype=torch.int32, device=dev)
    gen = torch.Generator().manual_seed(41)
    state = (torch.randn(full, H, 64, 64, generator=gen) * 0.1).to(dev, torch.bfloat16)
    elapsed = torch.randint(0, 100, (full,), generator=gen, dtype=torch.int32).to(dev)

    def fresh(seed):
        d = pkg.synthetic.make_inputs(Ba, 1, H, 64, seed=seed, bf16=True)
        return [to_dev(d[n], torch.bfloat16) for n in NAMES]

    static_in = fresh(50)

    def step(ins, st, el):
        out = wk.wkv7_infer_forward(*ins, ids, st, None, el)   # bf16 state: dither on
        el[ids.long()] += 1
        return out.output

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):             # warm-up off the capture, on copies
        step(static_in, state.clone(), elapsed.clone())
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    st_graph, el_graph = state.clone(), elapsed.clone()
    with torch.cuda.graph(g):
        y_graph = step(static_in, st_graph, el_graph)
    torch.cuda.synchronize()
    # capture records the work without running it: the eager copies start here
    st_eager, el_eager = state.clone(), elapsed.clone()
    for rep in range(4):
        new = fresh(60 + rep)
        for dst, src in zip(static_in, new):
            dst.copy_(src)
        g.replay()
        y_eager = step(new, st_eager, el_eager)
        torch.cuda.synchronize()
        assert torch.equal(y_graph, y_eager), rep
        assert torch.equal(st_graph, st_eager), rep
        assert torch.equal(el_graph, el_eager), rep


def test_decode_slots_past_2g_elements(wk, oracle):
    """A slot buffer past 2^31 elements ([8200, 64, 64, 64] fp32: 2.15e9
    elements, 8.6 GB): four rows mapped to the first and the last slots, one
    decode step, against the oracle on those slots; the slots between are
    untouched."""
    announce("decode slots past 2^31 elements")
    pkg = load_pkg()
    Ba, H, full = 4, 64, 8200
    assert full * H * 64 * 64 > 2 ** 31
    d = pkg.synthetic.make_inputs(Ba, 1, H, 64, seed=0x5EED00B2, bf16=True, with_grad=False)
    ids = np.array([full - 1, 0, full - 2, 1], np.int32)
    rng = np.random.default_rng(0x5EED00B2)
    picked = (rng.standard_normal((Ba, H, 64, 64), dtype=np.float32) * np.float32(0.1))
    st_gpu = torch.zeros(full, H, 64, 64, device="cuda")
    st_gpu[torch.from_numpy(ids.astype(np.int64)).cuda()] = to_dev(picked)
    probe = st_gpu[full // 2].clone()
    elapsed = np.zeros(full, np.int32)
    out = wk.wkv7_infer_forward(*(to_dev(d[n], torch.bfloat16) for n in NAMES),
                                torch.from_numpy(ids).cuda(), st_gpu, None,
                                torch.from_numpy(elapsed).cuda())
    torch.cuda.synchronize()
    # the oracle on a buffer of just the four slots, rows mapped in order
    st_ref = picked.copy()
    y_ref = oracle.infer_f32(*(d[n] for n in NAMES), np.arange(Ba, dtype=np.int32), st_ref, None,
                             np.zeros(Ba, np.uint32))
    err_y = rel_l2(to_np(out.output), pkg.synthetic.bf16_round(y_ref))
    got = to_np(st_gpu[torch.from_numpy(ids.astype(np.int64)).cuda()])
    err_s = rel_l2(got, st_ref)
    print("slots past 2^31", f"y {err_y:.2e} state {err_s:.2e}", flush=True)
    assert err_y < 1e-2 and err_s < 1e-5
    assert torch.equal(st_gpu[full // 2], probe)
    del st_gpu, out
    torch.cuda.empty_cache()
