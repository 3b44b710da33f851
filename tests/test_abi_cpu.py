"""CPU-only checks of the C ABI (include/wkv7.h, include/rwkv_neighbors.h,
include/rwkv_lm_loss.h):
the library loads, exports
every declared entry point, and rejects bad calls on the host with the right
status before any HIP call. No kernel is launched here: every call either
fails validation or has nothing to do."""

import ctypes
import os
import re

import pytest

from conftest import REPO, load_pkg

HEADER = os.path.join(REPO, "include", "wkv7.h")
NEIGHBORS_HEADER = os.path.join(REPO, "include", "rwkv_neighbors.h")
LOSS_HEADER = os.path.join(REPO, "include", "rwkv_lm_loss.h")


@pytest.fixture(scope="module")
def native():
    n = load_pkg()._native
    n.lib()
    return n


def declared_functions(header=HEADER, prefix="wkv7_"):
    text = open(header).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char \*)\s*(" + prefix + r"\w+)\s*\(",
                                 text, re.M)))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    assert len(names) == 17, names
    assert len(declared_functions(NEIGHBORS_HEADER, "rwkv_")) == 10
    assert len(declared_functions(LOSS_HEADER, "rwkv_")) == 2


def test_library_exports_every_declared_symbol(native):
    lib = native.lib()
    declared = (declared_functions() + declared_functions(NEIGHBORS_HEADER, "rwkv_")
                + declared_functions(LOSS_HEADER, "rwkv_"))
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(native.EXPORTS)


def test_version_and_strings(native):
    lib = native.lib()
    assert lib.wkv7_abi_version() == 2
    assert lib.wkv7_strerror(3).decode() == "chunk_len must divide sequence length"
    assert lib.wkv7_strerror(4).decode() == "head_size must be 64"
    assert lib.wkv7_strerror(123).decode() == "unknown wkv7 status"


def test_options_and_fault_query_validation(native):
    lib = native.lib()
    assert lib.wkv7_take_faults(None, None) == 1          # count pointer required
    msg = lib.wkv7_strerror(11).decode()
    assert "hand-over" in msg and "NaN" in msg
    bad = native.Wkv7Options(7, 0)                        # unknown kernel family
    assert lib.wkv7_forward_ex(*([FAKE] * 7), 1, 64, 4, 64, 16, 0, 1, 1, FAKE * 10,
                               FAKE * 20, FAKE * 30, FAKE * 40, native.options_ref(bad),
                               None) == 8
    assert lib.wkv7_backward_ex(*([FAKE] * 10), 1, 64, 4, 64, 16, 0, 1, 1,
                                *([FAKE * 10] * 7), native.options_ref(bad), None) == 8
    # the options are checked before anything else; valid options leave the
    # usual checks in place
    ok = native.Wkv7Options(native.KERNELS_STEP, 0)
    assert lib.wkv7_forward_ex(*([FAKE] * 7), 1, 60, 4, 64, 16, 0, 1, 1, FAKE * 10,
                               FAKE * 20, FAKE * 30, FAKE * 40, native.options_ref(ok),
                               None) == 3


def test_checkpoint_numel(native):
    f = native.lib().wkv7_checkpoint_numel
    assert f(8, 4096, 32, 64, 16) == 8 * 32 * 256 * 64 * 64
    assert f(1, 64, 4, 64, 16) == 4 * 4 * 64 * 64
    assert f(1, 0, 4, 64, 16) == 0
    assert f(1, 60, 4, 64, 16) == -1    # chunk_len does not divide context_len
    assert f(1, 64, 4, 32, 16) == -1    # head size
    assert f(-1, 64, 4, 64, 16) == -1


FAKE = 0x10000   # a 64 KiB-aligned address that is never dereferenced


def fwd(native, **over):
    a = dict(w=FAKE, r=FAKE * 2, k=FAKE * 3, v=FAKE * 4, a=FAKE * 5, b=FAKE * 6, s0=None,
             B=1, T=64, H=4, N=64, C=16, dtype=0, use_s0=0, ret_sT=0,
             state=FAKE * 100, sa=FAKE * 200, y=FAKE * 300, sT=None, stream=None)
    a.update(over)
    return native.lib().wkv7_forward(a["w"], a["r"], a["k"], a["v"], a["a"], a["b"], a["s0"],
                                     a["B"], a["T"], a["H"], a["N"], a["C"], a["dtype"],
                                     a["use_s0"], a["ret_sT"], a["state"], a["sa"], a["y"],
                                     a["sT"], a["stream"])


def test_forward_validation(native):
    assert fwd(native, N=32) == 4
    assert fwd(native, C=5) == 3
    assert fwd(native, C=0) == 3
    assert fwd(native, dtype=2) == 5
    assert fwd(native, B=-1) == 2
    assert fwd(native, B=70000) == 2
    assert fwd(native, w=None) == 1
    assert fwd(native, y=None) == 1
    assert fwd(native, use_s0=1) == 1          # initial_state required
    assert fwd(native, ret_sT=1) == 1          # final_state required
    assert fwd(native, use_s0=2) == 8
    assert fwd(native, k=FAKE + 4) == 6        # fp32 needs 16-byte alignment
    assert fwd(native, dtype=1, k=FAKE + 4) == 6
    assert fwd(native, y=FAKE * 2) == 7        # output aliases receptance
    assert fwd(native, sa=FAKE * 100 + 64) == 7  # removal_state overlaps state
    # nothing to do: no kernel launch, success
    assert fwd(native, B=0) == 0
    assert fwd(native, H=0) == 0


def test_backward_validation(native):
    lib = native.lib()

    def bwd(**over):
        a = dict(C=16, N=64, dtype=0, dsT_flag=0, ds0_flag=0, dw=FAKE * 400, ds0=None, dsT=None)
        a.update(over)
        return lib.wkv7_backward(FAKE, FAKE * 2, FAKE * 3, FAKE * 4, FAKE * 5, FAKE * 6,
                                 FAKE * 100, FAKE * 200, FAKE * 7, a["dsT"], 1, 64, 4, a["N"],
                                 a["C"], a["dtype"], a["dsT_flag"], a["ds0_flag"], a["dw"],
                                 FAKE * 500, FAKE * 600, FAKE * 700, FAKE * 800, FAKE * 900,
                                 a["ds0"], None)
    assert bwd(C=7) == 3
    assert bwd(N=128) == 4
    assert bwd(dsT_flag=1) == 1
    assert bwd(ds0_flag=1) == 1
    assert bwd(dw=None) == 1
    assert bwd(dw=FAKE * 7) == 7     # a gradient aliases output_grad


def test_infer_validation(native):
    lib = native.lib()

    def inf(**over):
        a = dict(ids=FAKE * 10, state=FAKE * 20, mask=None, et=None, Ba=2, T=1, H=4, N=64,
                 full=4, dtype=1, sdtype=0, dither=0, y=FAKE * 30)
        a.update(over)
        return lib.wkv7_infer_forward(FAKE, FAKE * 2, FAKE * 3, FAKE * 4, FAKE * 5, FAKE * 6,
                                      a["ids"], a["state"], a["mask"], a["et"], a["Ba"], a["T"],
                                      a["H"], a["N"], a["full"], a["dtype"], a["sdtype"],
                                      a["dither"], a["y"], None)
    assert inf(N=16) == 4
    assert inf(Ba=5) == 2             # more active rows than slots
    assert inf(ids=None) == 1
    assert inf(sdtype=1, dither=1) == 1   # elapsed_t required for the dither
    assert inf(dither=3) == 8
    # the reference dithers only a reduced-precision element type (host.rs:157)
    assert inf(dither=1, et=FAKE * 40) == 8
    assert inf(sdtype=1, dtype=0) == 5    # a bf16 state needs bf16 operands
    assert inf(sdtype=2) == 5
    assert inf(y=FAKE * 3) == 7       # output aliases key
    assert inf(state=FAKE) == 7       # state aliases weight_decay
    assert inf(state=FAKE * 20 + 8) == 6   # the state needs 16-byte alignment
    assert inf(Ba=0) == 0
    assert inf(Ba=0, sdtype=1) == 0


def test_python_mirror_checks_chunk_len_before_the_gpu():
    pytest.importorskip("torch")
    wk = load_pkg().wkv7
    with pytest.raises(ValueError, match="chunk_len must divide sequence length"):
        wk._check_chunk(60, 16)


def test_sizes_whose_byte_counts_overflow_are_refused(native):
    # batch 65535 x heads 65535 x 2^31 - 1 steps x 64 channels exceeds int64;
    # the checks must refuse it (not wrap around) before touching any pointer
    lib = native.lib()
    big_t = 2 ** 31 - 1
    fwd = lib.wkv7_forward(*([FAKE] * 6), None, 65535, big_t, 65535, 64, 1, 1, 0, 0,
                           FAKE * 10, FAKE * 20, FAKE * 30, None, None)
    assert fwd == 2
    bwd = lib.wkv7_backward(*([FAKE] * 9), None, 65535, big_t, 65535, 64, 1, 1, 0, 0,
                            *([FAKE * 10] * 6), None, None)
    assert bwd == 2
    assert lib.wkv7_checkpoint_numel(65535, big_t, 65535, 64, 1) == -1
    inf = lib.wkv7_infer_forward(*([FAKE] * 6), FAKE * 10, FAKE * 20, None, None, 65535, big_t,
                                 65535, 64, 65535, 1, 0, 0, FAKE * 30, None)
    assert inf == 2


def test_selftest_argument_checks(native):
    # refused on the host before any HIP call
    lib = native.lib()
    F = 0x10000
    assert lib.wkv7_selftest_bf16_ops(F, F, -1, F, F, None) == 2          # shape
    assert lib.wkv7_selftest_bf16_ops(F, F, 0, None, None, None) == 0      # nothing to do
    assert lib.wkv7_selftest_bf16_ops(None, F, 4, 2 * F, 3 * F, None) == 1
    assert lib.wkv7_selftest_bf16_ops(F + 2, 4 * F, 4, 2 * F, 3 * F, None) == 6
    assert lib.wkv7_selftest_bf16_ops(F, 4 * F, 4, F + 8, 3 * F, None) == 7   # split over a
