"""The bf16 building blocks the kernels rest on, run on the device through
``wkv7_selftest_bf16_ops`` (include/wkv7.h) and held bit for bit to their CPU
expectation, so that a toolchain change in how they are lowered fails here:

* the hi/lo split of the chunked kernels (``chunk::split2``): hi = RNE(x),
  lo = RNE(x - hi), the residual formed by a bf16 dot product with the
  constant pair (-1, -0). Were that pair emitted as the inline constant -1.0
  (which the instruction reads as another 16-bit value), every lo part would
  be wrong;
* the rounded sum of the bf16-state decode (``add_rb``): RNE(x) + RNE(p) by a
  bf16 dot product with (1, 1), whose result the decode only ever uses
  rounded to bf16. The oracle's bf16 decode (oracle/wkv7_oracle.c,
  ``infer_bf16``) forms that sum as an fp32 addition of two bf16 values.

Edge values: ties of both parities, values on either side of 2^-126 (where
residuals and sums turn subnormal), bf16-subnormal inputs, large magnitudes up
to bf16's largest finite value, signed zeros, cancellations, and random
values over the whole exponent range the kernels see.

Expectations, over inputs that are zero or normal in bf16:
* hi and lo parts: IEEE fp32 arithmetic bit for bit, subnormal residuals
  included (the residual x - hi is exact in fp32, so any rounding gives it);
* sums: their bf16 rounding equals that of the IEEE fp32 addition bit for
  bit (a zero's sign aside: the dot product's +0 accumulator turns
  (-0) + (-0) into +0). The fp32 sum itself is not IEEE's when one addend is below 2^-16 of
  the other (measured: it is then one fp32 ulp off, e.g. a tie rounded
  away from even), which cannot move the bf16 rounding: with e the sum's
  exponent, a bf16 midpoint m (a multiple of 2^(e-8)) is either the exact
  sum s or at least 2^(e-8) - 2^(e-15) from it when an addend is that
  small (the other addend is a bf16 value, never a midpoint), and every
  other sum lies on the 2^(e-23) grid, where s - m is 0 or at least one
  fp32 ulp. The test counts the fp32 sums that differ from IEEE's.
What the device does with bf16-subnormal inputs is reported, not held: no
kernel operand is that small."""

import numpy as np
import pytest
import torch

from conftest import announce, load_pkg

pytestmark = pytest.mark.gpu

TINY = np.float32(2.0 ** -126)


def rne_bits(x):
    """float32 -> bf16 bits, round to nearest even (NaN to the quiet NaN)."""
    u = np.asarray(x, np.float32).view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) & 0xFFFF
    r[(u & 0x7FFFFFFF) > 0x7F800000] = 0x7FC0
    return r.astype(np.uint32)


def bf16_value(bits):
    return (np.asarray(bits, np.uint32) << 16).view(np.float32)


def edge_values():
    one = np.float32(1.0)
    ulp = np.float32(2.0 ** -7)            # bf16 spacing at 1
    vals = [
        0.0, -0.0, 1.0, -1.0,
        one + ulp / 2, one + 3 * ulp / 2,  # ties: to the even neighbour (down, up)
        -(one + ulp / 2), -(one + 3 * ulp / 2),
        one + ulp / 2 + 2.0 ** -20,        # just above a tie
        one + ulp / 2 - 2.0 ** -20,        # just below
        3.0e38, 1.0e38, -2.5e38,
        float(bf16_value(0x7F7F)),         # bf16's largest finite value
        -float(bf16_value(0x7F7F)),
        2.0 ** -126, -(2.0 ** -126), 1.5 * 2.0 ** -126,
        2.0 ** -120 * 1.2345, 2.0 ** -118 * 1.0001, 2.0 ** -110 * 1.7,
        1.0e-39, -3.0e-40,                 # fp32 subnormals (bf16 subnormal after rounding)
        1.0e-30, 12345.678, -0.3333333, 6.1e-5, 65504.0,
    ]
    return np.array(vals, np.float32)


def make_pairs():
    rng = np.random.default_rng(7)
    e = edge_values()
    a = np.repeat(e, len(e))
    b = np.tile(e, len(e))
    # random values over the kernels' range of exponents, both signs
    ra = (rng.standard_normal(200000) * np.exp2(rng.integers(-40, 40, 200000))).astype(np.float32)
    rb_ = (rng.standard_normal(200000) * np.exp2(rng.integers(-40, 40, 200000))).astype(np.float32)
    # cancellations: p close to -x
    c = rng.standard_normal(20000).astype(np.float32)
    ca, cb = c, (-c * (1 + rng.standard_normal(20000).astype(np.float32) * 1e-3)).astype(np.float32)
    return (np.concatenate([a, ra, ca]).astype(np.float32),
            np.concatenate([b, rb_, cb]).astype(np.float32))


def expected(a, b):
    """(hi bits, lo bits, sum) as IEEE fp32 arithmetic gives them, with
    subnormal results kept; and which lo parts / sums are below 2^-126."""
    ha, hb = rne_bits(a), rne_bits(b)
    with np.errstate(over="ignore", invalid="ignore"):
        ra = (a - bf16_value(ha)).astype(np.float32)     # exact in fp32 when finite
        rb_ = (b - bf16_value(hb)).astype(np.float32)
        s = (bf16_value(ha).astype(np.float64) + bf16_value(hb).astype(np.float64)).astype(np.float32)
    la, lb = rne_bits(ra), rne_bits(rb_)
    tiny_lo = ((np.abs(ra) < TINY) & (ra != 0)) | ((np.abs(rb_) < TINY) & (rb_ != 0))
    tiny_s = (np.abs(s) < TINY) & (s != 0)
    return ha | (hb << 16), la | (lb << 16), s, tiny_lo, tiny_s


def test_bf16_split_and_rounded_sum_on_edge_values():
    pkg = load_pkg()
    lib = pkg._native.lib()
    a, b = make_pairs()
    n = a.size
    ba, bb = bf16_value(rne_bits(a)), bf16_value(rne_bits(b))
    # inputs that are subnormal in bf16 after rounding (nonzero, below 2^-126)
    sub_in = ((np.abs(ba) < TINY) & (ba != 0)) | ((np.abs(bb) < TINY) & (bb != 0))
    inf_hi = (np.abs(ba) == np.inf) | (np.abs(bb) == np.inf)
    announce("bf16 self-test", n, "pairs")
    dev = torch.device("cuda:0")
    ta, tb = torch.from_numpy(a).to(dev), torch.from_numpy(b).to(dev)
    split = torch.empty(2 * n, dtype=torch.int32, device=dev)
    total = torch.empty(n, dtype=torch.float32, device=dev)
    rc = lib.wkv7_selftest_bf16_ops(ta.data_ptr(), tb.data_ptr(), n, split.data_ptr(),
                                    total.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.wkv7_strerror(rc)
    torch.cuda.synchronize()
    got = split.cpu().numpy().view(np.uint32).reshape(n, 2)
    got_sum = total.cpu().numpy()
    hi, lo, s, tiny_lo, tiny_s = expected(a, b)
    gs, es = got_sum.view(np.uint32), s.view(np.uint32)
    lo_ok = got[:, 1] == lo
    s_ok = gs == es
    zero_lo = (got[:, 1] & 0x7FFF7FFF) == (lo & np.where(tiny_lo, 0, 0x7FFF7FFF))
    zero_s = (gs & 0x7FFFFFFF) == 0

    def report(label, sel):
        idx = np.nonzero(sel)[0]
        print(f"{label}: {idx.size} pairs; lo parts as IEEE {int(lo_ok[idx].sum())}, "
              f"flushed {int((~lo_ok[idx] & zero_lo[idx]).sum())}; sums as IEEE "
              f"{int(s_ok[idx].sum())}, flushed {int((~s_ok[idx] & zero_s[idx]).sum())}",
              flush=True)
    ok = ~sub_in & ~inf_hi      # normal or zero inputs, finite hi parts
    report("residual below 2^-126", ok & tiny_lo)
    report("sum below 2^-126", ok & tiny_s)
    report("bf16-subnormal input", sub_in & ~inf_hi)
    # hi parts: plain RNE, everywhere
    bad = np.nonzero(got[:, 0] != hi)[0]
    assert bad.size == 0, [(a[i], b[i], hex(got[i, 0]), hex(hi[i])) for i in bad[:8]]
    # lo parts: IEEE fp32 bit for bit over normal or zero inputs, subnormal
    # residuals included
    bad = np.nonzero(~lo_ok & ok)[0]
    assert bad.size == 0, [(a[i], b[i], hex(got[i, 1]), hex(lo[i])) for i in bad[:8]]
    # sums: the bf16 rounding (all the decode uses) equals IEEE's bit for bit,
    # but for the sign of a zero: the dot product adds a +0 accumulator, so
    # (-0) + (-0) gives +0 (equal values; a zero's sign changes no later sum)
    gb, eb = rne_bits(got_sum), rne_bits(s)
    zeros = ((gb & 0x7FFF) == 0) & ((eb & 0x7FFF) == 0)
    bad = np.nonzero((gb != eb) & ~zeros & ok)[0]
    assert bad.size == 0, [(a[i], b[i], got_sum[i], s[i]) for i in bad[:8]]
    off = ~s_ok & ~zeros & ok
    if off.any():
        ratio = np.minimum(np.abs(ba), np.abs(bb))[off] / np.maximum(np.abs(ba), np.abs(bb))[off]
        print(f"fp32 sums that differ from IEEE: {int(off.sum())} of {int(ok.sum())}, all one "
              f"ulp: {bool((np.abs(gs[off].astype(np.int64) - es[off].astype(np.int64)) == 1).all())}"
              f", largest addend ratio {float(ratio.max()):.3g}", flush=True)
        assert ratio.max() < 2.0 ** -15
    # the random values (exponents -40 .. 40) lie in that range
    assert ok[-220000:].all()
