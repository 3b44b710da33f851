"""CPU-only checks of the neighbour ops' C ABI (include/rwkv_neighbors.h):
workspace sizes, and host-side rejection of bad calls with the right status
before any HIP call (no kernel is launched: every call here fails
validation)."""

import ctypes

import pytest

from conftest import load_pkg

FAKE = 0x10000   # 64 KiB-aligned addresses that are never dereferenced
F32, BF16 = 0, 1


@pytest.fixture(scope="module")
def lib():
    n = load_pkg()._native
    return n.lib()


def ptrs(*addrs):
    arr = (ctypes.c_void_p * max(len(addrs), 1))()
    for i, a in enumerate(addrs):
        arr[i] = a
    return arr


def mix_fwd(lib, **over):
    a = dict(x=FAKE, shift=None, ids=None, mask=None, scales=FAKE * 2, K=2, B=2, T=8, C=64,
             full=2, dtype=F32, out=F32, mixes=ptrs(FAKE * 10, FAKE * 20), diff=None, nxt=None)
    a.update(over)
    return lib.rwkv_token_shift_mix_forward(a["x"], a["shift"], a["ids"], a["mask"], a["scales"],
                                            a["K"], a["B"], a["T"], a["C"], a["full"], a["dtype"],
                                            a["out"], a["mixes"], a["diff"], a["nxt"], None)


def test_token_shift_mix_workspace_bytes(lib):
    f = lib.rwkv_token_shift_mix_workspace_bytes
    # 32 rows per block: 8192 rows -> 256 blocks x 6 mixes x 768 channels x 4 B
    assert f(6, 16, 512, 768) == 256 * 6 * 768 * 4
    assert f(5, 1, 33, 64) == 2 * 5 * 64 * 4
    assert f(1, 0, 5, 64) == 0
    assert f(9, 1, 1, 64) == -1
    assert f(1, 1, 1, 6) == -1
    assert f(1, -1, 1, 64) == -1


def test_token_shift_mix_forward_validation(lib):
    assert mix_fwd(lib, dtype=2) == 5
    assert mix_fwd(lib, out=7) == 5
    assert mix_fwd(lib, K=9) == 2
    assert mix_fwd(lib, C=6) == 2
    assert mix_fwd(lib, B=-1) == 2
    assert mix_fwd(lib, B=70000, full=70000) == 2
    assert mix_fwd(lib, x=None) == 1
    assert mix_fwd(lib, scales=None) == 1
    assert mix_fwd(lib, mixes=ptrs(FAKE * 10, 0)) == 1
    assert mix_fwd(lib, x=FAKE + 4) == 6                     # fp32 needs 16 bytes
    assert mix_fwd(lib, mixes=ptrs(FAKE * 10, FAKE * 20 + 8)) == 6
    assert mix_fwd(lib, full=1) == 2                         # no batch ids: full batch >= batch
    assert mix_fwd(lib, mixes=ptrs(FAKE * 10, FAKE * 10)) == 7   # two outputs alias
    assert mix_fwd(lib, mixes=ptrs(FAKE, FAKE * 20)) == 7        # an output overlaps x


def test_token_shift_mix_backward_validation(lib):
    def bwd(**over):
        a = dict(x=FAKE, K=2, B=2, T=8, C=64, grads=ptrs(FAKE * 10, FAKE * 20), dx=FAKE * 30,
                 dsc=FAKE * 40, ws=FAKE * 50, wsb=1 << 20)
        a.update(over)
        return lib.rwkv_token_shift_mix_backward(a["x"], None, None, None, FAKE * 2, a["K"],
                                                 a["B"], a["T"], a["C"], 2, F32, F32, a["grads"],
                                                 None, a["dx"], None, a["dsc"], a["ws"], a["wsb"],
                                                 None)
    assert bwd(ws=None) == 2
    assert bwd(wsb=16) == 2
    assert bwd(dx=None) == 1
    assert bwd(dsc=None) == 1
    assert bwd(grads=ptrs(FAKE * 10, 0)) == 1
    assert bwd(dx=FAKE * 10) == 7                            # gradient output over a gradient input


def ro_fwd(lib, **over):
    a = dict(y=FAKE, r=FAKE * 2, k=FAKE * 3, v=FAKE * 4, g=FAKE * 5, bonus=FAKE * 6,
             w=FAKE * 7, b=FAKE * 8, eps=64e-5, rows=16, H=2, N=64, dtype=BF16, act=F32,
             out=FAKE * 20)
    a.update(over)
    return lib.rwkv_gated_readout_forward(a["y"], a["r"], a["k"], a["v"], a["g"], a["bonus"],
                                          a["w"], a["b"], a["eps"], a["rows"], a["H"], a["N"],
                                          a["dtype"], a["act"], a["out"], None)


def test_gated_readout_workspace_bytes(lib):
    f = lib.rwkv_gated_readout_workspace_bytes
    # 64 rows per block: 8192 rows -> 128 blocks x 3 sums x 768 channels x 4 B
    assert f(8192, 12, 64) == 128 * 3 * 768 * 4
    assert f(65, 1, 64) == 2 * 3 * 64 * 4
    assert f(0, 4, 64) == 0
    assert f(10, 4, 32) == -1
    assert f(10, 0, 64) == -1


def test_gated_readout_validation(lib):
    assert ro_fwd(lib, N=32) == 4
    assert ro_fwd(lib, dtype=3) == 5
    assert ro_fwd(lib, H=0) == 2
    assert ro_fwd(lib, rows=-1) == 2
    assert ro_fwd(lib, eps=-1.0) == 2
    assert ro_fwd(lib, eps=float("nan")) == 2
    assert ro_fwd(lib, y=None) == 1
    assert ro_fwd(lib, bonus=None) == 1
    assert ro_fwd(lib, out=None) == 1
    assert ro_fwd(lib, y=FAKE + 2) == 6                      # bf16 needs 8 bytes
    assert ro_fwd(lib, g=FAKE * 5 + 8) == 6                  # fp32 needs 16 bytes
    assert ro_fwd(lib, out=FAKE * 5) == 7                    # output over the gate
    # nothing to do, nothing required but the parameters
    assert ro_fwd(lib, rows=0, y=None, r=None, k=None, v=None, g=None, out=None) == 0


def prep_fwd(lib, **over):
    a = dict(k=FAKE, v=FAKE * 2, vf=FAKE * 3, lr=FAKE * 4, wd=FAKE * 5, vr=FAKE * 6,
             blr=FAKE * 7, bwd=FAKE * 8, bvr=FAKE * 9, ka=FAKE * 10, kk=FAKE * 11, rows=16, H=2,
             N=64, dtype=BF16, out=BF16, outs=(FAKE * 20, FAKE * 21, FAKE * 22, FAKE * 23,
                                             FAKE * 24))
    a.update(over)
    return lib.rwkv_weight_prepare_forward(a["k"], a["v"], a["vf"], a["lr"], a["wd"], a["vr"],
                                           a["blr"], a["bwd"], a["bvr"], a["ka"], a["kk"],
                                           a["rows"], a["H"], a["N"], a["dtype"], a["out"],
                                           *a["outs"], None)


def test_weight_prepare_workspace_bytes(lib):
    f = lib.rwkv_weight_prepare_workspace_bytes
    # 64 rows per block: 8192 rows -> 128 blocks x 5 sums x 768 channels x 4 B
    assert f(8192, 12, 64) == 128 * 5 * 768 * 4
    assert f(65, 1, 64) == 2 * 5 * 64 * 4
    assert f(0, 4, 64) == 0
    assert f(10, 4, 32) == -1
    assert f(-1, 4, 64) == -1
    assert f(10, 0, 64) == -1


def test_weight_prepare_forward_validation(lib):
    assert prep_fwd(lib, dtype=2) == 5
    assert prep_fwd(lib, out=9) == 5
    assert prep_fwd(lib, N=32) == 4
    assert prep_fwd(lib, H=0) == 2
    assert prep_fwd(lib, rows=-1) == 2
    assert prep_fwd(lib, k=None) == 1
    assert prep_fwd(lib, kk=None) == 1
    assert prep_fwd(lib, vf=None) == 1                      # residual on (its bias is given)
    assert prep_fwd(lib, vr=None) == 1
    assert prep_fwd(lib, bvr=None) == 2                     # residual inputs without their bias
    assert prep_fwd(lib, bvr=None, vf=None, vr=None, outs=(0, 0, 0, 0, 0)) == 1
    assert prep_fwd(lib, lr=FAKE * 4 + 2) == 6              # bf16 needs 8 bytes
    assert prep_fwd(lib, ka=FAKE * 10 + 8) == 6             # fp32 parameters need 16 bytes
    assert prep_fwd(lib, out=F32, outs=(FAKE * 20, FAKE * 21, FAKE * 22 + 8, FAKE * 23,
                                        FAKE * 24)) == 6
    assert prep_fwd(lib, outs=(FAKE * 20, FAKE * 20, FAKE * 22, FAKE * 23, FAKE * 24)) == 7
    assert prep_fwd(lib, outs=(FAKE * 20, FAKE * 21, FAKE * 22, FAKE * 23, FAKE * 5)) == 7
    # nothing to do: only the parameters are needed
    assert prep_fwd(lib, rows=0, k=None, v=None, vf=None, lr=None, wd=None, vr=None,
                    outs=(0, 0, 0, 0, 0)) == 0


def test_weight_prepare_backward_validation(lib):
    def bwd(**over):
        a = dict(bvr=FAKE * 9, gin=[FAKE * (30 + i) for i in range(5)],
                 gout=[FAKE * (40 + i) for i in range(6)], sums=[FAKE * (50 + i) for i in range(5)],
                 ws=FAKE * 60, wsb=1 << 20, vf=FAKE * 3, vr=FAKE * 6)
        a.update(over)
        g = a["gout"]
        return lib.rwkv_weight_prepare_backward(
            FAKE, FAKE * 2, a["vf"], FAKE * 4, FAKE * 5, a["vr"], FAKE * 7, FAKE * 8, a["bvr"],
            FAKE * 10, FAKE * 11, 16, 2, 64, BF16, BF16, *a["gin"], g[0], g[1], g[2], g[3], g[4],
            g[5], a["sums"][0], a["sums"][1], a["sums"][2], a["sums"][3], a["sums"][4], a["ws"],
            a["wsb"], None)
    assert bwd(ws=None) == 2
    assert bwd(wsb=64) == 2
    assert bwd(gin=[FAKE * 30, 0, FAKE * 32, FAKE * 33, FAKE * 34]) == 1
    assert bwd(gout=[FAKE * 40, FAKE * 41, FAKE * 42, FAKE * 43, 0, FAKE * 45]) == 1
    assert bwd(sums=[FAKE * 50, FAKE * 51, FAKE * 52, FAKE * 53, 0]) == 1   # residual bias grad
    assert bwd(sums=[FAKE * 50, 0, FAKE * 52, FAKE * 53, FAKE * 54]) == 1
    # no residual: its gradient outputs must be absent too
    assert bwd(bvr=None, vf=None, vr=None) == 2
    assert bwd(gout=[FAKE * 40, FAKE * 30, FAKE * 42, FAKE * 43, FAKE * 44, FAKE * 45]) == 7
    assert bwd(ws=FAKE * 50) == 7                           # workspace over a parameter gradient


def test_cross_entropy_l2wrap_validation(lib):
    def fwd(**over):
        a = dict(x=FAKE, t=FAKE * 2, rows=4, V=64, dt=BF16, outs=(FAKE * 3, FAKE * 4, FAKE * 5,
                                                                 FAKE * 6))
        a.update(over)
        return lib.rwkv_cross_entropy_l2wrap_forward(a["x"], a["t"], a["rows"], a["V"], a["dt"],
                                                     *a["outs"], None)

    def bwd(**over):
        a = dict(x=FAKE, t=FAKE * 2, scale=1e-4, rows=4, V=64, dt=BF16, dx=FAKE * 9)
        a.update(over)
        return lib.rwkv_cross_entropy_l2wrap_backward(a["x"], a["t"], FAKE * 3, FAKE * 4, FAKE * 5,
                                                      FAKE * 6, a["scale"], a["rows"], a["V"],
                                                      a["dt"], a["dx"], None)
    assert fwd(dt=4) == 5
    assert fwd(V=0) == 2
    assert fwd(rows=-1) == 2
    assert fwd(rows=1 << 31) == 2
    assert fwd(rows=(1 << 31) - 1, V=(1 << 31) - 1) == 2    # bytes beyond int64
    assert fwd(x=None) == 1
    assert fwd(outs=(FAKE * 3, 0, FAKE * 5, FAKE * 6)) == 1
    assert fwd(x=FAKE + 8) == 6                      # vector rows need 16 bytes
    assert fwd(t=FAKE * 2 + 4) == 6
    assert fwd(outs=(FAKE * 3, FAKE * 3, FAKE * 5, FAKE * 6)) == 7
    assert fwd(outs=(FAKE * 3, FAKE * 4, FAKE * 5, FAKE)) == 7    # an output over the logits
    assert fwd(rows=0, x=None, t=None, outs=(0, 0, 0, 0)) == 0
    assert bwd(scale=float("nan")) == 2
    assert bwd(dx=None) == 1
    assert bwd(dx=FAKE * 9 + 8) == 6
    assert bwd(V=63, dx=FAKE * 9 + 7) == 6           # element rows: bf16 needs 2 bytes
    assert bwd(dx=FAKE) == 7                         # gradient over the logits
    assert bwd(dx=FAKE * 5) == 7                     # gradient over a row array


def test_sizes_whose_byte_counts_overflow_are_refused(lib):
    # shapes valid per dimension whose byte counts (tensors or workspaces)
    # exceed int64: refused before any product wraps around
    assert lib.rwkv_token_shift_mix_workspace_bytes(6, 2 ** 20, 2 ** 20, 2 ** 24) == -1
    assert lib.rwkv_gated_readout_workspace_bytes(2 ** 62, 12, 64) == -1
    assert lib.rwkv_weight_prepare_workspace_bytes(2 ** 62, 12, 64) == -1
    # 2^40 slots x 2^23 channels x 4 bytes of token shift
    assert mix_fwd(lib, ids=FAKE * 3, shift=FAKE * 4, full=2 ** 40, C=2 ** 23) == 2
    assert ro_fwd(lib, rows=2 ** 37 - 64, H=65535) == 2
    assert prep_fwd(lib, rows=2 ** 37 - 64, H=65535) == 2


def test_hip_neighbour_ops_refuse_cpu_tensors():
    import torch
    nb = load_pkg().neighbors
    x = torch.zeros(1, 4, 8)
    with pytest.raises(ValueError):
        nb.token_shift_mix(x, [torch.zeros(8)])
    y = torch.zeros(1, 4, 1, 64)
    with pytest.raises(ValueError):
        nb.gated_readout(y, y, y, y, torch.zeros(1, 4, 64), torch.zeros(1, 64), torch.zeros(64),
                         torch.zeros(64))
