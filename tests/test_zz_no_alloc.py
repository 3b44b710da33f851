"""rwkv_gated_readout_backward_noalloc (include/rwkv_neighbors.h): the gated
readout backward on the library's fixed per-GPU scratch array instead of a
caller workspace. It has no counterpart in the reference; its outputs must
equal rwkv_gated_readout_backward's bit for bit, on consecutive calls that
share the array (the second smaller than the first), with bf16 and fp32
operands, when captured in a HIP graph and replayed (other calls that
overwrite the array between the replays), including a capture that holds
the process's first call on the device (which looks up the array's
address); calls that would need more than the array must be refused before
any HIP call."""

import os
import subprocess
import sys

import pytest
import torch

from conftest import announce, load_pkg

F32, BF16 = 0, 1
SCRATCH_BYTES = 4 * 1024 * 1024
FAKE = 0x10000   # aligned addresses that are never dereferenced


@pytest.fixture(scope="module")
def lib():
    return load_pkg()._native.lib()


def _noalloc_fake(lib, rows, H):
    p = [FAKE * (i + 1) for i in range(8)]
    g = [FAKE * (i + 20) for i in range(9)]
    return lib.rwkv_gated_readout_backward_noalloc(*p, 64e-5, rows, H, 64, BF16, BF16, *g, None)


def test_noalloc_refuses_sizes_beyond_its_array(lib):
    # 64 rows per block and three column sums of H * 64 channels per block
    assert lib.rwkv_gated_readout_workspace_bytes(8192, 12, 64) <= SCRATCH_BYTES
    big_rows = 64 * (SCRATCH_BYTES // (3 * 12 * 64 * 4) + 1)
    assert lib.rwkv_gated_readout_workspace_bytes(big_rows, 12, 64) > SCRATCH_BYTES
    assert _noalloc_fake(lib, big_rows, 12) == 10          # WKV7_ERR_SCRATCH_LIMIT
    assert b"scratch" in lib.wkv7_strerror(10)
    # the usual checks come first
    assert _noalloc_fake(lib, 16, 0) == 2
    assert _noalloc_fake(lib, -1, 12) == 2


def _inputs(rows, H, seed, dtype=torch.bfloat16):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"

    def rn(*s, dtype=dtype, scale=1.0):
        return (torch.randn(*s, generator=gen, device=dev) * scale).to(dtype).contiguous()
    C = H * 64
    return dict(y=rn(rows, H, 64), r=rn(rows, H, 64), k=rn(rows, H, 64), v=rn(rows, H, 64),
                gate=rn(rows, C), bonus=rn(H, 64, dtype=torch.float32, scale=0.1),
                weight=1.0 + rn(C, dtype=torch.float32, scale=0.1),
                bias=rn(C, dtype=torch.float32, scale=0.1), dout=rn(rows, C))


def _outputs(d):
    return dict(dy=torch.empty_like(d["y"]), dr=torch.empty_like(d["r"]),
                dk=torch.empty_like(d["k"]), dv=torch.empty_like(d["v"]),
                dgate=torch.empty_like(d["gate"]), dbonus=torch.empty_like(d["bonus"]),
                dweight=torch.empty_like(d["weight"]), dbias=torch.empty_like(d["bias"]))


def _launch(lib, d, outs, rows, H, noalloc, ws=None):
    """Enqueues one readout backward on the current stream; no synchronisation."""
    code = BF16 if d["y"].dtype == torch.bfloat16 else F32
    ins = [d[n].data_ptr() for n in ("y", "r", "k", "v", "gate", "bonus", "weight", "bias")]
    grads = [outs[n].data_ptr() for n in ("dy", "dr", "dk", "dv", "dgate", "dbonus",
                                           "dweight", "dbias")]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.rwkv_gated_readout_backward_noalloc(*ins, 64e-5, rows, H, 64, code, code,
                                                     d["dout"].data_ptr(), *grads, stream)
    else:
        nbytes = lib.rwkv_gated_readout_workspace_bytes(rows, H, 64)
        rc = lib.rwkv_gated_readout_backward(*ins, 64e-5, rows, H, 64, code, code,
                                             d["dout"].data_ptr(), *grads, ws.data_ptr(),
                                             nbytes, stream)
    assert rc == 0, lib.wkv7_strerror(rc)


def _backward(lib, d, rows, H, noalloc):
    outs = _outputs(d)
    ws = None
    if not noalloc:
        nbytes = lib.rwkv_gated_readout_workspace_bytes(rows, H, 64)
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device="cuda")
    _launch(lib, d, outs, rows, H, noalloc, ws)
    torch.cuda.synchronize()
    return outs


def _replays_match(lib, d, rows, H, want, between):
    """Captures one noalloc call in a HIP graph, then replays it three times;
    ``between`` (eager noalloc calls on other inputs, which overwrite the
    shared array) runs before each replay. Every replay must give ``want``
    bit for bit."""
    outs = _outputs(d)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        _launch(lib, d, outs, rows, H, noalloc=True)
    for i in range(3):
        between()
        for t in outs.values():
            t.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        for name in want:
            assert torch.equal(outs[name], want[name]), (i, rows, name)


@pytest.mark.gpu
def test_noalloc_matches_workspace_entry_point(lib):
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    # config[4]'s readout (B=16, T=512, H=12), then a smaller ragged call that
    # reuses the array the first one filled
    for rows, H, seed in ((8192, 12, 1), (111, 12, 2)):
        announce("gated readout backward noalloc", rows, H)
        d = _inputs(rows, H, seed)
        want = _backward(lib, d, rows, H, noalloc=False)
        got = _backward(lib, d, rows, H, noalloc=True)
        for name in want:
            assert torch.equal(got[name], want[name]), (rows, name)
        assert torch.count_nonzero(got["dweight"]) > 0


@pytest.mark.gpu
def test_noalloc_fp32_matches_workspace_entry_point(lib):
    for rows, H, seed in ((4096, 4, 3), (77, 4, 4)):
        announce("gated readout backward noalloc fp32", rows, H)
        d = _inputs(rows, H, seed, torch.float32)
        want = _backward(lib, d, rows, H, noalloc=False)
        got = _backward(lib, d, rows, H, noalloc=True)
        for name in want:
            assert torch.equal(got[name], want[name]), (rows, name)


@pytest.mark.gpu
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "fp32"])
def test_noalloc_captured_in_a_graph(lib, dtype):
    announce("gated readout backward noalloc under graph capture", str(dtype))
    rows, H = 2048, 12
    d = _inputs(rows, H, 5, dtype)
    want = _backward(lib, d, rows, H, noalloc=False)
    other = _inputs(4096, H, 6, dtype)

    def between():
        _backward(lib, other, 4096, H, noalloc=True)
    _replays_match(lib, d, rows, H, want, between)


def first_call_captured():
    """In a fresh process: the first noalloc call on the device, the one that
    looks up the array's address, is made under graph capture."""
    lib = load_pkg()._native.lib()
    rows, H = 1024, 12
    d = _inputs(rows, H, 7)
    want = _backward(lib, d, rows, H, noalloc=False)
    _replays_match(lib, d, rows, H, want, lambda: None)
    print("first captured call: replays match", flush=True)


@pytest.mark.gpu
def test_noalloc_first_call_under_capture():
    announce("gated readout backward noalloc: first call under capture (subprocess)")
    here = os.path.dirname(os.path.abspath(__file__))
    env = dict(os.environ, PYTHONPATH=os.pathsep.join(
        [here, os.path.dirname(here), os.environ.get("PYTHONPATH", "")]))
    code = "import test_zz_no_alloc as t; t.first_call_captured()"
    res = subprocess.run([sys.executable, "-c", code], env=env, capture_output=True, text=True,
                         timeout=300)
    print(res.stdout[-2000:], res.stderr[-4000:], flush=True)
    assert res.returncode == 0 and "replays match" in res.stdout
