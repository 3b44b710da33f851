"""rwkv_gated_readout_backward_noalloc (include/rwkv_neighbors.h): the gated
readout backward on the library's fixed per-GPU scratch array instead of a
caller workspace. It has no counterpart in the reference; its outputs must
equal rwkv_gated_readout_backward's bit for bit, on consecutive calls that
share the array (the second smaller than the first), and calls that would
need more than the array must be refused before any HIP call."""

import ctypes

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


def _inputs(rows, H, seed):
    gen = torch.Generator(device="cuda").manual_seed(seed)
    dev = "cuda"

    def rn(*s, dtype=torch.bfloat16, scale=1.0):
        return (torch.randn(*s, generator=gen, device=dev) * scale).to(dtype).contiguous()
    C = H * 64
    return dict(y=rn(rows, H, 64), r=rn(rows, H, 64), k=rn(rows, H, 64), v=rn(rows, H, 64),
                gate=rn(rows, C), bonus=rn(H, 64, dtype=torch.float32, scale=0.1),
                weight=1.0 + rn(C, dtype=torch.float32, scale=0.1),
                bias=rn(C, dtype=torch.float32, scale=0.1), dout=rn(rows, C))


def _backward(lib, d, rows, H, noalloc):
    outs = dict(dy=torch.empty_like(d["y"]), dr=torch.empty_like(d["r"]),
                dk=torch.empty_like(d["k"]), dv=torch.empty_like(d["v"]),
                dgate=torch.empty_like(d["gate"]), dbonus=torch.empty_like(d["bonus"]),
                dweight=torch.empty_like(d["weight"]), dbias=torch.empty_like(d["bias"]))
    ins = [d[n].data_ptr() for n in ("y", "r", "k", "v", "gate", "bonus", "weight", "bias")]
    grads = [outs[n].data_ptr() for n in ("dy", "dr", "dk", "dv", "dgate", "dbonus",
                                           "dweight", "dbias")]
    stream = torch.cuda.current_stream().cuda_stream
    if noalloc:
        rc = lib.rwkv_gated_readout_backward_noalloc(*ins, 64e-5, rows, H, 64, BF16, BF16,
                                                     d["dout"].data_ptr(), *grads, stream)
    else:
        nbytes = lib.rwkv_gated_readout_workspace_bytes(rows, H, 64)
        ws = torch.empty(max(nbytes // 4, 1), dtype=torch.float32, device="cuda")
        rc = lib.rwkv_gated_readout_backward(*ins, 64e-5, rows, H, 64, BF16, BF16,
                                             d["dout"].data_ptr(), *grads, ws.data_ptr(),
                                             nbytes, stream)
    assert rc == 0, lib.wkv7_strerror(rc)
    torch.cuda.synchronize()
    return outs


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
