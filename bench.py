"""WKV7 fwd+bwd benchmark on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--config cfg0|cfg1|cfg2|cfg3|cfg4]

A step is one forward and one backward pass of the WKV7 statepass operator
(initial state in, final-state gradient zero, 16-step checkpoints) over one
batch of synthetic operands, called through the C ABI with device-resident
buffers allocated once. The default workload is the headline one:
B=8, T=4096, H=32, N=64, bf16 operands, fp32 state and accumulation,
initial state ~ N(0, 0.1).

Printed JSON line: whole-job Mtokens/s (wall clock over the K timed steps),
ms per step, and:
- "dtype"/"arithmetic": what the kernels compute in. With bf16 operands and
  chunk_len 16 the chunked matrix-core kernels run: fp32 state and
  accumulation, products of fp32 operands from bf16 hi/lo halves
  (hi*hi + hi*lo + lo*hi); with fp32 operands the fp32 chunked kernels:
  fp32 products on the fp32 matrix cores and fp32 sums;
- "roofline": the dominant kernel (the backward): algorithmic FP32 FLOPs per
  launch / mean launch time (HIP events on the launch stream) against
  MI355X's 157.3 TFLOP/s FP32 peak, with "traffic" (HBM bytes per launch from
  rocprofv3 FETCH_SIZE / WRITE_SIZE, profiles/) and "units": the issued bf16
  MFMA FLOPs against the 2.5 PFLOP/s dense bf16 peak and the VALU issue
  share, from rocprofv3 SQ counters recorded in profiles/;
- "cpu_baseline": the oracle (the reference's fp32 algorithm in its
  operation order, built -march=native, OpenMP over (batch, head) pairs) on
  the GPU run's operand bytes, forward and backward timed separately, median
  of 3 after a warm-up, with the host CPU model and thread count.
config cfg3 is the batched decode step (T=1), which is HBM-bound
(--state-dtype bf16: the reference's bf16 instantiation). config cfg4 is a
whole RWKV-7 0.1B training step (12 cells, C=768, vocab 65536, B=16, T=512)
with the WKV7 operator on the HIP kernels and every other op in PyTorch; it
reports the step time and the WKV7 share.
"""

from __future__ import annotations

import argparse
import importlib
import json
import os
import sys
import time

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

N_HEAD = 64
FLOP_FWD = 9 * N_HEAD * N_HEAD      # per head-step: sa 2N^2, update 5N^2, y 2N^2
FLOP_BWD = 24 * N_HEAD * N_HEAD     # per head-step, non-redundant backward
PEAK_FP32 = 157.3e12                # MI355X FP32 peak (packed VALU; also dense fp32 MFMA)
PEAK_HBM = 8.0e12                   # MI355X HBM3E
COLD_BYTES = 2 * 256 * 2**20   # state bytes the decode bench rotates over: twice the last-level cache
PEAK_BF16 = 2.5e15                  # MI355X dense bf16 MFMA
CLOCK_HZ = 2.4e9                    # MI355X peak engine clock
N_SIMDS = 256 * 4                   # 256 CUs of 4 SIMDs
COPY_PROBE_BYTES = 512 << 20        # fp32 stream (read once, write once) of --copy-probe
# HBM traffic of the dominant kernel per launch, from rocprofv3 FETCH_SIZE /
# WRITE_SIZE passes scaled by the copy probe; written by --pmc-summary
TRAFFIC_FILE = os.path.join(HERE, "profiles", "wkv7_bwd_cfg1_traffic.md")
TRAFFIC_FILE_DECODE = os.path.join(HERE, "profiles", "wkv7_infer_cfg3_traffic.md")
# issued MFMA FLOPs and VALU instructions per launch, from rocprofv3 SQ counters
COUNTER_FILE = os.path.join(HERE, "profiles", "wkv7_cfg1_sq_counters.md")
METRIC = "WKV7 fwd+bwd Mtokens/s (B=8,T=4096,C=2048) + % FP32-VALU / HBM roofline"

CONFIGS = {
    "cfg0": dict(B=1, T=64, H=4, io="f32", s0_std=None),
    "cfg1": dict(B=8, T=4096, H=32, io="bf16", s0_std=0.1),
    "cfg2": dict(B=4, T=4096, H=64, io="bf16", s0_std=None),
    "cfg3": dict(B=256, T=1, H=40, io="bf16", s0_std=0.1),
    "cfg4": dict(B=16, T=512, H=12, io="bf16", vocab=65536, cells=12),
}


def cpu_cores() -> int:
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return max(1, min(n, 16))   # the box's CPU share for one GPU is 16


def cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(cfg, d, budget_s=24.0, reps=3):
    """The oracle (the reference's fp32 algorithm in its operation order,
    oracle/wkv7_oracle.c, built here with -march=native, OpenMP over (batch,
    head) pairs) on the same seeded operand bytes as the GPU run (copied from
    the device). Forward and backward are timed separately: one warm-up pass,
    then the median of `reps` passes each. When a pass over the whole batch
    would exceed the budget the leading batch rows are the sample."""
    import statistics
    import tempfile

    import oracle
    B, T, H = cfg["B"], cfg["T"], cfg["H"]
    cores = cpu_cores()
    build = "native"
    try:
        oracle.build_native(os.path.join(tempfile.mkdtemp(prefix="wkv7_cpu_"), "libwkv7_oracle.so"))
    except Exception as e:   # no compiler: the prebuilt x86-64-v3 library
        build = f"prebuilt x86-64-v3 ({type(e).__name__})"
    names = ("w", "r", "k", "v", "a", "b")

    def host(t):
        return None if t is None else t.float().cpu().numpy()

    def sample(nb):
        ins = [host(d[n][:nb]) for n in names]
        s0 = host(d["s0"][:nb]) if d["s0"] is not None else None
        return ins, s0, host(d["dy"][:nb])

    def fwd(ins, s0):
        return oracle.forward_f32(*ins, s0=s0, chunk_len=16, nthreads=cores)

    def bwd(ins, f, dy):
        return oracle.backward_f32(*ins, f["state"], f["removal_state"], dy, chunk_len=16,
                                   nthreads=cores)

    # size the sample from one batch row, then warm up on the sample
    ins, s0, dy = sample(1)
    t0 = time.perf_counter()
    bwd(ins, fwd(ins, s0), dy)
    per_row = time.perf_counter() - t0
    nb = max(1, min(B, int(budget_s / (reps + 1) / max(per_row, 1e-6))))
    ins, s0, dy = sample(nb)
    f = fwd(ins, s0)
    bwd(ins, f, dy)
    tf, tb = [], []
    for _ in range(reps):
        t0 = time.perf_counter()
        f = fwd(ins, s0)
        t1 = time.perf_counter()
        bwd(ins, f, dy)
        t2 = time.perf_counter()
        tf.append(t1 - t0)
        tb.append(t2 - t1)
    mf, mb = statistics.median(tf), statistics.median(tb)
    tokens = nb * T
    return {"value": tokens / (mf + mb) / 1e6, "unit": "Mtokens/s", "cores": cores,
            "kind": "port",
            "fwd_s": mf, "bwd_s": mb, "cpu_model": cpu_model(), "nproc": os.cpu_count(),
            "sample": f"{nb} of {B} batch rows x {H} heads x T={T} (the GPU run's operand "
                      f"bytes), chunk 16; forward and backward timed separately, median of "
                      f"{reps} after one warm-up: fwd {mf:.3f} s, bwd {mb:.3f} s on {cores} "
                      f"OpenMP threads of '{cpu_model()}'; oracle/wkv7_oracle.c "
                      f"(reference operation order, fp32, {build} build)"}


def recorded_traffic(kernel: str, path: str = TRAFFIC_FILE):
    """Bytes per launch of `kernel` recorded in `path` ("traffic_bytes
    <kernel>: <int>" lines), or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"traffic_bytes {kernel}:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def recorded_counter(name: str, kernel: str, path: str):
    """A "<name> <kernel>: <int>" line of `path`, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.startswith(f"{name} {kernel}:"):
                    return int(line.split(":")[1])
    except OSError:
        pass
    return None


def copy_probe():
    """One streaming kernel over COPY_PROBE_BYTES (each byte read once and
    written once; an elementwise absolute value, since a same-dtype copy_ may
    become a DMA transfer instead of a kernel, and nothing else here launches
    that kernel): the scale for rocprofv3's FETCH_SIZE and WRITE_SIZE
    counters."""
    import torch
    n = COPY_PROBE_BYTES // 4
    src = torch.ones(n, device="cuda:0")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    torch.abs(src, out=dst)
    torch.cuda.synchronize()
    del src, dst


def pmc_summary(dirs):
    """Mean counter value per dispatch for each WKV7 kernel and the copy probe
    in rocprofv3 --pmc CSV output, and the traffic scaled by the probe."""
    import csv
    import glob
    from collections import defaultdict
    keys = ("wkv7_fwd_chunk_kernel", "wkv7_bwd_chunk_kernel", "wkv7_fwd_kernel",
            "wkv7_bwd_kernel", "wkv7_infer_kernel", "wkv7_infer_bf16_kernel", "AbsFunctor")
    per = defaultdict(lambda: defaultdict(lambda: defaultdict(float)))
    for d in dirs:
        for path in glob.glob(os.path.join(d, "**", "*counter_collection.csv"), recursive=True):
            with open(path) as f:
                for row in csv.DictReader(f):
                    name = row["Kernel_Name"]
                    key = next((k for k in keys if k in name), None)
                    if key is None:
                        continue
                    # rows of one dispatch (one per XCD / shader engine) add up
                    per[key][row["Counter_Name"]][row["Dispatch_Id"]] += float(row["Counter_Value"])
    # the probe is the last dispatch of its kernel
    for c, v in per.get("AbsFunctor", {}).items():
        last = max(v, key=int)
        per["AbsFunctor"][c] = {last: v[last]}
    mean = {k: {c: sum(v.values()) / len(v) for c, v in cs.items()} for k, cs in per.items()}
    probe_kib = COPY_PROBE_BYTES / 1024
    scale = {c: probe_kib / mean["AbsFunctor"][c] for c in ("FETCH_SIZE", "WRITE_SIZE")
             if "AbsFunctor" in mean and c in mean["AbsFunctor"]}
    print("| kernel | counter | KiB per dispatch | scale | bytes per dispatch |")
    print("|---|---|---|---|---|")
    totals = {}
    for k in keys:
        for c, v in sorted(mean.get(k, {}).items()):
            sc = scale.get(c)
            b = v * 1024 * sc if sc else None
            if b is not None and k != "AbsFunctor":
                totals[k] = totals.get(k, 0) + b
            print(f"| {k} | {c} | {v:.0f} | {sc if sc else '-'} | "
                  f"{'-' if b is None else f'{b:.0f}'} |")
    print()
    for k, b in totals.items():
        print(f"traffic_bytes {k}: {int(round(b))}")
    # the hardware units' view: issued bf16 MFMA FLOPs (the MOPS counter
    # counts in units of 512 FLOPs) and VALU instructions per dispatch
    for k in keys:
        cs = mean.get(k, {})
        if "SQ_INSTS_VALU_MFMA_MOPS_BF16" in cs:
            print(f"mfma_flop_issued {k}: {int(round(cs['SQ_INSTS_VALU_MFMA_MOPS_BF16'] * 512))}")
        if "SQ_INSTS_VALU" in cs:
            print(f"valu_insts {k}: {int(round(cs['SQ_INSTS_VALU']))}")


def short_kernel_name(name: str) -> str:
    """A rocprofv3 kernel name without return type, namespaces and arguments."""
    name = name.replace("void ", "").replace("(anonymous namespace)::", "")
    for ns in ("wkv7::", "rwkv_nb::", "rwkv_loss::"):
        name = name.replace(ns, "")
    return name.split("(")[0]


def neighbor_bytes(cfg):
    """Algorithmic HBM bytes per dispatch of the fused kernels beside the
    operator in the config[4] step (R tokens x C channels; fp32 residual
    stream, bf16 mixes, operands and gradients; bf16 logits)."""
    R, C, V = cfg["B"] * cfg["T"], cfg["H"] * N_HEAD, cfg["vocab"]
    rc = R * C
    return {
        "shift_mix_forward_kernel<false, true, 6>": (rc * 4 + 6 * rc * 2, "x fp32 in, 6 bf16 mixes out"),
        "shift_mix_forward_serial_kernel<false, true, 1>": (rc * 4 + rc * 2, "x fp32 in, 1 bf16 mix out"),
        "shift_mix_backward_kernel<false, true, 6>": (6 * rc * 2 + 2 * rc * 4, "6 bf16 mix grads + x in, dx fp32 out"),
        "shift_mix_backward_phased_kernel<false, true, 1>": (rc * 2 + 2 * rc * 4, "1 bf16 mix grad + x in, dx fp32 out"),
        "readout_forward_kernel<true, true>": (6 * rc * 2, "y, r, k~, v, gate bf16 in, out bf16"),
        "readout_backward_kernel<true, true>": (11 * rc * 2, "+ dout in; dy, dr, dk~, dv, dgate out"),
        "prepare_forward_kernel<true, true, true>": (11 * rc * 2, "6 bf16 products in, 5 bf16 operands out"),
        "prepare_forward_kernel<true, true, false>": (9 * rc * 2, "first cell: 4 in, 5 out"),
        "prepare_backward_kernel<true, true, true>": (17 * rc * 2, "6 products + 5 operand grads in, 6 grads out"),
        "prepare_backward_kernel<true, true, false>": (13 * rc * 2, "first cell: 4 + 5 in, 4 out"),
        "xent_forward_kernel<true, true>": (R * V * 2, f"bf16 logits in ({R} x {V})"),
        "xent_backward_kernel<true, true>": (2 * R * V * 2, "bf16 logits in, bf16 gradient out"),
    }


def kernel_category(name: str) -> str:
    if "wkv7::" in name:
        return "WKV7 (this library)"
    if "rwkv_nb::" in name:
        return "fused neighbours (this library)"
    if "rwkv_loss::" in name:
        return "fused loss (this library)"
    if name.startswith(("Cijk", "Custom_Cijk")):
        return "GEMM (hipBLASLt)"
    if "elementwise" in name or "Functor" in name:
        return "element-wise (torch)"
    if "reduce_kernel" in name:
        return "reductions (torch)"
    if "norm" in name.lower() or "GammaBeta" in name:
        return "layer/group norm (torch)"
    if "multi_tensor_apply" in name:
        return "optimizer (torch fused AdamW)"
    if "copyBuffer" in name or "fillBuffer" in name:
        return "runtime copies / fills"
    return "other (torch)"


def stats_summary(directory, config, traced_steps):
    """Markdown tables from a rocprofv3 --kernel-trace --stats CSV directory:
    this library's kernels (dispatches per traced step, mean / median / min /
    max duration); for cfg4 also GPU time by category and the fused
    neighbour kernels against their algorithmic bytes."""
    import csv
    import glob
    from collections import defaultdict

    def one(pattern):
        paths = glob.glob(os.path.join(directory, "**", pattern), recursive=True)
        if not paths:
            raise SystemExit(f"no {pattern} under {directory}")
        with open(paths[0]) as f:
            return list(csv.DictReader(f))

    stats, trace = one("*kernel_stats.csv"), one("*kernel_trace.csv")
    durs = defaultdict(list)
    for r in trace:
        durs[r["Kernel_Name"]].append(int(r["End_Timestamp"]) - int(r["Start_Timestamp"]))
    mine = [r for r in stats if any(s in r["Name"] for s in ("wkv7::", "rwkv_nb::", "rwkv_loss::"))]
    print(f"Traced steps: {traced_steps} (warm-up + timed).\n")
    print("| kernel | dispatches / step | mean µs | median µs | min µs | max µs | ms / step |")
    print("|---|---|---|---|---|---|---|")
    for r in sorted(mine, key=lambda r: -float(r["TotalDurationNs"])):
        d = sorted(durs[r["Name"]])
        print(f"| `{short_kernel_name(r['Name'])}` | {int(r['Calls']) / traced_steps:g} | "
              f"{float(r['AverageNs']) / 1e3:.1f} | {d[len(d) // 2] / 1e3:.1f} | "
              f"{float(r['MinNs']) / 1e3:.1f} | {float(r['MaxNs']) / 1e3:.1f} | "
              f"{float(r['TotalDurationNs']) / 1e6 / traced_steps:.3f} |")
    if config != "cfg4":
        return
    total = sum(float(r["TotalDurationNs"]) for r in stats)
    cats = defaultdict(float)
    for r in stats:
        cats[kernel_category(r["Name"])] += float(r["TotalDurationNs"])
    print(f"\nTraced GPU kernel time: {total / 1e6 / traced_steps:.2f} ms per step.\n")
    print("| category | ms / step | share |\n|---|---|---|")
    for c, v in sorted(cats.items(), key=lambda kv: -kv[1]):
        print(f"| {c} | {v / 1e6 / traced_steps:.2f} | {100 * v / total:.1f}% |")
    alg = neighbor_bytes(CONFIGS[config])
    print("\nFused neighbour and loss kernels against their algorithmic bytes (median "
          "dispatch; MI355X HBM peak 8 TB/s):\n")
    print("| kernel | median µs | algorithmic MB | achieved TB/s | of peak | bytes |")
    print("|---|---|---|---|---|---|")
    for name, d in durs.items():
        k = short_kernel_name(name)
        if k in alg:
            d = sorted(d)
            med = d[len(d) // 2] * 1e-9
            nb, what = alg[k]
            print(f"| `{k}` | {med * 1e6:.1f} | {nb / 1e6:.1f} | {nb / med / 1e12:.2f} | "
                  f"{nb / med / PEAK_HBM:.2f} | {what} |")


def bench_train(cfg, steps, warmup, with_cpu, probe=False, kernels="auto"):
    import torch
    pkg = importlib.import_module("rwkv-rs_amd")
    native = importlib.import_module("rwkv-rs_amd._native")
    lib = native.lib()
    B, T, H, C = cfg["B"], cfg["T"], cfg["H"], 16
    io = torch.bfloat16 if cfg["io"] == "bf16" else torch.float32
    dev = torch.device("cuda:0")
    d = pkg.synthetic.make_inputs_torch(B, T, H, N_HEAD, seed=0x5EED0001, s0_std=cfg["s0_std"],
                                        dtype=io, device=dev)
    s0 = d["s0"] if d["s0"] is not None else torch.zeros(B, H, N_HEAD, N_HEAD, device=dev)
    names = ("w", "r", "k", "v", "a", "b")
    ins = [d[n].data_ptr() for n in names]
    ckpt = torch.empty(B, H, T // C, N_HEAD, N_HEAD, device=dev)
    sa = torch.empty(B, T, H, N_HEAD, device=dev)
    y = torch.empty(B, T, H, N_HEAD, device=dev, dtype=io)
    sT = torch.empty_like(s0)
    dsT = torch.zeros_like(s0)
    grads = [torch.empty(B, T, H, N_HEAD, device=dev, dtype=io) for _ in range(6)]
    ds0 = torch.empty_like(s0)
    dtype_code = native.DTYPE_BF16 if io == torch.bfloat16 else native.DTYPE_F32
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    # the statepass operator (flags 1, 1 both ways) with an explicit kernel family
    opts = native.Wkv7Options(native.KERNELS_STEP if kernels == "step" else native.KERNELS_AUTO, 0)
    optp = native.options_ref(opts)

    def fwd():
        native.check(lib.wkv7_forward_ex(*ins, s0.data_ptr(), B, T, H, N_HEAD, C, dtype_code,
                                         1, 1, ckpt.data_ptr(), sa.data_ptr(), y.data_ptr(),
                                         sT.data_ptr(), optp, sp))

    def bwd():
        native.check(lib.wkv7_backward_ex(*ins, ckpt.data_ptr(), sa.data_ptr(),
                                          d["dy"].data_ptr(), dsT.data_ptr(), B, T, H, N_HEAD, C,
                                          dtype_code, 1, 1, *(g.data_ptr() for g in grads),
                                          ds0.data_ptr(), optp, sp))

    for _ in range(warmup):
        fwd()
        bwd()
    torch.cuda.synchronize()
    if probe:
        copy_probe()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True),
           torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for e0, e1, e2 in ev:
        e0.record(stream)
        fwd()
        e1.record(stream)
        bwd()
        e2.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # outside the timed region: no chunked forward gave up a hand-over wait
    importlib.import_module("rwkv-rs_amd.wkv7").check_faults(dev)
    fwd_each = sorted(a.elapsed_time(b) for a, b, _ in ev)
    bwd_each = sorted(b.elapsed_time(c) for _, b, c in ev)
    fwd_ms = sum(fwd_each) / steps          # mean launch time, as rocprofv3's average
    bwd_ms = sum(bwd_each) / steps
    ms_per_step = wall * 1e3 / steps
    head_steps = B * T * H
    tok = B * T
    bwd_flops = FLOP_BWD * head_steps
    fwd_flops = FLOP_FWD * head_steps
    achieved = bwd_flops / (bwd_ms * 1e-3)
    e = 2 if io == torch.bfloat16 else 4
    # which kernels ran (launch_forward / launch_backward dispatch; chunk_len
    # is 16 here): the chunked kernels of the operand type, or the step kernels
    chunked = C == 16 and T % 16 == 0 and kernels == "auto"
    f32_chunked = chunked and io == torch.float32
    tag = "f32_chunk" if f32_chunked else "chunk"
    bwd_kernel = f"wkv7_bwd_{tag}_kernel" if chunked else "wkv7_bwd_kernel"
    fwd_kernel = f"wkv7_fwd_{tag}_kernel" if chunked else "wkv7_fwd_kernel"
    # algorithmic HBM bytes per head-step: fwd 7 rows in/out (e bytes) + sa
    # out + 1/16 of a checkpoint; bwd 7 rows + sa in, 6 gradients out, 1/16
    # of a checkpoint in
    fwd_bytes = head_steps * (7 * N_HEAD * e + N_HEAD * 4 + N_HEAD * N_HEAD * 4 / C)
    bwd_bytes = head_steps * (13 * N_HEAD * e + N_HEAD * 4 + N_HEAD * N_HEAD * 4 / C)
    if f32_chunked:
        arithmetic = ("fp32 throughout: the chunked matrix form with fp32 products on the fp32 "
                      "matrix cores (v_mfma_f32_16x16x4_f32) and fp32 sums; fp32 operands and "
                      "outputs")
        dtype = "f32"
    elif chunked:
        arithmetic = ("fp32 state, checkpoints and accumulation; matrix products of two fp32 "
                      "operands formed from bf16 hi/lo halves as hi*hi + hi*lo + lo*hi on the "
                      "bf16 matrix cores (about 16 significant bits per product), products with "
                      "a bf16 input exact; bf16 operands and outputs")
        dtype = "f32-acc/split-bf16-mfma"
    else:
        arithmetic = "fp32 VALU throughout (fp32 products and sums); operands and outputs " + cfg["io"]
        dtype = "f32"
    # the hardware units' view of the dominant kernel: issued MFMA FLOPs and
    # VALU instructions per launch (rocprofv3 counters recorded in profiles/)
    units = {}
    mops = recorded_counter("mfma_flop_issued", bwd_kernel, COUNTER_FILE)
    valu = recorded_counter("valu_insts", bwd_kernel, COUNTER_FILE)
    if mops:
        units["mfma_bf16_tflops"] = mops / (bwd_ms * 1e-3) / 1e12
        units["mfma_bf16_frac"] = mops / (bwd_ms * 1e-3) / PEAK_BF16
    if valu:
        units["valu_issue_frac"] = valu * 4 / (bwd_ms * 1e-3 * CLOCK_HZ * N_SIMDS)
    if mops and valu:
        # a SIMD does not overlap VALU and MFMA instructions (measured on the
        # box: a wave of independent FMAs and a wave of independent MFMAs on
        # one SIMD take the sum of their times alone), so the share of the
        # SIMDs' time spent issuing the two is the sum of the two fractions
        units["simd_busy_frac"] = units["valu_issue_frac"] + units["mfma_bf16_frac"]
    out = {
        "metric": METRIC,
        "value": tok / (ms_per_step * 1e-3) / 1e6,
        "unit": "Mtokens/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": ms_per_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dtype,
        "arithmetic": arithmetic,
        "data": "synthetic",
        "config": {"workload": "wkv7_statepass_fwd_bwd", "batch": B, "context_len": T,
                   "num_heads": H, "head_size": N_HEAD, "chunk_len": C, "io_dtype": cfg["io"],
                   "state_dtype": "f32", "initial_state_std": cfg["s0_std"]},
        "roofline": {"bound": "mfma" if chunked else "valu", "kernel": bwd_kernel,
                     "achieved": achieved / 1e12,
                     "peak": PEAK_FP32 / 1e12, "unit": "TFLOP/s", "frac": achieved / PEAK_FP32,
                     "traffic": recorded_traffic(bwd_kernel),
                     "algorithmic_bytes": bwd_bytes,
                     "flop_per_launch": bwd_flops, "launch_ms": bwd_ms,
                     "launch_ms_median": bwd_each[steps // 2],
                     "peak_note": "FP32-equivalent: the metric's algorithmic fp32 FLOPs "
                                  "against MI355X's 157.3 TFLOP/s FP32 peak",
                     "units": units},
        "kernels": ("chunked-mfma-f32" if f32_chunked else "chunked-mfma") if chunked else "step-valu",
        "fwd_ms": fwd_ms,
        "fwd_ms_median": fwd_each[steps // 2],
        "bwd_ms": bwd_ms,
        "bwd_ms_median": bwd_each[steps // 2],
        "fwd_roofline_frac": fwd_flops / (fwd_ms * 1e-3) / PEAK_FP32,
        "fwd_bwd_roofline_frac": (fwd_flops + bwd_flops) / ((fwd_ms + bwd_ms) * 1e-3) / PEAK_FP32,
        "fwd_hbm_frac_algorithmic": fwd_bytes / (fwd_ms * 1e-3) / PEAK_HBM,
        "bwd_hbm_frac_algorithmic": bwd_bytes / (bwd_ms * 1e-3) / PEAK_HBM,
        "fwd_traffic": recorded_traffic(fwd_kernel),
    }
    if with_cpu:
        out["cpu_baseline"] = cpu_baseline(cfg, d)
    return out


def bench_decode(cfg, steps, warmup, probe=False, state_dtype="f32"):
    import torch
    pkg = importlib.import_module("rwkv-rs_amd")
    native = importlib.import_module("rwkv-rs_amd._native")
    lib = native.lib()
    B, T, H = cfg["B"], cfg["T"], cfg["H"]
    dev = torch.device("cuda:0")
    d = pkg.synthetic.make_inputs_torch(B, T, H, N_HEAD, seed=0x5EED0003, s0_std=0.1,
                                        dtype=torch.bfloat16, device=dev)
    bf16_state = state_dtype == "bf16"
    state = d["s0"].to(torch.bfloat16 if bf16_state else torch.float32).contiguous()
    # A serving loop decodes every layer in turn, so between two steps of one
    # layer the other layers' states pass through the caches: the timed steps
    # rotate over state buffers whose total exceeds MI355X's 256 MB last-level
    # cache, so that each step reads its state from HBM. One buffer, reused
    # step after step, is timed too (hot: the state stays cached).
    nbuf = -(-COLD_BYTES // (state.numel() * state.element_size()))
    states = [state] + [state.clone() for _ in range(nbuf - 1)]
    ids = torch.arange(B, dtype=torch.int32, device=dev)
    et = torch.zeros(B, dtype=torch.int32, device=dev)
    y = torch.empty(B, T, H, N_HEAD, device=dev, dtype=torch.bfloat16)
    names = ("w", "r", "k", "v", "a", "b")
    stream = torch.cuda.current_stream(dev)

    def step(st):
        native.check(lib.wkv7_infer_forward(*(d[n].data_ptr() for n in names), ids.data_ptr(),
                                            st.data_ptr(), None, et.data_ptr(), B, T, H,
                                            N_HEAD, B, native.DTYPE_BF16,
                                            native.DTYPE_BF16 if bf16_state else native.DTYPE_F32,
                                            int(bf16_state), y.data_ptr(), stream.cuda_stream))

    def timed(bufs):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0 = time.perf_counter()
        e0.record(stream)
        for i in range(steps):
            step(bufs[i % len(bufs)])
        e1.record(stream)
        torch.cuda.synchronize()
        return time.perf_counter() - t0, e0.elapsed_time(e1) / steps

    for i in range(warmup):
        step(states[i % nbuf])
    torch.cuda.synchronize()
    if probe:
        copy_probe()
    wall, launch_ms = timed(states)
    _, hot_ms = timed([state])
    nbytes = B * H * (2 * N_HEAD * N_HEAD * (2 if bf16_state else 4) + 7 * T * N_HEAD * 2)
    return {
        "metric": "WKV7 batched decode Mtokens/s (B=256, T=1, H=40)",
        "value": B * T / (wall / steps) / 1e6, "unit": "Mtokens/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": wall * 1e3 / steps,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "bf16" if bf16_state else "f32",
        "data": "synthetic",
        "config": {"workload": "wkv7_infer_decode", "batch": B, "context_len": T,
                   "num_heads": H, "head_size": N_HEAD, "io_dtype": "bf16",
                   "state_dtype": state_dtype, "dither": bool(bf16_state)},
        "roofline": {"bound": "hbm",
                     "kernel": "wkv7_infer_bf16_kernel" if bf16_state else "wkv7_infer_kernel",
                     "achieved": nbytes / (launch_ms * 1e-3) / 1e9, "peak": PEAK_HBM / 1e9,
                     "unit": "GB/s", "frac": nbytes / (launch_ms * 1e-3) / PEAK_HBM,
                     "traffic": recorded_traffic("wkv7_infer_bf16_kernel" if bf16_state else "wkv7_infer_kernel",
                                                 TRAFFIC_FILE_DECODE),
                     "algorithmic_bytes": nbytes, "launch_ms": launch_ms,
                     "state_buffers": nbuf,
                     "hot": {"launch_ms": hot_ms, "achieved": nbytes / (hot_ms * 1e-3) / 1e9,
                             "note": "one state buffer reused: the state stays in the "
                                     "last-level cache between steps"}},
    }


# The reference's own kernel benchmark cases (crates/rwkv-nn/benches/kernels/
# mod.rs:109-113): (name, batch, context_len, heads, chunk_len), head size 64,
# run by its Criterion benches at element type f32 (mod.rs:11-12, Cuda<f32, i32>).
CRITERION_CASES = (("b1_t128_h8_d64_c32", 1, 128, 8, 32),
                   ("b2_t256_h8_d64_c32", 2, 256, 8, 32),
                   ("b4_t512_h16_d64_c64", 4, 512, 16, 64))


def bench_criterion(steps, warmup, with_cpu):
    """The calls the reference's Criterion benches time (benches/kernels/
    wkv7_{pretrain,statepass,statetune}/{forward,backward}.rs and
    wkv7_infer/forward.rs), on their three cases, through the C ABI: fp32
    operands, every input N(0, 1) as mod.rs:115-178 draws them (initial state,
    output and final-state gradients too), the infer call over the whole
    context with a Bernoulli(0.95) mask, batch_ids 0..B-1 and elapsed_t 0.
    Per call: the GPU time from HIP events around `steps` back-to-back calls,
    and the host time per call over the same loop (enqueue included, one
    synchronisation at the end, as a Criterion iteration without a device
    sync inside measures)."""
    import torch
    native = importlib.import_module("rwkv-rs_amd._native")
    lib = native.lib()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    sp = stream.cuda_stream
    F32 = native.DTYPE_F32
    g = torch.Generator(device="cpu").manual_seed(0x5EED0005)
    cases, cpu = {}, {}
    total_us = 0.0
    for name, B, T, H, C in CRITERION_CASES:
        def rnd(*shape):
            return torch.randn(*shape, generator=g).to(dev)
        ins = [rnd(B, T, H, N_HEAD) for _ in range(6)]
        ip = [t.data_ptr() for t in ins]
        s0, dy, dsT = rnd(B, H, N_HEAD, N_HEAD), rnd(B, T, H, N_HEAD), rnd(B, H, N_HEAD, N_HEAD)
        mask = (torch.rand(B, T, generator=g) < 0.95).float().to(dev)
        ids = torch.arange(B, dtype=torch.int32, device=dev)
        et = torch.zeros(B, dtype=torch.int32, device=dev)
        ckpt = torch.empty(B, H, T // C, N_HEAD, N_HEAD, device=dev)
        sa, y = torch.empty(B, T, H, N_HEAD, device=dev), torch.empty(B, T, H, N_HEAD, device=dev)
        sT, ds0 = torch.empty_like(s0), torch.empty_like(s0)
        grads = [torch.empty(B, T, H, N_HEAD, device=dev) for _ in range(6)]
        gp = [t.data_ptr() for t in grads]
        state = s0.clone()
        dims = (B, T, H, N_HEAD, C)
        calls = {
            "pretrain_forward": lambda: lib.wkv7_pretrain_forward(
                *ip, *dims, F32, ckpt.data_ptr(), sa.data_ptr(), y.data_ptr(), sp),
            "pretrain_backward": lambda: lib.wkv7_pretrain_backward(
                *ip, ckpt.data_ptr(), sa.data_ptr(), dy.data_ptr(), *dims, F32, *gp, sp),
            "statepass_forward": lambda: lib.wkv7_statepass_forward(
                *ip, s0.data_ptr(), *dims, F32, ckpt.data_ptr(), sa.data_ptr(), y.data_ptr(),
                sT.data_ptr(), sp),
            "statepass_backward": lambda: lib.wkv7_statepass_backward(
                *ip, ckpt.data_ptr(), sa.data_ptr(), dy.data_ptr(), dsT.data_ptr(), *dims, F32,
                *gp, ds0.data_ptr(), sp),
            "statetune_forward": lambda: lib.wkv7_statetune_forward(
                *ip, s0.data_ptr(), *dims, F32, ckpt.data_ptr(), sa.data_ptr(), y.data_ptr(), sp),
            "statetune_backward": lambda: lib.wkv7_statetune_backward(
                *ip, ckpt.data_ptr(), sa.data_ptr(), dy.data_ptr(), *dims, F32, *gp,
                ds0.data_ptr(), sp),
            "infer_forward": lambda: lib.wkv7_infer_forward(
                *ip, ids.data_ptr(), state.data_ptr(), mask.data_ptr(), et.data_ptr(), B, T, H,
                N_HEAD, B, F32, F32, 0, y.data_ptr(), sp),
        }
        res = {}
        for call, fn in calls.items():
            for _ in range(warmup):
                native.check(fn())
            torch.cuda.synchronize()
            e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            t0 = time.perf_counter()
            e0.record(stream)
            for _ in range(steps):
                native.check(fn())
            e1.record(stream)
            torch.cuda.synchronize()
            host = (time.perf_counter() - t0) / steps
            res[call] = {"gpu_us": e0.elapsed_time(e1) * 1e3 / steps, "host_us": host * 1e6}
        cases[name] = res
        total_us += res["statepass_forward"]["gpu_us"] + res["statepass_backward"]["gpu_us"]
        if with_cpu:
            import oracle
            hn = [t.cpu().numpy() for t in ins]
            t0 = time.perf_counter()
            f = oracle.forward_f32(*hn, s0=s0.cpu().numpy(), chunk_len=C, nthreads=1)
            t1 = time.perf_counter()
            oracle.backward_f32(*hn, f["state"], f["removal_state"], dy.cpu().numpy(),
                                ds_T=dsT.cpu().numpy(), chunk_len=C, nthreads=1)
            t2 = time.perf_counter()
            cpu[name] = {"statepass_forward_us": (t1 - t0) * 1e6, "statepass_backward_us": (t2 - t1) * 1e6}
    out = {
        "metric": "WKV7 statepass forward+backward latency on the reference's Criterion cases "
                  "(F=f32), summed over the three cases",
        "value": total_us, "unit": "us", "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": total_us / 1e3, "higher_is_better": False, "scaling": "strong",
        "vs_baseline": None, "dtype": "f32", "data": "synthetic",
        "config": {"workload": "wkv7_criterion_cases",
                   "cases": [dict(zip(("name", "batch", "context_len", "num_heads", "chunk_len"), c))
                             for c in CRITERION_CASES]},
        "cases": cases,
    }
    if with_cpu:
        out["cpu_baseline"] = {
            "value": sum(v["statepass_forward_us"] + v["statepass_backward_us"] for v in cpu.values()),
            "unit": "us", "cores": 1, "kind": "port", "cpu_model": cpu_model(),
            "sample": "the same three cases and operand bytes, statepass forward and backward "
                      "once each on one thread (oracle/wkv7_oracle.c, reference operation order)",
            "cases": cpu}
    return out


def bench_lm(cfg, steps, warmup, neighbor_ops="hip"):
    """config[4]: one RWKV-7 0.1B training step (forward, loss, backward, Adam
    update) on the host framework with the WKV7 operator on the HIP kernels;
    reports the step time and the share of it spent in the WKV7 launches,
    from timing events recorded around each launch on the launch stream."""
    import torch
    model_mod = importlib.import_module("rwkv-rs_amd.model")
    wkv7 = importlib.import_module("rwkv-rs_amd.wkv7")
    B, T, H = cfg["B"], cfg["T"], cfg["H"]
    C, V, L = H * N_HEAD, cfg["vocab"], cfg["cells"]
    dev = torch.device("cuda:0")
    gen = torch.Generator(device=dev).manual_seed(0x5EED0004)
    model = model_mod.AutoRegressiveModel(V, L, C, H, N_HEAD, neighbor_ops=neighbor_ops)
    model = model.to(dev).init_random(0.02, gen)
    opt = model_mod.make_optimizer(model)
    tokens = torch.randint(0, V, (B, T + 1), device=dev, generator=gen)
    inputs, targets = tokens[:, :-1].contiguous(), tokens[:, 1:].contiguous()
    for _ in range(warmup):
        loss = model_mod.train_step(model, opt, inputs, targets)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream(dev)
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    log = []
    t0 = time.perf_counter()
    e0.record(stream)
    with wkv7.kernel_events(log):
        for _ in range(steps):
            loss = model_mod.train_step(model, opt, inputs, targets)
    e1.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    wkv7.check_faults(dev)
    step_ms = e0.elapsed_time(e1) / steps
    fwd_ms = sum(a.elapsed_time(b) for n, a, b in log if n == "forward") / steps
    bwd_ms = sum(a.elapsed_time(b) for n, a, b in log if n == "backward") / steps
    ms_per_step = wall * 1e3 / steps
    return {
        "metric": "RWKV-7 0.1B train step tokens/s (B=16, T=512) + WKV7 share",
        "value": B * T / (ms_per_step * 1e-3), "unit": "tokens/s", "n_gpus": 1,
        "steps": steps, "warmup": warmup, "ms_per_step": ms_per_step,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "rwkv7_0.1b_train_step", "batch": B, "context_len": T,
                   "num_cells": L, "embedded_dim": C, "num_heads": H, "head_size": N_HEAD,
                   "vocab": V, "wkv7_io_dtype": "bf16", "matmul": "bf16 autocast",
                   "neighbor_ops": neighbor_ops,
                   "optimizer": "AdamW(0.9, 0.99, eps 1e-16)"},
        "gpu_step_ms": step_ms,
        "wkv7_fwd_ms_per_step": fwd_ms, "wkv7_bwd_ms_per_step": bwd_ms,
        "wkv7_share": (fwd_ms + bwd_ms) / step_ms,
        "wkv7_launches_per_step": len(log) / steps,
        "final_loss": float(loss),
    }


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    # the backward's dispatch time settles only after about 20 back-to-back
    # passes (about 30 ms of load: 1.16 ms falling to 0.89 ms at config[1],
    # the forward unchanged); the default warm-up covers that ramp
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--config", default="cfg1", choices=sorted(CONFIGS) + ["criterion"],
                    help="cfg0-cfg4: the metric's configurations config[0]-config[4] (CONFIGS); criterion: the calls of the "
                         "reference's own Criterion benches on their three cases")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--state-dtype", default="f32", choices=("f32", "bf16"),
                    help="cfg3: the decode state's element type")
    ap.add_argument("--kernels", default="auto", choices=("auto", "step"),
                    help="cfg0-cfg2: the library's choice, or the step-by-step kernels throughout")
    ap.add_argument("--io", default=None, choices=("bf16", "f32"),
                    help="cfg0-cfg2: the operands' element type instead of the configuration's "
                         "own (e.g. config[1]'s shape with fp32 operands)")
    ap.add_argument("--neighbor-ops", default="hip", choices=("hip", "torch"),
                    help="cfg4: the ops beside the operator as fused kernels or torch ops")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also launch one plain copy of known size (counter calibration)")
    ap.add_argument("--pmc-summary", nargs="+", metavar="DIR",
                    help="summarise rocprofv3 --pmc CSV output directories and exit")
    ap.add_argument("--stats-summary", metavar="DIR",
                    help="summarise a rocprofv3 --kernel-trace --stats CSV directory of a "
                         "--config run and exit")
    ap.add_argument("--traced-steps", type=int, default=0,
                    help="--stats-summary: steps the trace holds (default warm-up + steps)")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(args.pmc_summary)
        return
    if args.stats_summary:
        stats_summary(args.stats_summary, args.config,
                      args.traced_steps or (args.steps + args.warmup))
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the WKV7 operator needs no collective, and "
              "this build runs one process on one GPU (sharding over (batch, head) pairs "
              "across GPUs is not built)",
              file=sys.stderr)
        sys.exit(2)
    if args.config == "criterion":
        print(json.dumps(bench_criterion(args.steps, args.warmup, with_cpu=not args.no_cpu)), flush=True)
        return
    cfg = CONFIGS[args.config]
    if args.config == "cfg4":
        out = bench_lm(cfg, args.steps, args.warmup, args.neighbor_ops)
    elif args.config == "cfg3":
        out = bench_decode(cfg, args.steps, args.warmup, probe=args.copy_probe,
                           state_dtype=args.state_dtype)
    else:
        if args.io:
            cfg = dict(cfg, io=args.io)
        out = bench_train(cfg, args.steps, args.warmup,
                          with_cpu=(not args.no_cpu and args.config == "cfg1"),
                          probe=args.copy_probe, kernels=args.kernels)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
