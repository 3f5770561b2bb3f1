#!/usr/bin/env python3
"""SpartonHead forward+backward throughput on one MI355X.

A step is one training pass of the head over one batch of synthetic inputs already
resident in HBM: reps = head(hidden, mask); reps.backward(grad) through
SpartonHead + autograd (grads set to None first, as an optimizer's
zero_grad(set_to_none=True) does). The workload is BASELINE.json's headline
configuration (B=32, S=256, D=768, V=30522, bf16) unless --config says otherwise.

Prints ONE JSON line. Besides the throughput it reports:
  roofline      the forward's main kernel (MFMA-bound): useful flops
                2*D*V*sum_b(len_b) per launch / its mean duration, measured with HIP
                events that sparton_fwd_profile records on the launch stream just before
                and after that kernel, vs 2.5 PFLOP/s. The whole forward op (plan + main +
                fixup kernels) is also timed with HIP events around the forward of each
                step of a separate, untimed pass of steps (`op_ms`). `traffic` is the kernel's HBM bytes per launch from
                rocprofv3 FETCH_SIZE/WRITE_SIZE passes, read from
                profiles/hbm_traffic_cfg<N>.json when that file covers this workload.
  bwd_roofline  the backward kernels (HBM-bound): compulsory bytes per call / their
                mean duration from the same in-step HIP events, vs 8 TB/s.
The timed region holds the K steps and nothing else: an event recorded between two
kernels drains the queue, so the per-op events live in their own pass.
  transform     the MLM transform in front of the head (dense, gelu, LayerNorm) at the
                same rows and width: fused op vs eager torch fwd+bwd, and each HIP
                epilogue kernel's compulsory bytes / mean duration vs 8 TB/s.
  loss          the SPLADE loss on reps of this shape (B queries, B documents): fused
                vs eager torch fwd+bwd, and the HIP passes' compulsory bytes vs 8 TB/s.
  library_gemm  torch.matmul (hipBLASLt) at the main kernel's executed GEMM shape.
  cpu_baseline  the reference's torch head (training/model.py:56-62, restated in
                oracle/) fwd+bwd on the host cores, on a bounded sample of batch rows;
                also its forward alone and the peak resident memory a step adds.
"""
import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "fused head fwd+bwd tokens/sec & MFMA util, B32 S256 V30522 bf16; peak GB"
PEAK_TFLOPS = {"bf16": 2500.0, "fp16": 2500.0, "fp32": 157.3}
PEAK_HBM_GBS = 8000.0
DTYPE_NAME = {"torch.bfloat16": "bf16", "torch.float16": "fp16", "torch.float32": "fp32"}


def parse():
    p = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--config", type=int, default=2, help="workload index (BASELINE.json configs, 1-based)")
    p.add_argument("--kernel-reps", type=int, default=50, help="back-to-back launches per kernel timing")
    p.add_argument("--cpu-seconds", type=float, default=25.0, help="budget (s) of the CPU baseline leg")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--fp32-precision", choices=["high", "highest"], default="high",
                   help="torch float32 matmul precision for fp32 workloads; the reference sets "
                        "'high' when it is imported (sparton_kernel.py:14)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="after timing, launch one device copy of this many MiB (PMC calibration)")
    return p.parse_args()


def cpu_model():
    try:
        for ln in open("/proc/cpuinfo"):
            if ln.startswith("model name"):
                return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


FWD_KERNEL = "sparton::fwd::sparton_fwd_kernel<%s>"
KNAME = {"bf16": "bf16", "fp16": "f16", "fp32": "f32"}
# Batches of at most 128 rows (B * S) run one kernel, one wave per 32 vocab columns: fp32
# always, 16-bit up to B * S * V = 2^24.
SMALL_MAX_ROWS = 128
SMALL_KERNEL = "sparton::fwd::fwd_small_kernel<%s, %d, %s>"
SMALL_TNAME = {"bf16": "__bf16", "fp16": "_Float16", "fp32": "float"}


def small_path(w, dname):
    return w.B * w.S <= SMALL_MAX_ROWS and (dname == "fp32" or w.B * w.S * w.V <= 1 << 24)


def fwd_kernel_name(w, dname, split):
    if small_path(w, dname):
        return SMALL_KERNEL % (SMALL_TNAME[dname], min(4, -(-w.B * w.S // 32)),
                               "true" if split else "false")
    return FWD_KERNEL % KNAME[dname]


def measured_traffic(config, kernel):
    """HBM bytes per launch of `kernel` from the committed PMC summary for this config
    (sparton_amd.profiling traffic output), or (None, reason)."""
    path = os.path.join(ROOT, "profiles", f"hbm_traffic_cfg{config}.json")
    try:
        with open(path) as f:
            k = json.load(f)["kernels"][kernel]
    except (OSError, KeyError, ValueError):
        return None, "no PMC summary for this workload"
    return k["traffic_bytes"], os.path.relpath(path, ROOT)


def time_events(torch, fn, reps):
    """Mean GPU time of fn() from HIP events on the current stream, fn launched
    back to back so the GPU never waits for the host between launches."""
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    fn()
    torch.cuda.synchronize()
    start.record()
    for _ in range(reps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / reps


def _rss_kib(field):
    """VmRSS / VmHWM of this process in KiB (Linux /proc), or None."""
    try:
        for ln in open("/proc/self/status"):
            if ln.startswith(field + ":"):
                return int(ln.split()[1])
    except OSError:
        pass
    return None


def _reset_peak_rss():
    """Reset this process's peak resident set size (VmHWM) to its current size; True if the
    kernel took the request (Linux >= 4.0, /proc/self/clear_refs)."""
    try:
        with open("/proc/self/clear_refs", "w") as f:
            f.write("5")
        return True
    except OSError:
        return False


def cpu_baseline(torch, w, inp, budget_s):
    """The reference torch head on the host, on the first rows of the batch: fwd+bwd through
    autograd (the value), the forward alone (autograd on, as in training), and the peak
    resident memory one fwd+bwd step adds to the process."""
    import resource

    import oracle
    # every core this process may run on (its CPU affinity), recorded beside the host's count
    threads = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    torch.set_num_threads(threads)
    state = {}

    def prepare(rows):
        state["rows"] = rows
        state["H"] = inp.hidden[:rows].clone().requires_grad_()
        state["W"] = inp.weight.clone().requires_grad_()
        state["b"] = inp.bias.clone().requires_grad_() if inp.bias is not None else None
        state["m"], state["G"] = inp.mask[:rows], inp.grad[:rows]

    def fwd():
        return oracle.torch_head_chunked(state["H"], state["W"], state["b"], state["m"], v_chunk=8192)

    def step():
        fwd().backward(state["G"])

    def timed(fn=step):
        t0 = time.perf_counter()
        fn()
        return time.perf_counter() - t0

    # Size the sample so that about 5 timed steps fill the budget; when the whole batch takes
    # less, repeat it so that the timed steps fill about 60% of the budget and the timed
    # forwards about 20% (at least 5 of each, at most 50).
    prepare(1)
    timed()  # first call pays one-time costs
    per_row = timed()
    rows = max(1, min(w.B, int(budget_s / (5 * per_row))))
    prepare(rows)
    t_warm = timed()  # warm-up at the final size
    reps = max(5, min(50, int(0.6 * budget_s / max(t_warm, 1e-6))))
    times = [timed() for _ in range(reps)]
    t = statistics.median(times)
    t_fwd_warm = timed(fwd)
    fwd_reps = max(5, min(50, int(0.2 * budget_s / max(t_fwd_warm, 1e-6))))
    fwd_times = [timed(fwd) for _ in range(fwd_reps)]
    t_fwd = statistics.median(fwd_times)
    # peak memory of one fwd+bwd step above what the process held before it
    hwm_reset = _reset_peak_rss()
    rss0, maxrss0 = _rss_kib("VmRSS"), resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
    step()
    hwm1, maxrss1 = _rss_kib("VmHWM"), resource.getrusage(resource.RUSAGE_SELF).ru_maxrss
    peak_delta_kib = (hwm1 - rss0) if (hwm_reset and hwm1 is not None and rss0 is not None) \
        else maxrss1 - maxrss0
    n = len(times)
    return {
        "value": rows * w.S / t,
        "seconds": round(sum(times) + sum(fwd_times), 2),
        "unit": "tokens/s",
        "cores": torch.get_num_threads(),
        "fwd_tokens_per_s": rows * w.S / t_fwd,
        "fwd_bwd_ms": round(t * 1e3, 2),
        "fwd_ms": round(t_fwd * 1e3, 2),
        "peak_rss_delta_gb": round(peak_delta_kib * 1024 / 1e9, 3),
        "peak_rss_basis": ("VmHWM after one fwd+bwd step minus VmRSS before it, the peak reset "
                           "through /proc/self/clear_refs" if hwm_reset else
                           "getrusage ru_maxrss delta over one fwd+bwd step (a lower bound: the "
                           "process's earlier peak could not be reset)"),
        "host_cpu_count": os.cpu_count(),
        "affinity_cpus": threads,
        "omp_num_threads_env": os.environ.get("OMP_NUM_THREADS"),
        "kind": "port",
        "fp32_matmul_precision": torch.get_float32_matmul_precision(),
        "sample": (f"torch head (training/model.py:56-62, restated in oracle/) fwd+bwd autograd "
                   f"(value) and fwd alone, {DTYPE_NAME[str(w.dtype)]}, {rows} of {w.B} batch rows "
                   f"({rows * w.S} tokens), V-chunked by 8192, median of {n} fwd+bwd steps and of "
                   f"{len(fwd_times)} forwards, each after 1 warm-up; "
                   f"host CPU: {cpu_model()}"),
    }


def time_main_kernel(torch, H, W, b, mask, reps_n):
    """Mean device time (ms) of the forward's main kernel: sparton_fwd_profile brackets
    its launch with HIP events on the launch stream (plan and fixup run as usual)."""
    import ctypes
    from sparton_amd import _lib
    L = _lib.load()
    B, S, D = H.shape
    V = W.shape[0]
    dt = _lib.fwd_dtype_code(H.dtype)
    reps = torch.empty((B, V), dtype=H.dtype, device=H.device)
    idx = torch.empty((B, V), dtype=torch.int32, device=H.device)
    reps32 = torch.empty((B, V), dtype=torch.float32, device=H.device)
    ws_bytes = int(L.sparton_fwd_workspace_bytes(B, S, D, V, dt))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=H.device)
    stream = torch.cuda.current_stream().cuda_stream
    ms = ctypes.c_float()
    times = []
    for i in range(reps_n + 3):
        rc = L.sparton_fwd_profile(H.data_ptr(), W.data_ptr(), _lib.ptr(b), mask.data_ptr(),
                                   _lib.MASK_CODE[mask.dtype], reps.data_ptr(), idx.data_ptr(),
                                   reps32.data_ptr(), B, S, D, V, dt, ws.data_ptr(), ws_bytes,
                                   stream, ctypes.byref(ms))
        _lib.check(rc, "sparton_fwd_profile")
        if i >= 3:
            times.append(ms.value)
    return statistics.mean(times)


def mfma_ceiling(torch, dtype_name, target_ms=1.0):
    """The MFMA rate all CUs sustain together on random 16-bit register operands, and their
    shader clock (sparton_mfma_probe): under a full MFMA load the GPU is power-limited, so
    this, not the nominal peak, is what the forward's main kernel can approach on this box."""
    import ctypes
    from sparton_amd import _lib
    if dtype_name not in ("bf16", "fp16"):
        return None
    L = _lib.load()
    dt = _lib.DTYPE_CODE[torch.bfloat16 if dtype_name == "bf16" else torch.float16]
    grid = torch.cuda.get_device_properties(0).multi_processor_count
    out = torch.empty(grid * 256, dtype=torch.float32, device="cuda")
    clk = torch.empty(grid * 2, dtype=torch.int64, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    flop_per_iter = grid * 4 * 16 * 2 * 32 * 32 * 16

    def run(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        _lib.check(L.sparton_mfma_probe(dt, grid, iters, out.data_ptr(), clk.data_ptr(), stream),
                   "sparton_mfma_probe")
        e1.record()
        torch.cuda.synchronize()
        return e0.elapsed_time(e1)

    run(200)
    iters = max(200, int(200 * target_ms / max(run(200), 1e-3)))
    ms = run(iters)
    c = clk.view(grid, 2).double()
    mhz = float((c[:, 0] / (c[:, 1] / 100.0)).mean())  # s_memrealtime ticks at 100 MHz
    return {"tflops": round(flop_per_iter * iters / (ms * 1e-3) / 1e12, 1), "clock_mhz": round(mhz),
            "ms": round(ms, 3), "workgroups": grid,
            "what": "sparton_mfma_probe: 4 waves per CU, independent v_mfma_f32_32x32x16 on random "
                    "register operands, all CUs at once (power-limited rate); HIP events"}


def library_gemm(torch, w, mask, reps_n):
    """torch.matmul (hipBLASLt) at the forward main kernel's executed GEMM shape: M = the
    packed rows it multiplies (active 16-position groups, rounded up to whole 256-row
    tiles), K = D, N = V, in the workload's 16-bit dtype, output in that dtype; timed back to
    back with HIP events. A dense library GEMM on random operands, for comparison with the
    fused kernel's rate (the kernel also reduces over S and never writes the [M, V] logits)."""
    if w.dtype not in (torch.bfloat16, torch.float16):
        return None
    dev = mask.device
    valid = torch.nn.functional.pad(mask.ne(0), (0, (-w.S) % 16))
    groups = int(valid.view(w.B, -1, 16).any(-1).sum())
    M = -(-groups // 16) * 256
    gen = torch.Generator(device=dev).manual_seed(3)
    A = torch.randn(M, w.D, device=dev, generator=gen).to(w.dtype)
    Wm = (torch.randn(w.V, w.D, device=dev, generator=gen) * 0.02).to(w.dtype)
    out = torch.empty(M, w.V, device=dev, dtype=w.dtype)
    fn = lambda: torch.matmul(A, Wm.t(), out=out)
    fn()
    ms = time_events(torch, fn, reps_n)
    flops = 2.0 * M * w.D * w.V
    tf = flops / (ms * 1e-3) / 1e12
    peak = PEAK_TFLOPS[DTYPE_NAME[str(w.dtype)]]
    del A, Wm, out
    return {"M": M, "K": w.D, "N": w.V, "ms": round(ms, 4), "tflops": round(tf, 1),
            "frac_of_peak": round(tf / peak, 4),
            "out_bytes": M * w.V * torch.tensor([], dtype=w.dtype).element_size(),
            "what": "torch.matmul(A[M,K], W[N,K].t()) -> [M,N] (hipBLASLt), the main kernel's "
                    "executed rows; HIP events over back-to-back calls"}


def time_device(torch, fn, reps):
    """Mean GPU time of fn() when the host is never the bottleneck: a bounded spin kernel
    (torch.cuda._sleep) holds the queue while all reps are enqueued, so the events bracket
    back-to-back GPU work only. Two held passes run and the second is reported: the first
    held pass of a process has measured up to 4x slower on the host (launch resources the
    runtime sets up the first time that many launches are outstanding). Returns (device ms,
    host-bound ms of plain back-to-back, host ms to enqueue the reps)."""
    host_ms = time_events(torch, fn, reps)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    for _ in range(2):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        torch.cuda._sleep(int(2.5e6 * (host_ms * reps * 2.0 + 5.0)))  # cycles at <= 2.5 GHz
        start.record()
        for _ in range(reps):
            fn()
        end.record()
        enqueue_ms = (time.perf_counter() - t0) * 1e3
        torch.cuda.synchronize()
    dev_ms = start.elapsed_time(end) / reps
    return dev_ms, host_ms, enqueue_ms


def transform_timing(torch, w, dev, reps_n):
    """The MLM transform at this workload's M=B*S rows and width D (training/model.py:14-40):
    SpartonMLMTransform's path (hipBLASLt GEMMs + the HIP epilogues) against the same
    computation in eager torch, both fwd+bwd through autograd, and each epilogue kernel alone
    against the bytes it must move (z read and y written; dy and z read and dz written; fp32
    row statistics)."""
    import torch.nn.functional as F
    from sparton_amd import _lib
    from sparton_amd import _eager
    L = _lib.load()
    M, D, dt = w.B * w.S, w.D, w.dtype
    if D % 4 or D > 3072:
        return None
    gen = torch.Generator(device=dev).manual_seed(7)
    x = torch.randn(M, D, device=dev, generator=gen).to(dt).requires_grad_()
    W = (torch.randn(D, D, device=dev, generator=gen) / D ** 0.5).to(dt).requires_grad_()
    vec = [torch.randn(D, device=dev, generator=gen).mul_(0.1).requires_grad_() for _ in range(3)]
    vec[1].data.add_(1.0)
    dy = torch.randn(M, D, device=dev, generator=gen).to(dt)
    eps = 1e-12

    def fused():
        x.grad = W.grad = None
        for v in vec:
            v.grad = None
        _eager.load().mlm_transform(x, W, vec[0], vec[1], vec[2], eps).backward(dy)

    vl = [v.detach().to(dt).requires_grad_() for v in vec]

    def eager():
        x.grad = W.grad = None
        for v in vl:
            v.grad = None
        F.layer_norm(F.gelu(F.linear(x, W, vl[0])), (D,), vl[1], vl[2], eps).backward(dy)

    fused_ms, fused_host, fused_enq = time_device(torch, fused, reps_n)
    eager_ms, eager_host, eager_enq = time_device(torch, eager, reps_n)

    with torch.no_grad():
        y, z, mean, rstd = torch.ops.sparton.mlm_transform_fwd(x, W, vec[0], vec[1], vec[2], eps)
    dz = torch.empty_like(z)
    dg, dbt, dbd = (torch.empty(D, dtype=torch.float32, device=dev) for _ in range(3))
    ws_bytes = int(L.sparton_transform_workspace_bytes(M, D))
    ws = torch.empty((max(ws_bytes, 1),), dtype=torch.uint8, device=dev)
    code, stream = _lib.DTYPE_CODE[dt], torch.cuda.current_stream().cuda_stream
    b0, g0, t0 = (v.detach() for v in vec)

    def epi_fwd():
        _lib.check(L.sparton_transform_fwd(z.data_ptr(), b0.data_ptr(), g0.data_ptr(), t0.data_ptr(),
                                           eps, y.data_ptr(), mean.data_ptr(), rstd.data_ptr(),
                                           M, D, code, stream), "sparton_transform_fwd")

    def epi_bwd():
        _lib.check(L.sparton_transform_bwd(dy.data_ptr(), z.data_ptr(), b0.data_ptr(), g0.data_ptr(),
                                           mean.data_ptr(), rstd.data_ptr(), dz.data_ptr(),
                                           dg.data_ptr(), dbt.data_ptr(), dbd.data_ptr(),
                                           ws.data_ptr(), ws_bytes, M, D, code, stream),
                   "sparton_transform_bwd")

    fwd_epi_ms = time_events(torch, epi_fwd, reps_n)
    bwd_epi_ms = time_events(torch, epi_bwd, reps_n)
    e = z.element_size()
    fwd_bytes = 2 * M * D * e + 8 * M + 3 * D * 4
    bwd_bytes = 3 * M * D * e + 8 * M + 5 * D * 4

    def roof(nbytes, ms):
        gbs = nbytes / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_call": nbytes, "mean_ms": round(ms, 4)}

    return {"rows": M, "D": D, "dtype": DTYPE_NAME[str(dt)],
            "fwd_bwd_ms": round(fused_ms, 4), "eager_torch_fwd_bwd_ms": round(eager_ms, 4),
            "speedup_vs_eager": round(eager_ms / fused_ms, 3),
            "timing": "HIP events over back-to-back autograd fwd+bwd (GEMMs included), mean of "
                      "--kernel-reps, queue pre-filled by a spin kernel so host dispatch is hidden",
            "host_bound_ms": {"sparton": round(fused_host, 4), "eager_torch": round(eager_host, 4)},
            "enqueue_ms_per_step": {"sparton": round(fused_enq / reps_n, 4),
                                    "eager_torch": round(eager_enq / reps_n, 4)},
            "epilogue_fwd": roof(fwd_bytes, fwd_epi_ms),
            "epilogue_bwd": roof(bwd_bytes, bwd_epi_ms)}


def autocast_timing(torch, w, inp, dev, reps_n):
    """The head's training fwd+bwd as mixed-precision training runs it (training/train.py under
    bf16/fp16 autocast): fp32 master W and bias, fp32 hidden states, compute in the workload's
    dtype. SpartonHead's autocast path (fp32 gradients straight from the kernels) against the
    plain one (cast the parameters, run the 16-bit training op, autograd casts the gradients
    back to fp32), both through autograd on the same data."""
    import torch.nn.functional as F
    import sparton_amd
    dt = w.dtype
    if dt not in (torch.bfloat16, torch.float16):
        return None
    head = sparton_amd.SpartonHead(w.V, w.D, use_bias=inp.bias is not None).to(dev)
    with torch.no_grad():
        head.weight.copy_(inp.weight.float())
        if inp.bias is not None:
            head.bias.copy_(inp.bias.float())
    h = inp.hidden.float().requires_grad_()
    g = inp.grad  # the workload's upstream gradient, as in the timed steps
    params = [p for p in head.parameters()]

    def fused():
        for t in [h] + params:
            t.grad = None
        with torch.autocast("cuda", dtype=dt):
            out = head(h, inp.mask)
        out.backward(g)

    def plain():
        for t in [h] + params:
            t.grad = None
        b = head.bias.to(dt) if head.bias is not None else None
        out = torch.ops.sparton.fused_sparton_fwd_train(h.to(dt), head.weight.to(dt), b, inp.mask)[0]
        out.backward(g)

    fused_ms, _, _ = time_device(torch, fused, reps_n)
    plain_ms, _, _ = time_device(torch, plain, reps_n)
    return {"dtype": DTYPE_NAME[str(dt)], "params": "fp32", "hidden": "fp32",
            "fwd_bwd_ms": round(fused_ms, 4), "cast_grads_fwd_bwd_ms": round(plain_ms, 4),
            "speedup": round(plain_ms / fused_ms, 3),
            "timing": "HIP events over back-to-back autograd fwd+bwd, queue pre-filled by a spin "
                      "kernel so host dispatch is hidden"}


def loss_timing(torch, w, dev, reps_n):
    """The SPLADE loss on this workload's reps shape (training/train.py:73-197): B query and
    B document reps [B, V] in the reps dtype, train.py's default weights. sparton_amd.loss
    against the same formulas in eager torch, both fwd+bwd through autograd, and the two HIP
    passes alone against the bytes they must move (q and d read; q and d read, dq and dd
    written)."""
    import torch.nn.functional as F
    from sparton_amd import _lib
    from sparton_amd import loss as sl
    B, V, dt = w.B, w.V, w.dtype
    gen = torch.Generator(device=dev).manual_seed(11)

    def reps():
        x = torch.randn(B, V, device=dev, generator=gen) - 1.0
        return torch.log1p(torch.relu(x)).to(dt).requires_grad_()

    q, d = reps(), reps()
    T, w_l1, w_fl = 1.0, 1e-4, 1e-4

    def fused():
        q.grad = d.grad = None
        sl.splade_loss(q, d, T, w_l1, w_fl).total.backward()

    def eager():
        q.grad = d.grad = None
        s = torch.matmul(q, d.t()) / T
        ce = F.cross_entropy(s, torch.arange(B, device=dev))
        reg = (w_l1 * (q.abs().sum(-1).mean() + d.abs().sum(-1).mean())
               + w_fl * ((q.sum(0) ** 2).mean() + (d.sum(0) ** 2).mean()))
        (ce + reg).backward()

    fused_ms, fused_host, _ = time_device(torch, fused, reps_n)
    eager_ms, eager_host, _ = time_device(torch, eager, reps_n)

    L = _lib.load()
    code, stream = _lib.DTYPE_CODE[dt], torch.cuda.current_stream().cuda_stream
    out = torch.empty(6, dtype=torch.float32, device=dev)
    probs = torch.empty(B, B, dtype=torch.float32, device=dev)
    g = torch.ones(6, dtype=torch.float32, device=dev)
    gq, gd = torch.empty_like(q), torch.empty_like(d)
    nbytes = int(L.sparton_loss_workspace_bytes(B, B, V))
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)

    def fwd():
        _lib.check(L.sparton_loss_fwd(q.data_ptr(), d.data_ptr(), B, B, V, T, 1.0, w_l1, w_fl,
                                      out.data_ptr(), probs.data_ptr(), ws.data_ptr(), nbytes,
                                      code, stream), "sparton_loss_fwd")

    def bwd():
        _lib.check(L.sparton_loss_bwd(q.data_ptr(), d.data_ptr(), probs.data_ptr(), g.data_ptr(),
                                      B, B, V, 1.0, w_l1, w_fl, gq.data_ptr(), gd.data_ptr(), code,
                                      stream), "sparton_loss_bwd")

    fwd_ms = time_events(torch, fwd, reps_n)
    bwd_ms = time_events(torch, bwd, reps_n)
    e = q.element_size()

    def roof(nbytes_, ms):
        gbs = nbytes_ / (ms * 1e-3) / 1e9
        return {"bound": "hbm", "achieved": round(gbs, 1), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                "frac": round(gbs / PEAK_HBM_GBS, 4), "bytes_per_call": nbytes_, "mean_ms": round(ms, 4)}

    return {"Bq": B, "Bd": B, "V": V, "dtype": DTYPE_NAME[str(dt)],
            "fwd_bwd_ms": round(fused_ms, 4), "eager_torch_fwd_bwd_ms": round(eager_ms, 4),
            "speedup_vs_eager": round(eager_ms / fused_ms, 3),
            "timing": "HIP events over back-to-back autograd fwd+bwd, queue pre-filled by a spin "
                      "kernel so host dispatch is hidden",
            "host_bound_ms": {"sparton": round(fused_host, 4), "eager_torch": round(eager_host, 4)},
            "fwd_passes": roof(2 * B * V * e, fwd_ms), "bwd_pass": roof(4 * B * V * e, bwd_ms)}


def main():
    args = parse()
    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print("bench.py: this build measures the SpartonHead path on exactly one GPU; "
              f"--gpus {args.gpus} (WORLD_SIZE={world}) is not supported. "
              "Sharding over GPUs is designed but not built in this library.", file=sys.stderr)
        sys.exit(2)

    import torch

    import sparton
    from sparton_amd.workloads import WORKLOADS, make_inputs

    torch.set_float32_matmul_precision(args.fp32_precision)

    assert torch.cuda.is_available(), "bench.py needs a ROCm device"
    dev = torch.device("cuda:0")
    w = WORKLOADS[args.config]
    dname = DTYPE_NAME[str(w.dtype)]
    inp_cpu = make_inputs(w)
    inp = inp_cpu.to(dev)
    has_bias = inp.bias is not None

    head = sparton.SpartonHead(w.V, w.D, use_bias=has_bias).to(dev).to(w.dtype)
    with torch.no_grad():
        head.weight.copy_(inp.weight)
        if has_bias:
            head.bias.copy_(inp.bias)
    H = inp.hidden.clone().requires_grad_()
    mask, G = inp.mask, inp.grad
    params = [p for p in head.parameters()]
    torch.cuda.synchronize()
    input_bytes = torch.cuda.memory_allocated()

    def step():
        H.grad = None
        for p in params:
            p.grad = None
        reps = head(H, mask)
        reps.backward(G)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    torch.cuda.reset_peak_memory_stats()

    # ---- timed region: exactly K steps --------------------------------------------
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    peak_bytes = torch.cuda.max_memory_allocated()

    # In-step op times, from a separate pass: events bracket the forward and the backward
    # of each step, recorded on torch's current stream (the stream the kernels run on).
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(args.steps)]

    def evented_step(e):
        H.grad = None
        for p in params:
            p.grad = None
        e[0].record()
        reps = head(H, mask)
        e[1].record()
        reps.backward(G)
        e[2].record()

    for i in range(args.steps):
        evented_step(ev[i])
    torch.cuda.synchronize()
    fwd_live = statistics.mean(e[0].elapsed_time(e[1]) for e in ev)
    bwd_live = statistics.mean(e[1].elapsed_time(e[2]) for e in ev)
    ms_per_step = elapsed * 1e3 / args.steps
    tokens = w.B * w.S
    value = tokens / (elapsed / args.steps)

    # ---- per-op timing outside the step (HIP events, back-to-back launches) ----------
    Hd, Wd, bd = H.detach(), head.weight.detach(), (head.bias.detach() if has_bias else None)
    fwd_b2b = time_events(torch, lambda: torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, mask),
                          args.kernel_reps)
    enc_ms = time_events(torch, lambda: torch.ops.sparton.fused_sparton_encode(Hd, Wd, bd, mask), args.kernel_reps)
    _, idx, reps = torch.ops.sparton.fused_sparton_fwd_train(Hd, Wd, bd, mask)
    bwd_b2b = time_events(torch, lambda: torch.ops.sparton.fused_sparton_bwd_train(G, reps, idx, Hd, Wd, bd, mask),
                          args.kernel_reps)
    fwd_ms, bwd_ms = fwd_live, bwd_live
    # host cost of a step: the queue is held by a spin kernel while the steps are enqueued
    step_dev_ms, step_host_ms, step_enq_ms = time_device(torch, step, args.kernel_reps)
    main_ms = time_main_kernel(torch, Hd.contiguous(), Wd.contiguous(), bd, mask, args.kernel_reps)
    # fp32 products as bf16 hi/lo parts (torch 'high'/'medium'): small batches only
    split = dname == "fp32" and args.fp32_precision != "highest" and small_path(w, dname)
    main_ms_exact = None
    if split:
        torch.set_float32_matmul_precision("highest")
        main_ms_exact = time_main_kernel(torch, Hd.contiguous(), Wd.contiguous(), bd, mask,
                                         args.kernel_reps)
        torch.set_float32_matmul_precision(args.fp32_precision)
    xf = transform_timing(torch, w, dev, args.kernel_reps)
    lossr = loss_timing(torch, w, dev, args.kernel_reps)
    mixed = autocast_timing(torch, w, inp, dev, args.kernel_reps)
    if args.copy_probe_mib > 0:
        src = torch.empty(args.copy_probe_mib << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        del src, dst

    # forward roofline: useful flops on valid positions (masked positions are skipped)
    valid_tokens = int(inp_cpu.mask.ne(0).sum())
    useful_flops = 2.0 * w.D * w.V * valid_tokens
    dense_flops = 2.0 * w.B * w.S * w.D * w.V
    fwd_tflops = useful_flops / (main_ms * 1e-3) / 1e12
    peak_tf = PEAK_TFLOPS[dname]

    # backward roofline: compulsory bytes (each needed byte moved once)
    e = torch.tensor([], dtype=w.dtype).element_size()
    r = reps.float()
    gp = torch.where(r > 0, G.float() * torch.exp(-r), torch.zeros_like(r))
    gp = gp * mask.gather(1, idx.long()).float()
    act = gp != 0
    nnz = int(act.sum())
    u_w = int(act.any(0).sum())
    rows = (torch.arange(w.B, device=dev).view(-1, 1) * w.S + idx.long())[act]
    u_h = int(torch.unique(rows).numel())
    # G (e bytes) + fp32 reps + int32 idx per (b,v), the gathered H and W rows, and the
    # dense gradients dH, dW, dbias written once in the parameters' dtype (e bytes)
    bwd_bytes = (w.B * w.V * (e + 4 + 4) + u_w * w.D * e + u_h * w.D * e
                 + w.B * w.S * w.D * e + w.V * w.D * e + (w.V * e if has_bias else 0))
    bwd_gbs = bwd_bytes / (bwd_ms * 1e-3) / 1e9
    kname = fwd_kernel_name(w, dname, split)
    # The forward kernel's bound: useful flops at the MFMA peak (three bf16 MFMAs per fp32
    # product in split mode) against its compulsory bytes at the HBM peak: H, W, bias and the
    # mask read once; reps, int32 argmax and fp32 reps written once.
    mask_e = mask.element_size()
    fwd_bytes = (w.B * w.S * w.D * e + w.V * w.D * e + (w.V * e if has_bias else 0)
                 + w.B * w.S * mask_e + w.B * w.V * (e + 4 + 4))
    mfma_peak = PEAK_TFLOPS["bf16"] / 3.0 if split else peak_tf
    t_mfma = useful_flops / (mfma_peak * 1e12)
    t_hbm = fwd_bytes / (PEAK_HBM_GBS * 1e9)
    fwd_bound = "mfma" if t_mfma >= t_hbm else "hbm"
    traffic, traffic_src = measured_traffic(args.config, kname)
    ceiling = mfma_ceiling(torch, dname)
    libgemm = library_gemm(torch, w, mask, args.kernel_reps)
    # whole-step roofline: the forward at the MFMA peak plus the backward's
    # compulsory bytes at HBM peak, over the measured step; useful flops only
    t_step = elapsed / args.steps
    t_roof = max(t_mfma, t_hbm) + bwd_bytes / (PEAK_HBM_GBS * 1e9)
    step_flops = useful_flops + 4.0 * nnz * w.D

    out = {
        "metric": METRIC,
        "value": round(value, 1),
        "unit": "tokens/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": dname,
        "data": "synthetic (seeded; BASELINE.json distributions), random-init head weights",
        "config": {"workload": f"{w.name} SpartonHead fwd+bwd", "B": w.B, "S": w.S, "D": w.D, "V": w.V,
                   "global_batch": w.B, "seq_len": w.S, "use_bias": has_bias,
                   "valid_tokens": valid_tokens, "parallelism": "none (1 GPU)",
                   **({"fp32_matmul_precision": args.fp32_precision,
                       "fp32_products": ("bf16 hi*hi + hi*lo + lo*hi, fp32 accumulation (within 3*2^-16 "
                                         "relative per product)" if split else "fp32 MFMA"),
                       "main_ms_fp32_highest": (round(main_ms_exact, 4) if main_ms_exact else None)}
                      if dname == "fp32" else {})},
        "roofline": {**({"bound": "mfma", "achieved": round(fwd_tflops, 2), "peak": round(mfma_peak, 1),
                          "unit": "TFLOP/s", "frac": round(fwd_tflops / mfma_peak, 4)}
                         if fwd_bound == "mfma" else
                         {"bound": "hbm", "achieved": round(fwd_bytes / (main_ms * 1e-3) / 1e9, 1),
                          "peak": PEAK_HBM_GBS, "unit": "GB/s",
                          "frac": round(fwd_bytes / (main_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}),
                     "kernel": kname, "bytes_per_launch": fwd_bytes,
                     "mfma_bound_ms": round(t_mfma * 1e3, 4), "hbm_bound_ms": round(t_hbm * 1e3, 4),
                     "tflops": round(fwd_tflops, 2),
                     "traffic": traffic, "traffic_source": traffic_src, "flops_per_launch": useful_flops,
                     "flops_basis": "useful: 2*D*V*valid_tokens (fully masked 32-row blocks are skipped)",
                     "dense_equiv_tflops": round(dense_flops / (main_ms * 1e-3) / 1e12, 2),
                     "mean_ms": round(main_ms, 4),
                     "timing": "HIP events recorded on the launch stream around the main kernel "
                               "(sparton_fwd_profile), mean of --kernel-reps launches",
                     "op_ms": round(fwd_ms, 4), "op_timing": "HIP events around the forward of each step of an untimed pass after the timed one",
                     "op_tflops": round(useful_flops / (fwd_ms * 1e-3) / 1e12, 2),
                     "op_ms_back_to_back": round(fwd_b2b, 4),
                     "frac_of_mfma_ceiling": (round(fwd_tflops / ceiling["tflops"], 4)
                                              if ceiling and not split and dname != "fp32" else None)},
        "step_roofline": {"frac": round(t_roof / t_step, 4), "roofline_ms": round(t_roof * 1e3, 4),
                          "step_ms": round(t_step * 1e3, 4),
                          "basis": "(useful F_fwd / MFMA peak + compulsory bwd bytes / 8 TB/s) / measured step"},
        "step_tflops": round(step_flops / t_step / 1e12, 2),
        "step_tflops_basis": "(2*D*V*valid_tokens + 4*nnz*D) / measured step",
        "mfma_ceiling": ceiling,
        "library_gemm": libgemm,
        "bwd_roofline": {"bound": "hbm", "achieved": round(bwd_gbs, 1), "peak": PEAK_HBM_GBS,
                         "unit": "GB/s", "frac": round(bwd_gbs / PEAK_HBM_GBS, 4),
                         "bytes_per_call": bwd_bytes, "nnz": nnz, "U_W": u_w, "U_H": u_h,
                         "mean_ms": round(bwd_ms, 4), "mean_ms_back_to_back": round(bwd_b2b, 4)},
        "host": {"enqueue_ms_per_step": round(step_enq_ms / args.kernel_reps, 4),
                 "device_ms_per_step": round(step_dev_ms, 4),
                 "enqueue_over_device": round(step_enq_ms / args.kernel_reps / step_dev_ms, 3),
                 "timing": "the step's fwd+bwd enqueued back to back while a spin kernel holds the "
                           "queue (host time per step), and the same steps' device time; "
                           "second of two held passes"},
        "fwd_ms": round(fwd_ms, 4),
        "encode_ms": round(enc_ms, 4),
        "bwd_ms": round(bwd_ms, 4),
        "fwd_tokens_per_s": round(tokens / (fwd_ms * 1e-3), 1),
        "encode_tokens_per_s": round(tokens / (enc_ms * 1e-3), 1),
        "peak_gb": round(peak_bytes / 1e9, 4),
        "peak_extra_gb": round((peak_bytes - input_bytes) / 1e9, 4),
        "bsv_logits_gb_avoided": round(w.B * w.S * w.V * e / 1e9, 3),
        "transform": xf,
        "loss": lossr,
        "autocast_fp32_params": mixed,
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline and int(os.environ.get("RANK", "0")) == 0:
        out["cpu_baseline"] = cpu_baseline(torch, w, inp_cpu, args.cpu_seconds)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
