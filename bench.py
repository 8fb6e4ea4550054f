"""Benchmark of the FlashAttention hot path on one MI355X.

Workload (benchmark config C3, configs[2] of the benchmark definition, the
headline): B=4, S=4096, H=32, D=128,
bf16, causal, dropout 0; q, k, v, dO ~ N(0, 1) from torch.Generator('cpu')
seed 42.  One step = forward + backward through the C ABI (fa_fwd, fa_bwd)
with inputs resident in HBM.  Algorithmic FLOPs: F_fwd = 4*B*H*S*S*D/2,
F_fwd+bwd = 3.5 * F_fwd.

Prints ONE JSON line: value = fwd+bwd TFLOP/s; forward-only TFLOP/s, % of the
dense bf16 MFMA peak, per-kernel times (HIP events on the launch stream), the
roofline of the dominant kernel and the CPU baseline (the reference's PyTorch
math path restated in oracle/, fp32 on this host, on a bounded sample of the
same workload) ride along.

With ``--bias full`` (a (B, H, S, S) bf16 additive bias) or ``--bias heads``
(a (1, H, S, S) one, shared over the batch) the same step runs the bias path of
the kernels; ``--dbias`` also produces the bias gradient in the bias dtype (dS
from the dK/dV kernel, accumulated in fp32; for ``heads`` its sum over the batch,
done by the library), inside the timed step.
The FLOP count is the same (the bias adds no matrix products).

With ``--all-configs`` it instead prints one JSON line per benchmark config
(C1-C5: GPU time and TFLOP/s of the config's pass, and the same CPU baseline on
a bounded sample of that config); the dropout configs run the autograd
default, the forward storing the keep bits that the backward reads.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu-baseline]
                    [--bias {none,full,heads}] [--dbias] [--all-configs [--config NAME ...]]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(REPO, "flash-attn-v100_amd"))
sys.path.insert(0, REPO)

PEAK_BF16_TFLOPS = 2516.6  # MI355X dense bf16 MFMA (AMD published)
PEAK_FP32_TFLOPS = 157.3   # MI355X dense fp32 MFMA
PEAK_HBM_GBS = 8000.0
METRIC = "attention TFLOP/s fwd & fwd+bwd, bf16 S=4096 D=128 causal; % of MFMA peak"
B, S, H, D = 4, 4096, 32, 128
CAUSAL = True


def _sig4(x: float) -> float:
    """Four significant digits (a fixed number of decimals rounds a small CPU sample to 0)."""
    return float(f"{x:.4g}")


def f_fwd(b=B, h=H, s=S, d=D, causal=CAUSAL):
    return 4.0 * b * h * s * s * d * (0.5 if causal else 1.0)


BIAS_SHAPES = {"full": (B, H, S, S), "heads": (1, H, S, S)}


def gpu_bench(steps: int, warmup: int, bias_kind: str = "none", want_dbias: bool = False):
    import ctypes

    import torch

    from flash_attention_v100 import _lib

    lib = _lib.load()
    g = torch.Generator("cpu").manual_seed(42)
    q, k, v, do = (torch.randn(B, S, H, D, generator=g, dtype=torch.float32).to(torch.bfloat16).cuda()
                   for _ in range(4))
    scale = D ** -0.5
    o = torch.empty_like(q)
    lse = torch.empty(B, H, S, device="cuda", dtype=torch.float32)
    dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
    pb = dbias = None
    if bias_kind != "none":
        bias = torch.randn(BIAS_SHAPES[bias_kind], device="cuda", dtype=torch.float32).to(torch.bfloat16)
        pb = _lib.prepare_bias(bias, B, H, S, S, torch.bfloat16)
        if want_dbias:  # bias dtype; (1, H, S, S) for the shared bias: the library sums over the batch
            dbias = torch.empty(BIAS_SHAPES[bias_kind], device="cuda", dtype=torch.bfloat16)
    fa = _lib.fwd_args(q, k, v, o, lse, None, CAUSAL, scale, 0.0, 0, 0, pb)
    ba = _lib.bwd_args(q, k, v, o, do, lse, dq, dk, dv, CAUSAL, scale, 0.0, 0, 0, pb, dbias)
    ws_bytes = lib.fa_bwd_workspace_size(ctypes.byref(ba))
    ws = torch.empty(ws_bytes, device="cuda", dtype=torch.uint8)
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)
    wsp = ctypes.c_void_p(ws.data_ptr())

    def fwd():
        st = lib.fa_fwd(ctypes.byref(fa), sp)
        if st:
            raise RuntimeError(_lib.strerror(st))

    def bwd_stage(s):
        st = lib.fa_bwd_stage(ctypes.byref(ba), wsp, ws_bytes, s, sp)
        if st:
            raise RuntimeError(_lib.strerror(st))

    def step():
        fwd()
        bwd_stage(-1)

    for _ in range(warmup):
        step()
    torch.cuda.synchronize()

    # ---- timed region: exactly `steps` fwd+bwd steps ----
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        step()
    torch.cuda.synchronize()
    t_step = (time.perf_counter() - t0) / steps

    # ---- per-kernel averages with HIP events on the launch stream ----
    def timed(fn, n):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / n  # ms

    # the stages fa_bwd runs (include/fa_abi.h): with dQ read from the stored
    # dS, the delta pre-pass (0), dK/dV (1), dQ (2); otherwise the dQ pass that
    # also writes the delta rows (3), then dK/dV (1)
    stages = (0, 1, 2) if (bias_kind != "none" and want_dbias) else (3, 1)
    n = max(steps, 10)
    fwd_ms = timed(fwd, n)
    stage_ms = {s: timed(lambda s=s: bwd_stage(s), n) for s in stages}
    fwd_bwd_ms = timed(step, n)
    ok = bool(torch.isfinite(o).all() and torch.isfinite(dq).all() and torch.isfinite(dk).all()
              and torch.isfinite(dv).all())
    return dict(t_step=t_step, fwd_ms=fwd_ms, stage_ms=stage_ms,
                fwd_bwd_ms=fwd_bwd_ms, finite=ok, device=torch.cuda.get_device_name(0))


def cpu_baseline(target_s: float = 12.0, bias_kind: str = "none"):
    """The reference's math path (oracle.attention, fp32, autograd backward) on
    this host's cores, on B=1 and as many heads of the workload as fit about
    ``target_s`` seconds; reported with the same algorithmic FLOP count."""
    import torch

    from oracle import attention as oa

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator("cpu").manual_seed(42)

    def run(h):
        q, k, v, do = (torch.randn(1, S, h, D, generator=g, dtype=torch.float32) for _ in range(4))
        bias = None if bias_kind == "none" else torch.randn(1, h, S, S, generator=g, dtype=torch.float32)
        t0 = time.perf_counter()
        oa.attention_autograd(q, k, v, do, CAUSAL, D ** -0.5, dtype=torch.float32, bias=bias)
        return time.perf_counter() - t0

    run(1)  # warm-up
    t1 = run(1)
    h = int(max(1, min(H, target_s / max(t1, 1e-3))))
    times = [run(h) for _ in range(2)]
    t = min(times)
    flop = 3.5 * f_fwd(b=1, h=h)
    return {"value": _sig4(flop / t / 1e12), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port",
            "sample": f"fwd+bwd of B=1, H={h} of the workload (S=4096, D=128, causal"
                      f"{'' if bias_kind == 'none' else ', additive bias with its gradient'}) in fp32 via "
                      f"oracle.attention_autograd; best of 2 runs, {t:.2f} s each",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count()}


# benchmark configs C1-C5: name, (B, S, H, D), dtype, causal, dropout p, with backward
ALL_CONFIGS = [
    ("C1", (2, 1024, 12, 64), "float16", False, 0.0, False),
    ("C2", (2, 1024, 12, 64), "float16", True, 0.0, True),
    ("C3", (4, 4096, 32, 128), "bfloat16", True, 0.0, True),
    ("C4-causal", (1, 16384, 16, 128), "bfloat16", True, 0.0, True),
    ("C4-full", (1, 16384, 16, 128), "bfloat16", False, 0.0, True),
] + [(f"C5-D{d}-{'fp32' if dt == 'float32' else 'fp16'}", (8, 1000, 16, d), dt, True, 0.1, True)
     for d in (32, 64, 128) for dt in ("float32", "float16")] + [
    # not a BASELINE config: head dim 256 (16-bit inputs, no bias) at a full-size shape
    ("X-D256", (2, 4096, 16, 256), "bfloat16", True, 0.0, True),
]


def all_configs(n: int, cpu: bool, cpu_target_s: float = 3.0, only=None, warmup: int = 5):
    """One JSON line per benchmark config: GPU time of its pass (HIP events,
    mean of ``n`` calls after at least ``warmup`` untimed ones and 0.2 s of
    work, so that the clock has left the idle state the CPU sample of the
    previous config put it in) and,
    unless ``cpu`` is False, the fp32 math path of oracle/ on this host for B=1
    and as many heads as fit ``cpu_target_s``."""
    import ctypes

    import torch

    from flash_attention_v100 import _lib

    lib = _lib.load()
    stream = torch.cuda.current_stream()
    sp = ctypes.c_void_p(stream.cuda_stream)

    def timed(fn):
        # warm-up: at least `warmup` calls and 0.2 s of back-to-back work (the
        # clock ramps up over tens of milliseconds of load)
        t_end = time.perf_counter() + 0.2
        k = 0
        while k < max(1, warmup) or time.perf_counter() < t_end:
            fn()
            k += 1
            if k % 8 == 0:
                torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(n):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / n  # ms

    for name, (b, s, h, d), dts, causal, p, with_bwd in ALL_CONFIGS:
        if only and name not in only:
            continue
        dt = getattr(torch, dts)
        g = torch.Generator("cpu").manual_seed(42)
        q, k, v, do = (torch.randn(b, s, h, d, generator=g) for _ in range(4))
        if name.startswith("C4"):  # q, k ~ N(0, 2^2): the outlier-heavy long-sequence case
            q, k = 2.0 * q, 2.0 * k
        q, k, v, do = (t.to(dt).cuda() for t in (q, k, v, do))
        o = torch.empty_like(q)
        lse = torch.empty(b, h, s, device="cuda")
        dq, dk, dv = torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)
        bits = _lib.alloc_keep_bits(b, h, s, s, q.device) if p > 0 else None
        fa = _lib.fwd_args(q, k, v, o, lse, None, causal, d ** -0.5, p, 42, 0, None, bits)
        ba = _lib.bwd_args(q, k, v, o, do, lse, dq, dk, dv, causal, d ** -0.5, p, 42, 0, None, None, bits)
        ws = torch.empty(max(256, lib.fa_bwd_workspace_size(ctypes.byref(ba))), device="cuda", dtype=torch.uint8)

        def fwd():
            st = lib.fa_fwd(ctypes.byref(fa), sp)
            if st:
                raise RuntimeError(_lib.strerror(st))

        def bwd():
            st = lib.fa_bwd(ctypes.byref(ba), ctypes.c_void_p(ws.data_ptr()), ws.numel(), sp)
            if st:
                raise RuntimeError(_lib.strerror(st))

        fwd_ms = timed(fwd)
        bwd_ms = timed(bwd) if with_bwd else None
        F = f_fwd(b, h, s, d, causal)
        flop = 3.5 * F if with_bwd else F
        ms = fwd_ms + (bwd_ms or 0.0)
        tf = flop / (ms * 1e-3) / 1e12
        peak = PEAK_FP32_TFLOPS if dt == torch.float32 else PEAK_BF16_TFLOPS
        out = {"config": name, "shape_bshd": [b, s, h, d], "dtype": dts, "causal": causal, "dropout_p": p,
               "pass": "fwd+bwd" if with_bwd else "fwd", "fwd_ms": round(fwd_ms, 4),
               "bwd_ms": None if bwd_ms is None else round(bwd_ms, 4), "tflops": round(tf, 2),
               "pct_peak": round(100 * tf / peak, 2), "peak_tflops": peak,
               "dropout_mask": "keep bits (forward writes, backward reads)" if p > 0 else None}
        if cpu:
            out["cpu_baseline"] = _cpu_sample(s, h, d, causal, p, with_bwd, cpu_target_s)
        print(json.dumps(out), flush=True)
        del q, k, v, do, o, lse, dq, dk, dv, bits, ws
        torch.cuda.empty_cache()


def _cpu_sample(s, h_max, d, causal, p, with_bwd, target_s):
    """fp32 math path (oracle.attention) for B=1 and as many heads as fit
    about ``target_s`` seconds; dropout applies a torch.rand mask (the CPU
    path's cost, not the kernels' Philox stream)."""
    import torch

    from oracle import attention as oa

    cores = len(os.sched_getaffinity(0))
    torch.set_num_threads(cores)
    g = torch.Generator("cpu").manual_seed(42)

    def run(h):
        q, k, v, do = (torch.randn(1, s, h, d, generator=g) for _ in range(4))
        keep = (torch.rand(1, h, s, s, generator=g) > p) if p > 0 else None
        t0 = time.perf_counter()
        if with_bwd:
            oa.attention_autograd(q, k, v, do, causal, d ** -0.5, keep, p, dtype=torch.float32)
        else:
            oa.attention_forward(q, k, v, causal, d ** -0.5, keep, p, torch.float32)
        return time.perf_counter() - t0

    run(1)
    t1 = run(1)
    h = int(max(1, min(h_max, target_s / max(t1, 1e-3))))
    t = min(run(h) for _ in range(2))
    flop = f_fwd(1, h, s, d, causal) * (3.5 if with_bwd else 1.0)
    return {"value": _sig4(flop / t / 1e12), "unit": "TFLOP/s", "cores": torch.get_num_threads(),
            "kind": "port", "sample": f"B=1, H={h} in fp32 via oracle.attention; best of 2 runs, {t:.2f} s each"}


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ln.startswith("model name"):
                    return ln.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def _profiled_traffic(kernel: str, profile: str):
    """HBM bytes per launch of ``kernel`` (read + write) from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE summary ``profiles/<profile>`` of this
    workload, already scaled by the copy calibration; None if the kernel (or
    the workload) was not profiled."""
    path = os.path.join(REPO, "profiles", profile)
    try:
        with open(path) as f:
            k = json.load(f)["kernels"].get(kernel)
    except (OSError, ValueError):
        return None
    return None if k is None else int(k["hbm_read_bytes"] + k["hbm_write_bytes"])


def copy_calibration(gib: float = 1.0, reps: int = 5):
    """A plain device copy of known size, for scaling rocprofv3's FETCH_SIZE /
    WRITE_SIZE counters (KiB per dispatch) to bytes."""
    import torch

    n = int(gib * (1 << 30)) // 2
    src = torch.ones(n, dtype=torch.bfloat16, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"copy_calibration_bytes_read": n * 2, "copy_calibration_bytes_written": n * 2,
                      "reps": reps}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    # 30 untimed steps bring the clocks to their steady state under this load:
    # after only 5 the first timed steps run slower (C3 on one box: 2.39-2.41 ms
    # per step against 2.347 after 30, the latter equal to the event-timed step)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=30)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--bias", choices=("none", "full", "heads"), default="none",
                    help="run the additive-bias path: full = (B, H, S, S), heads = (1, H, S, S), bf16")
    ap.add_argument("--dbias", action="store_true", help="with --bias: also produce the bias gradient")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run a 1 GiB device copy (counter calibration for rocprofv3 --pmc)")
    ap.add_argument("--all-configs", action="store_true",
                    help="one JSON line per benchmark config (C1-C5) instead of the headline line")
    ap.add_argument("--config", action="append", choices=[c[0] for c in ALL_CONFIGS],
                    help="with --all-configs: only these configs (repeatable)")
    a = ap.parse_args()
    if a.copy_calibration:
        copy_calibration()
        return
    if a.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(the reference's multi-GPU helpers are out of scope)", file=sys.stderr)
        sys.exit(2)

    if a.dbias and a.bias == "none":
        ap.error("--dbias needs --bias")
    if a.all_configs:
        all_configs(max(a.steps, 10), not a.no_cpu_baseline, only=a.config, warmup=a.warmup)
        return
    r = gpu_bench(a.steps, a.warmup, a.bias, a.dbias)
    F = f_fwd()
    Ftot = 3.5 * F
    value = Ftot / r["t_step"] / 1e12
    fwd_tflops = F / (r["fwd_ms"] * 1e-3) / 1e12
    names = {0: "delta_kernel", 1: "dkdv_kernel", 2: "dq_kernel", 3: "dq_kernel"}
    kernels = {"fwd_kernel": r["fwd_ms"]}
    kernels.update({names[st]: ms for st, ms in r["stage_ms"].items()})
    # the kernels each stage launches at this workload (the keys above name the stages)
    stage_kernels = {"fwd_kernel": "fwd_pp_kernel (256-query ping-pong workgroups)",
                     "dkdv_kernel": "dkdv_pp_kernel (256-key ping-pong workgroups)"}
    if 3 in r["stage_ms"]:
        stage_kernels["dq_kernel"] = ("dq_pp_kernel (256-query ping-pong workgroups; computes and writes the "
                                      "delta rows; runs before dK/dV)")
    else:
        stage_kernels["delta_kernel"] = "delta_kernel"
        stage_kernels["dq_kernel"] = "dq_pp_kernel (256-query ping-pong workgroups)"
    if a.bias != "none":
        stage_kernels["fwd_kernel"] = "fwd_kernel (256-query workgroups, bias staged through LDS)"
        stage_kernels["dkdv_kernel"] = "dkdv8_kernel" + (" + dbias_reduce_kernel" if a.bias == "heads" and a.dbias else "")
        stage_kernels["dq_kernel"] = "dq_ds_kernel (dQ = dS K from the stored dS)" if a.dbias else "dq_kernel"

    # algorithmic FLOPs per launch: fwd = QK^T + PV; dkdv = 4 of the 5 backward GEMMs
    # (QK^T recompute, dO V^T, P^T dO, dS^T Q); dq = dS K (its S/dP recompute is extra work)
    algo = {"fwd_kernel": F, "dkdv_kernel": 2.0 * F, "dq_kernel": 0.5 * F}
    dom = max(kernels, key=kernels.get)
    tag = "" if a.bias == "none" else f"_bias_{a.bias}{'_dbias' if a.dbias else ''}"
    traffic = _profiled_traffic(dom, f"c3_bf16_causal{tag}_traffic.json")
    if dom in algo:
        ach = algo[dom] / (kernels[dom] * 1e-3) / 1e12
        roof = {"kernel": dom, "bound": "mfma", "achieved": round(ach, 2), "peak": PEAK_BF16_TFLOPS,
                "unit": "TFLOP/s", "frac": round(ach / PEAK_BF16_TFLOPS, 4), "traffic": traffic,
                "algorithmic_flop_per_launch": algo[dom]}
    else:
        nbytes = 2 * B * S * H * D * 2 + 4 * B * H * S
        ach = nbytes / (kernels[dom] * 1e-3) / 1e9
        roof = {"kernel": dom, "bound": "hbm", "achieved": round(ach, 1), "peak": PEAK_HBM_GBS,
                "unit": "GB/s", "frac": round(ach / PEAK_HBM_GBS, 4), "traffic": traffic}
    out = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": a.steps,
        "warmup": a.warmup,
        "ms_per_step": round(r["t_step"] * 1e3, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "C3: B=4 S=4096 H=32 D=128 bf16 causal, fwd+bwd (BASELINE configs[2])"
                               + ("" if a.bias == "none" else
                                  f", additive bf16 bias {BIAS_SHAPES[a.bias]}"
                                  + (" with its gradient" if a.dbias else "")),
                   "batch": B, "seq_len": S, "heads": H, "head_dim": D, "causal": CAUSAL,
                   "bias": a.bias, "dbias": a.dbias, "parallelism": "single-gpu"},
        "fwd_bwd_tflops": round(value, 2),
        "fwd_bwd_pct_peak": round(100 * value / PEAK_BF16_TFLOPS, 2),
        "fwd_tflops": round(fwd_tflops, 2),
        "fwd_pct_peak": round(100 * fwd_tflops / PEAK_BF16_TFLOPS, 2),
        "kernel_ms": {kk: round(vv, 4) for kk, vv in kernels.items()},
        "stage_kernels": stage_kernels,
        "fwd_bwd_event_ms": round(r["fwd_bwd_ms"], 4),
        "outputs_finite": r["finite"],
        "device": r["device"],
        "roofline": roof,
    }
    if not a.no_cpu_baseline:
        out["cpu_baseline"] = cpu_baseline(bias_kind=a.bias)
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
