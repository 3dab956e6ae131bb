"""Benchmark of the eas hot path on one MI355X.

Headline workload: fp32 elementwise add ``c = a + b``
written as an ``@eas.kernel`` SPMD kernel (``mk.arange`` lanes, masked tail),
N = 2^28 (1 GiB per operand), inputs ~ N(0,1) float32 from seeds 0/1, already
resident in HBM.  A step is one launch over the whole array; W untimed steps,
then exactly K steps between device synchronisations.

Prints ONE JSON line: the driver's fields plus ``roofline`` (achieved HBM GB/s
of the kernel from HIP events on its launch stream, vs 8 TB/s) and
``cpu_baseline``: the reference's own CPU expression for the workload (the NumPy
expressions its tests compute expected values with: ``np.add(a, b, out=c)``,
``a*b+c``, ``A32 @ B32``, ``A16.astype(np.float32) @ B16.astype(np.float32)``)
timed on this host's cores on the same arrays, with the host described.  ``vendor`` times the same operation through torch (ROCm:
``torch.add``, hipBLASLt/rocBLAS ``torch.matmul``, or ``torch.mm(..., out_dtype=torch.float32)``
where the eas kernel writes f32 from 16-bit inputs) on the same device-resident inputs with the
eas kernel's output dtype, in the same run, with the same event method; for a matmul the eas and
vendor event trials alternate.  Each matmul entry under ``extra`` carries its ``torch_matmul``.
Secondary measurements ride along under ``extra``.

``--workload copy|fma|read|write`` measures the other elementwise kernels the same way
(``copy`` is the known-size kernel that calibrates HBM byte counters; ``read`` and
``write`` measure one-direction HBM streaming on the same GPU).

``--workload mma`` makes the f16-input / f32-accumulate simdgroup-MMA matmul at
M=N=K=4096 (configs[3]; lifted to the MFMA GEMM) the primary line, with the
roofline against the f16 dense MFMA peak; ``mma_k4100``, ``mma_bf16`` (bf16
inputs, an addition to the reference's dtypes), ``decode``, ``prefill``,
``tiled1024`` and ``tiled2048`` select the other matmul configurations.  The
default run reports all of them under ``extra``.
"""

from __future__ import annotations

import argparse
import json
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "tests"))

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2516.6  # dense f16 (and bf16) MFMA, MI355X
F32_PEAK_TFLOPS = 157.3  # fp32 dense MFMA (= vector fp32), MI355X
N_ELEM = 1 << 28
PRIMARY_BLOCK = 256

# name -> (kernel attribute in tests/kernels.py, input count, algorithmic bytes per element)
WORKLOADS = {
    "add": ("add_kernel", 2, 12),
    "fma": ("fma_kernel", 3, 16),
    # the reference's own fma kernel, thread mode (tests/test_fma.py:13-23)
    "fma_thread": ("simple_fma_kernel", 3, 16),
    "copy": ("copy_kernel", 1, 8),
    "read": ("read_kernel", 1, 4),
    "write": ("fill_kernel", 0, 4),
}


# matmul configurations: (kernel in tests/kernels.py, M, N, K, A distribution, B distribution, description)
MATMULS = {
    "mma": ("matmul_mma_kernel", 4096, 4096, 4096, "u", "u",
            "f16-in/f32-acc simdgroup-MMA matmul (mk.dot), M=N=K=4096, f32 out"),
    "mma_k4100": ("matmul_mma_kernel", 4096, 4096, 4100, "u", "u",
                  "f16-in/f32-acc simdgroup-MMA matmul (mk.dot), M=N=4096, K=4100, f32 out"),
    "mma_bf16": ("matmul_mma_bf16_kernel", 4096, 4096, 4096, "ubf", "ubf",
                 "bf16-in/f32-acc simdgroup-MMA matmul (mk.dot, bf16 threadgroup tiles), M=N=K=4096, f32 out"),
    "decode": ("matmul_mma_f16out_kernel", 16, 14336, 4096, "act", "w",
               "f16 LLM decode linear M=16 N=14336 K=4096 (mk.dot), f32 acc, f16 out"),
    "prefill": ("matmul_mma_f16out_kernel", 8192, 8192, 8192, "act", "w",
                "f16 LLM prefill linear M=N=K=8192 (mk.dot), f32 acc, f16 out"),
    "tiled1024": ("matmul_tiled_kernel", 1024, 1024, 1024, "n", "n",
                  "fp32 tiled matmul (threadgroup tiles + mk.dot, 32x32 tiles; lifted to fp32 MFMA), M=N=K=1024"),
    "tiled2048": ("matmul_tiled_kernel", 2048, 2048, 2048, "n", "n",
                  "fp32 tiled matmul (threadgroup tiles + mk.dot, 32x32 tiles; lifted to fp32 MFMA), M=N=K=2048"),
}


# rocprofv3 counter summaries (profiles/<name>.pmc.json) that give a matmul line its HBM traffic
MATMUL_PROFILES = {"mma": "mma_f16_4096", "mma_bf16": "mma_bf16_4096", "decode": "decode_f16_16x14336x4096",
                   "prefill": "prefill_f16_8192",
                   "tiled1024": "tiled_f32_1024", "tiled2048": "tiled_f32_2048"}


def _log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def _inputs(n: int, seeds: tuple[int, ...]) -> list[np.ndarray]:
    return [np.random.default_rng(s).standard_normal(n, dtype=np.float32) for s in seeds]


EVENT_TRIALS = 5


SETTLE_BATCH = 10
SETTLE_MAX_LAUNCHES = 400
SETTLE_LOG: list[dict] = []


def _settle_until_stable(batch_seconds, label: str) -> int:
    """Untimed launches until the device's clocks have settled: after any idle gap (0.2 s is
    enough) the GPU runs an HBM-bound launch fast for ~3 launches, then up to ~30 % slower for
    ~20 more while its power management ramps, then steadily.  ``batch_seconds()`` runs
    SETTLE_BATCH launches and returns their event time; batches run until two in a row agree
    within 2 % (at most SETTLE_MAX_LAUNCHES launches).  None of them is part of any
    reported time; the count is logged in the output line."""
    prev, n = None, 0
    while n < SETTLE_MAX_LAUNCHES:
        t = batch_seconds()
        n += SETTLE_BATCH
        if prev is not None and n >= 3 * SETTLE_BATCH and abs(t - prev) <= 0.02 * min(t, prev):
            break
        prev = t
    SETTLE_LOG.append({"kernel": label, "launches": n})
    return n


def _settle(rt, ck, rargs, meta, **launch) -> int:
    label = ck.geometry.entry if ck.geometry is not None else ck.ir.name
    return _settle_until_stable(lambda: rt.benchmark(ck, rargs, meta, repeat=SETTLE_BATCH, warmup=0, **launch),
                                label)


def _time_kernel(rt, ck, rargs, meta, steps: int, warmup: int, torch, **launch) -> tuple[float, float]:
    """(wall ms/step bracketed by device syncs, HIP-event ms/launch on the launch stream: the
    median of EVENT_TRIALS trials of ``steps`` back-to-back launches).  The device is settled
    first (``_settle``), then ``warmup`` untimed steps run, then the ``steps`` timed ones."""
    _settle(rt, ck, rargs, meta, **launch)
    for _ in range(warmup):
        rt.run(ck, rargs, meta, sync=False, **launch)
    rt.synchronize()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        rt.run(ck, rargs, meta, sync=False, **launch)
    rt.synchronize()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    trials = sorted(rt.benchmark(ck, rargs, meta, repeat=steps, warmup=0, **launch) for _ in range(EVENT_TRIALS))
    return wall_ms, trials[EVENT_TRIALS // 2] * 1e3


def _interleaved_event_ms(rt, ck, rargs, meta, fn, steps: int, torch, **launch) -> tuple[float, float]:
    """(eas ms/launch, torch ms/call): EVENT_TRIALS trials of ``steps`` back-to-back launches of
    each, alternating eas and torch trial by trial, medians of each.  The shader clock keeps
    ramping for a while after a burst starts, so timing one side's trials after the other's
    gives the later side a faster clock; alternating gives both the same.  Both are settled
    before (``_time_kernel``, ``_torch_event_ms``)."""
    ours, theirs = [], []
    for _ in range(EVENT_TRIALS):
        ours.append(rt.benchmark(ck, rargs, meta, repeat=steps, warmup=0, **launch) * 1e3)
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            fn()
        t1.record()
        t1.synchronize()
        theirs.append(t0.elapsed_time(t1) / steps)
    return sorted(ours)[EVENT_TRIALS // 2], sorted(theirs)[EVENT_TRIALS // 2]


def _dispatch_probe(rt, workgroups: int, threads: int, trials: int = EVENT_TRIALS) -> float:
    """Workgroups per ns the command processor dispatches on this box: an empty kernel of
    ``workgroups`` workgroups of ``threads`` threads (the add's launch shape), timed with HIP
    events, 20 launches per trial, median of ``trials``.  An elementwise kernel whose
    workgroups arrive at close to this rate is bound by dispatch, not by HBM."""
    from easy_as_amd.runtime.hip import compile_code

    mod = rt._mod()
    src = 'extern "C" __global__ void eas_dispatch_probe() {}\n'
    k = mod.load(compile_code(mod, src, "eas_dispatch_probe"), "eas_dispatch_probe")
    ms = sorted(mod.launch_timed(k, [], [], (workgroups, 1, 1), (threads, 1, 1), repeat=20, warmup=5)
                for _ in range(trials))[trials // 2]
    return workgroups / (ms * 1e6)


def _torch_event_ms(fn, steps: int, warmup: int, torch) -> float:
    """ms per call of a torch operation on torch's current stream: the median of EVENT_TRIALS
    trials of ``steps`` back-to-back calls between torch events (the vendor comparison), after
    the same settling as the eas kernels."""

    def batch() -> float:
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(SETTLE_BATCH):
            fn()
        t1.record()
        t1.synchronize()
        return t0.elapsed_time(t1) * 1e-3

    _settle_until_stable(batch, "torch")
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    trials = []
    for _ in range(EVENT_TRIALS):
        t0, t1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        t0.record()
        for _ in range(steps):
            fn()
        t1.record()
        t1.synchronize()
        trials.append(t0.elapsed_time(t1) / steps)
    return sorted(trials)[EVENT_TRIALS // 2]


# --shape M,N,K: the same kernel and input distributions at another shape (for scaling
# studies such as the K sweep behind a GEMM's time budget; not a metric configuration)
SHAPE_OVERRIDE: dict[str, tuple[int, int, int]] = {}


def _config(name: str) -> tuple:
    """(kernel, M, N, K, A distribution, B distribution, description) of a matmul workload."""
    kname, m, n, k, da, db, desc = MATMULS[name]
    if name in SHAPE_OVERRIDE:
        m, n, k = SHAPE_OVERRIDE[name]
        desc = f"{desc.split(',')[0]}, shape override M={m} N={n} K={k} (not the configuration's shape)"
    return kname, m, n, k, da, db, desc


def _matmul_inputs(name: str, torch) -> tuple[object, object]:
    """Host inputs: NumPy arrays, or torch bfloat16 CPU tensors (NumPy has no bfloat16), from
    the configurations' seeds: A from default_rng(0), B from default_rng(1)."""
    _, m, n, k, da, db, _ = _config(name)
    rng_a, rng_b = np.random.default_rng(0), np.random.default_rng(1)

    def draw(rng, dist, size):
        if dist == "u":
            return rng.uniform(-1, 1, size).astype(np.float16)
        if dist == "ubf":
            return torch.from_numpy(rng.uniform(-1, 1, size).astype(np.float32)).to(torch.bfloat16)
        if dist == "act":
            return rng.standard_normal(size, dtype=np.float32).astype(np.float16)
        if dist == "w":
            return (0.02 * rng.standard_normal(size, dtype=np.float32)).astype(np.float16)
        return (rng.standard_normal(size, dtype=np.float32) / np.float32(np.sqrt(k))).astype(np.float32)

    return draw(rng_a, da, m * k), draw(rng_b, db, k * n)


# --data for matmul workloads: the configs' seeded distributions (the metric), or the same
# shapes on constant data, to show how much of the time goes to the MFMA's data-dependent power
MATMUL_DATA = ("seeded", "zeros", "ones", "signs")


def _matmul(name: str, rt, torch, steps: int, warmup: int, data: str = "seeded", cpu_baseline: bool = False) -> dict:
    """Time one matmul configuration and check a seeded sample of its rows against float64;
    with ``cpu_baseline``, also time the reference's CPU expression on the same operands."""
    import kernels as K

    kname, m, n, k, _, _, desc = _config(name)
    kern = getattr(K, kname)
    dev = torch.device("cuda:0")
    ha, hb = _matmul_inputs(name, torch)
    if data != "seeded":
        # same dtype and shape; zeros, ones, or the signs (+-1) of the seeded values
        def const(x):
            t = x if isinstance(x, torch.Tensor) else torch.from_numpy(x)
            return {"zeros": torch.zeros_like, "ones": torch.ones_like, "signs": torch.sign}[data](t)
        ha, hb = const(ha), const(hb)
    a, b = (x.to(dev) if isinstance(x, torch.Tensor) else torch.from_numpy(x).to(dev) for x in (ha, hb))
    # float64 reference operands: the values the kernel multiplies (bf16 widens exactly)
    ha, hb = (x.float().numpy() if isinstance(x, torch.Tensor) else x for x in (ha, hb))
    tiled = kname == "matmul_tiled_kernel"
    out_dt = torch.float32 if (tiled or kname in ("matmul_mma_kernel", "matmul_mma_bf16_kernel")) else torch.float16
    c = torch.full((m * n,), float("nan"), dtype=out_dt, device=dev)
    if tiled:
        meta = {"BM": 32, "BN": 32, "BK": 32, "K": k, "NT": 256}
        args = (a, b, c, m, n, 0, 0)
        rargs = dict(zip(("a", "b", "c", "M", "N", "PID_M_BASE", "PID_N_BASE"), args))
        grid = (K.cdiv(n, 32), K.cdiv(m, 32), 1)
        tptg = (256, 1, 1)
    else:
        meta = {"BM": 32, "BN": 32, "BK": 8, "K": k, "NT": 512}
        args = (a, b, c, m, n)
        rargs = dict(zip(("a", "b", "c", "M", "N"), args))
        grid = (K.cdiv(n, 32), K.cdiv(m, 32), 1)
        tptg = (512, 1, 1)
    t0 = time.perf_counter()
    ck = kern.compile(*args, **meta)
    compile_s = time.perf_counter() - t0
    wall_ms, ev_ms = _time_kernel(rt, ck, rargs, meta, steps, warmup, torch, grid=grid, tptg=tptg)
    tms = vendor_op = None
    if data == "seeded":
        # vendor comparison on the same device-resident operands, with the eas kernel's output
        # dtype: hipBLASLt/rocBLAS through torch.matmul (fp32, and f16 output), or torch.mm with
        # out_dtype=float32 for 16-bit inputs into an f32 C.  After both are settled, their event
        # trials alternate and both medians come from them.
        A2, B2 = a.view(m, k), b.view(k, n)
        if out_dt == torch.float32 and a.dtype != torch.float32:
            mm = lambda: torch.mm(A2, B2, out_dtype=torch.float32)  # noqa: E731
            vendor_op = "torch.mm(A, B, out_dtype=torch.float32)"
        else:
            out_t = torch.empty((m, n), dtype=a.dtype, device=dev)
            mm = lambda: torch.matmul(A2, B2, out=out_t)  # noqa: E731
            vendor_op = "torch.matmul(A, B, out=C)"
        _torch_event_ms(mm, steps, warmup, torch)
        ev_ms, tms = _interleaved_event_ms(rt, ck, rargs, meta, mm, steps, torch, grid=grid, tptg=tptg)
        del mm
        out_t = None
    flops = 2.0 * m * n * k
    # parity: rows sampled with a fixed seed, float64 reference of the (rounded) inputs
    c.fill_(float("nan"))
    rt.run(ck, rargs, meta, grid=grid, tptg=tptg)
    torch.cuda.synchronize()
    got = c.float().cpu().numpy().reshape(m, n)
    rows = np.sort(np.random.default_rng(7).choice(m, min(m, 32), replace=False))
    ref = ha.reshape(m, k)[rows].astype(np.float64) @ hb.reshape(k, n).astype(np.float64)
    err = _f64_rel_err(got[rows], ref)
    # elementwise: |C - R| / (|R| + max|R| * 1e-3), the worst element of the sampled rows
    diff = np.abs(got[rows].astype(np.float64) - ref)
    elem_err = float(np.max(diff / (np.abs(ref) + 1e-3 * float(np.max(np.abs(ref)) or 1.0))))
    if tiled:
        tol, tol_s = 1e-5 * np.sqrt(k), "1e-5*sqrt(K)"
    elif out_dt == torch.float16:
        tol, tol_s = 2e-2, "2e-2 (f16 output)"
    else:
        tol, tol_s = min(2e-2, 1e-5 * np.sqrt(k)), "min(2e-2, 1e-5*sqrt(K))"
    ok = bool(np.isfinite(got).all() and err <= tol)
    peak = F32_PEAK_TFLOPS if tiled else MFMA_F16_PEAK_TFLOPS
    tf = flops / (ev_ms * 1e-3) / 1e12
    bytes_min = (m * k + k * n) * a.element_size() + m * n * (2 if out_dt == torch.float16 else 4)
    # roofline: HBM-bound below the ridge point (peak flop/s / peak bytes/s), compute-bound above
    hbm_bound = flops / bytes_min < peak * 1e12 / (HBM_PEAK_GBS * 1e9)
    gbs = bytes_min / (ev_ms * 1e-3) / 1e9
    res = {
        "desc": desc, "kernel": ck.geometry.kind if ck.geometry is not None else "thread",
        # the tiled fp32 kernel runs lifted on fp32 MFMA (its literal lowering is VALU)
        "bound": "hbm" if hbm_bound else ("mfma" if ck.geometry is not None and ck.geometry.kind == "gemm" else "valu"),
        "frac_of_bound": round(gbs / HBM_PEAK_GBS if hbm_bound else tf / peak, 4),
        "TFLOP/s": round(tf, 1), "frac": round(tf / peak, 4), "peak_TFLOP/s": peak,
        "wall_TFLOP/s": round(flops / (wall_ms * 1e-3) / 1e12, 1), "ms_per_launch": round(ev_ms, 5),
        "min_hbm_GB/s": round(bytes_min / (ev_ms * 1e-3) / 1e9, 1),
        "parity": f"max rel err {err:.2e} on 32 sampled rows vs float64 (tol {tol_s})" + ("" if ok else " FAIL"),
        "elementwise_err": float(f"{elem_err:.3e}"), "max_abs_err": float(f"{float(diff.max()):.3e}"),
        "parity_ok": ok, "compile_s": round(compile_s, 1),
    }
    _log(f"{name}: {res['TFLOP/s']} TFLOP/s ({100 * res['frac']:.1f}% of {peak}), {ev_ms:.4f} ms/launch, "
         f"parity {res['parity']}, compile {compile_s:.1f} s")
    if tms is not None:
        res["torch_matmul"] = {"op": vendor_op, "TFLOP/s": round(flops / (tms * 1e-3) / 1e12, 1),
                               "ms_per_launch": round(tms, 5), "out_dtype": str(out_dt).replace("torch.", ""),
                               "timing": "event trials alternating with the eas kernel's; each call is issued "
                                         "from Python, so a kernel shorter than the call's host cost "
                                         "(~30 us) reads slow here, where a kernel trace times it exactly"}
        _log(f"{name}: {vendor_op} {res['torch_matmul']['TFLOP/s']} TFLOP/s, {tms:.4f} ms/launch")
    if cpu_baseline and data == "seeded":
        res["cpu_baseline"] = _matmul_cpu_baseline(name, ha, hb, m, n, k)
        _log(f"{name}: cpu baseline {res['cpu_baseline']['value']} TFLOP/s ({res['cpu_baseline']['cores']} threads)")
    del a, b, c
    torch.cuda.empty_cache()
    return res


# --phases: in-kernel timestamps of the 8-wave GEMM entry (the fp32 entries: below).  s_memrealtime counts a constant
# 100 MHz clock; hardware register XCC_ID (id 20, bits 0-3) names the XCD a workgroup runs on.
_PHASE_SLOTS = 8  # per wave group: entry, loop start, loop end, stores issued, stores done, XCD id
_PHASE_STAMP = (
    "#define EAS_STAMP(slot) do { if (threadIdx.x == 0 || threadIdx.x == 256) "
    "__eas_stamps[(blockIdx.x * 2u + (threadIdx.x >> 8)) * 8u + (slot)] = __builtin_amdgcn_s_memrealtime(); "
    "} while (0)\n"
    "#define EAS_STAMP_XCD() do { if (threadIdx.x == 0 || threadIdx.x == 256) "
    "__eas_stamps[(blockIdx.x * 2u + (threadIdx.x >> 8)) * 8u + 5u] = "
    "(unsigned long long)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u); } while (0)\n")


def _stamped_pp_source(src: str, entry: str) -> str:
    """The generated GEMM source with a stamp buffer appended to the 8-wave entry's arguments and
    stamps written (lane 0 of waves 0 and 4) at five points of ``eas_gemm_pp``: entry, start of the
    K loop (prologue DMA landed), end of the K loop, C stores issued, C stores complete.  Raises if
    the source does not have the expected shape (16 x 16 x 32 MFMA body, one 8-wave entry)."""
    src = src.split("\n", 1)[1]  # the eas-launch line describes the unstamped argument list
    body = ("eas_op_t* smem) {\n  constexpr int BM = 256, BN = 256, BK = 32, NSTAGE = 4, KT = (K + BK - 1) / BK;\n"
            "  constexpr int STAGE_H = BM * BK;\n  eas_op_t* As = smem;\n  eas_op_t* Bs = smem + NSTAGE * STAGE_H;\n"
            "  const int tid = threadIdx.x, lane = tid & 63;\n"
            "  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);\n  const int g = wave >> 2, p = wave & 3;\n")
    edits = [
        (body, body.replace("eas_op_t* smem) {", "eas_op_t* smem, unsigned long long* __eas_stamps) {")
         + "  EAS_STAMP(0);\n  EAS_STAMP_XCD();\n"),
        ("    if (g == 1) __syncthreads();\n    for (int kt = 0; kt < KT; ++kt) stage(kt, kt % NSTAGE, b_fast);",
         "    if (g == 1) __syncthreads();\n    EAS_STAMP(1);\n    for (int kt = 0; kt < KT; ++kt) stage(kt, kt % NSTAGE, b_fast);"),
        ("  // the K loop is done: no LDS is read or written below\n",
         "  // the K loop is done: no LDS is read or written below\n  EAS_STAMP(2);\n"),
        ("(CT)acc16[i][j][r];\n        }\n  }\n}\n\n// Guard body",
         "(CT)acc16[i][j][r];\n        }\n  }\n  EAS_STAMP(3);\n  __builtin_amdgcn_s_waitcnt(0);\n"
         "  EAS_STAMP(4);\n}\n\n// Guard body"),
        ("eas_gemm_pp<CT, K, 16>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);",
         "eas_gemm_pp<CT, K, 16>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem, __eas_stamps);"),
    ]
    for old, new in edits:
        if src.count(old) != 1:
            raise RuntimeError(f"--phases: unexpected GEMM source shape at {old[:48]!r}")
        src = src.replace(old, new)
    head = src.index(f"void {entry}(")
    close = src.index(") {", head)
    src = src[:close] + ",\n    unsigned long long* __restrict__ __eas_stamps" + src[close:]
    return _PHASE_STAMP + src


# The fp32 entries: lane 0 of consumer wave 0 of each workgroup stamps slots 0-4 as above and the
# XCD id (slot 5); slots 6 and 7 take s_memtime, which counts shader clocks, at the start and end
# of the K loop, so the loop's clocks per BK = 32 stage come out independent of the clock rate.
_PHASE_STAMP_F32 = (
    "#define EAS_F32_STAMP(slot) do { if (threadIdx.x == 0) "
    "__eas_stamps[blockIdx.x * 8u + (slot)] = __builtin_amdgcn_s_memrealtime(); } while (0)\n"
    "#define EAS_F32_CLOCK(slot) do { if (threadIdx.x == 0) "
    "__eas_stamps[blockIdx.x * 8u + (slot)] = __builtin_amdgcn_s_memtime(); } while (0)\n"
    "#define EAS_F32_XCD() do { if (threadIdx.x == 0) __eas_stamps[blockIdx.x * 8u + 5u] = "
    "(unsigned long long)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u); } while (0)\n")


def _stamped_f32_source(src: str, entry: str) -> str:
    """The generated fp32 GEMM source with a stamp buffer appended to ``entry``'s arguments (either
    fp32 entry) and stamps at: entry, start of the K loop (stage 0 landed), end of the K loop (last
    MFMA issued), C stores issued, C stores complete.  Raises if the entry does not have the
    expected shape."""
    src = src.split("\n", 1)[1]  # the eas-launch line describes the unstamped argument list
    start = src.rindex('extern "C"', 0, src.index(f"void {entry}("))
    nxt = src.find('extern "C"', start + 10)
    end = nxt if nxt >= 0 else len(src)
    body = src[start:end]
    edits = [
        ("  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);\n",
         "  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);\n  EAS_F32_STAMP(0);\n  EAS_F32_XCD();\n"),
        ("  __syncthreads();  // stage 0 landed\n",
         "  __syncthreads();  // stage 0 landed\n  EAS_F32_STAMP(1);\n  EAS_F32_CLOCK(6);\n"),
        ("  } else {\n    mfmas(a0, b0);\n  }\n",
         "  } else {\n    mfmas(a0, b0);\n  }\n  EAS_F32_STAMP(2);\n  EAS_F32_CLOCK(7);\n"),
    ]
    for old, new in edits:
        if body.count(old) != 1:
            raise RuntimeError(f"--phases: unexpected fp32 GEMM source shape at {old[:48]!r}")
        body = body.replace(old, new)
    close = body.index(") {")
    body = body[:close] + ",\n    unsigned long long* __restrict__ __eas_stamps" + body[close:]
    last = body.rindex("}")
    body = body[:last] + "  EAS_F32_STAMP(3);\n  __builtin_amdgcn_s_waitcnt(0);\n  EAS_F32_STAMP(4);\n" + body[last:]
    return _PHASE_STAMP_F32 + src[:start] + body + src[end:]


# The f16 smaller-tile entries (128 x 128, 128 x 256, 64 x 64, 128 x 64): the same stamps as the
# fp32 entries, written by lane 0 of consumer wave 0, inside the body they share; the entries not
# measured pass a null stamp pointer.
_PHASE_STAMP_WS = (
    "#define EAS_WS_STAMP(slot) do { if (__eas_stamps && threadIdx.x == 0) "
    "__eas_stamps[blockIdx.x * 8u + (slot)] = __builtin_amdgcn_s_memrealtime(); } while (0)\n"
    "#define EAS_WS_CLOCK(slot) do { if (__eas_stamps && threadIdx.x == 0) "
    "__eas_stamps[blockIdx.x * 8u + (slot)] = __builtin_amdgcn_s_memtime(); } while (0)\n"
    "#define EAS_WS_XCD() do { if (__eas_stamps && threadIdx.x == 0) __eas_stamps[blockIdx.x * 8u + 5u] = "
    "(unsigned long long)(__builtin_amdgcn_s_getreg((3 << 11) | 20) & 15u); } while (0)\n")


def _stamped_ws_source(src: str, entry: str) -> str:
    """The generated f16 GEMM source with a stamp buffer appended to ``entry``'s arguments (the
    128 x 128, 128 x 256 or 128 x 64 entry) and stamps at: entry, start of the K loop (stage 0 landed),
    end of the K loop (last MFMA issued), C stores issued, C stores complete, plus shader clocks
    around the K loop.  Raises if the source does not have the expected shape."""
    src = src.split("\n", 1)[1]  # the eas-launch line describes the unstamped argument list
    bm, bn = {"__t128x256": (128, 256), "__t128x64": (128, 64), "__t64x64": (64, 64)}.get(
        entry[entry.rindex("__"):], (128, 128))
    from easy_as_amd.codegen.gemm_kernels import pp_mfma

    # the 128 x 128 and 128 x 256 entries take the MFMA shape EAS_HIP_GEMM_MFMA selects; 128 x 64
    # and 64 x 64 fix 16 x 16 x 32
    t64 = "eas_gemm_t128<CT, K, 64, 16, 64>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);"
    call = "eas_gemm_t128<CT, K, {}, {}>((const eas_op_t*)A, (const eas_op_t*)B, C, ldb, M, N, m0, n0, smem);"
    call128, call256, call64 = call.format(128, pp_mfma()), call.format(256, pp_mfma()), call.format(64, 16)
    edits = [
        ("eas_op_t* smem) {\n  static_assert((BN == 64 || BN == 128 || BN == 256)",
         "eas_op_t* smem, unsigned long long* __restrict__ __eas_stamps) {\n"
         "  static_assert((BN == 64 || BN == 128 || BN == 256)"),
        ("(2 * ((r >> 3) & 1));\n  };\n  if (wave >= 4) {",
         "(2 * ((r >> 3) & 1));\n  };\n  EAS_WS_STAMP(0);\n  EAS_WS_XCD();\n  if (wave >= 4) {"),
        ("  __syncthreads();  // stage 0 landed\n  afrag_t a0, a1;\n",
         "  __syncthreads();  // stage 0 landed\n  EAS_WS_STAMP(1);\n  EAS_WS_CLOCK(6);\n  afrag_t a0, a1;\n"),
        ("  } else {\n    mask_tail(a0);\n    mfmas(a0, b0);\n  }\n",
         "  } else {\n    mask_tail(a0);\n    mfmas(a0, b0);\n  }\n  EAS_WS_STAMP(2);\n  EAS_WS_CLOCK(7);\n"),
        ("(CT)acc16[i][j][r];\n        }\n  }\n}\n\n// Skinny path",
         "(CT)acc16[i][j][r];\n        }\n  }\n  EAS_WS_STAMP(3);\n"
         "  __builtin_amdgcn_s_waitcnt(0);\n  EAS_WS_STAMP(4);\n}\n\n// Skinny path"),
        (call128, call128[:-2] + (", __eas_stamps);" if (bm, bn) == (128, 128) else ", nullptr);")),
        (call256, call256[:-2] + (", __eas_stamps);" if bn == 256 else ", nullptr);")),
        (call64, call64[:-2] + (", __eas_stamps);" if bn == 64 and bm == 128 else ", nullptr);")),
        (t64, t64[:-2] + (", __eas_stamps);" if bm == 64 else ", nullptr);")),
    ]
    for old, new in edits:
        if src.count(old) != 1:
            raise RuntimeError(f"--phases: unexpected f16 GEMM source shape at {old[:48]!r}")
        src = src.replace(old, new)
    head = src.index(f"void {entry}(")
    close = src.index(") {", head)
    src = src[:close] + ",\n    unsigned long long* __restrict__ __eas_stamps" + src[close:]
    return _PHASE_STAMP_WS + src


def _gemm_phases(name: str, rt, torch, trials: int = 5, lead: int = 20) -> dict:
    """Per-phase time budget of one launch of the 8-wave GEMM entry, of an f16 smaller-tile entry,
    or of either fp32 entry, on the configuration's seeded inputs: after settling, ``trials`` times
    run ``lead`` launches back to back and one more, and read the last launch's stamps.  Medians
    over the trials of: spread of workgroup starts, prologue, K loop (median, min, max over wave
    groups, median per XCD), C store issue, store completion, median and last end; all in
    microseconds from the first workgroup's start.  The fp32 and smaller-tile entries add the K loop's
    shader clocks per BK = 32 stage and the shader clock they imply."""
    import kernels as K
    from easy_as_amd.runtime.hip import compile_code, plan_launch, struct

    kname, m, n, k, _, _, _ = _config(name)
    dev = torch.device("cuda:0")
    ha, hb = _matmul_inputs(name, torch)
    a, b = (x.to(dev) if isinstance(x, torch.Tensor) else torch.from_numpy(x).to(dev) for x in (ha, hb))
    tiled = kname == "matmul_tiled_kernel"
    out_dt = torch.float32 if kname in ("matmul_mma_kernel", "matmul_mma_bf16_kernel") or tiled else torch.float16
    c = torch.zeros(m * n, dtype=out_dt, device=dev)
    if tiled:
        ck = K.matmul_tiled_kernel.compile(a, b, c, m, n, 0, 0, BM=32, BN=32, BK=32, K=k, NT=256)
        args = {"a": a, "b": b, "c": c, "M": m, "N": n, "PID_M_BASE": 0, "PID_N_BASE": 0}
    else:
        ck = getattr(K, kname).compile(a, b, c, m, n, BM=32, BN=32, BK=8, K=k, NT=512)
        args = {"a": a, "b": b, "c": c, "M": m, "N": n}
    mod = rt._mod()
    plan = plan_launch(ck, args, grid=(K.cdiv(n, 32), K.cdiv(m, 32), 1), compute_units=rt._cus)
    entry = plan.entry or ck.geometry.entry if plan is not None else None
    ws = entry is not None and entry.endswith(("__t128", "__t128x256", "__t128x64", "__t64x64")) and not tiled
    if tiled:
        src, per_wg = _stamped_f32_source(ck.src, entry), 1
    elif ws:
        src, per_wg = _stamped_ws_source(ck.src, entry), 1
    elif entry is None or not entry.endswith("__pp"):
        raise RuntimeError(f"--phases needs the 8-wave GEMM entry; {name} launches {entry}")
    else:
        src, per_wg = _stamped_pp_source(ck.src, entry), 2
    kern = mod.load(compile_code(mod, src, ck.ir.name), entry)
    groups = plan.grid[0] * plan.grid[1] * plan.grid[2]
    stamps = torch.zeros(groups * per_wg * _PHASE_SLOTS, dtype=torch.int64, device=dev)
    argv, writable, _, stream = rt.build_argv(ck.ir, args, ck.writes)
    argv += [struct.pack("<I", h) for h in plan.hidden] + [mod.wrap_pointer(stamps.data_ptr(), stamps.nbytes,
                                                                            stamps)]
    writable += [False] * len(plan.hidden) + [True]

    def launches(count: int) -> None:
        for _ in range(count):
            mod.launch_groups_async(kern, argv, writable, plan.grid, plan.block, stream=stream)

    def batch() -> float:
        t0 = time.perf_counter()
        launches(SETTLE_BATCH)
        rt.synchronize()
        return time.perf_counter() - t0

    _settle_until_stable(batch, entry + " (stamped)")
    runs = []
    for _ in range(trials):
        launches(lead + 1)
        rt.synchronize()
        s = stamps.cpu().numpy().reshape(groups, per_wg, _PHASE_SLOTS)
        xcd = s[:, 0, 5].astype(np.int64)
        t = s[:, :, :5].astype(np.float64) * 0.01  # 100 MHz ticks -> us
        t -= t[:, :, 0].min()
        loop = t[:, :, 2] - t[:, :, 1]
        if tiled or ws:  # shader clocks over the K loop (slots 6, 7), per BK = 32 stage
            clk = (s[:, 0, 7] - s[:, 0, 6]).astype(np.float64)
            runs.append({"loop_clocks_per_stage": float(np.median(clk)) / -(-k // 32),
                         "loop_shader_GHz": float(np.median(clk / (loop[:, 0] * 1e3)))})
        else:
            runs.append({})
        runs[-1].update({
            "start_spread": t[:, :, 0].max(), "prologue": np.median(t[:, :, 1] - t[:, :, 0]),
            "loop_median": np.median(loop), "loop_min": loop.min(), "loop_max": loop.max(),
            "store_issue": np.median(t[:, :, 3] - t[:, :, 2]), "store_complete": np.median(t[:, :, 4] - t[:, :, 3]),
            "end_median": np.median(t[:, :, 4]), "end_last": t[:, :, 4].max(),
            "loop_median_per_xcd": [float(np.median(loop[xcd == x])) if (xcd == x).any() else None
                                    for x in range(8)],
            "workgroup_to_xcd_is_modulo_8": bool((xcd == np.arange(groups) % 8).all()),
        })
    out = {key: round(float(np.median([r[key] for r in runs])), 2) for key in runs[0]
           if not isinstance(runs[0][key], (list, bool))}
    out["loop_median_per_xcd"] = [round(float(np.median([r["loop_median_per_xcd"][x] for r in runs])), 2)
                                  for x in range(8) if runs[0]["loop_median_per_xcd"][x] is not None]
    out["workgroup_to_xcd_is_modulo_8"] = all(r["workgroup_to_xcd_is_modulo_8"] for r in runs)
    out.update({"unit": "us", "entry": entry, "workgroups": groups, "trials": trials,
                "method": f"median over {trials} trials of the last of {lead + 1} back-to-back launches; "
                          "s_memrealtime stamps by lane 0 of each wave group"
                          + (" (consumer wave 0); s_memtime shader clocks over the K loop" if tiled or ws else "")})
    if tiled or ws:
        out["loop_clocks_per_stage"] = round(float(np.median([r["loop_clocks_per_stage"] for r in runs])), 1)
        out["loop_shader_GHz"] = round(float(np.median([r["loop_shader_GHz"] for r in runs])), 3)
    if tiled:
        # v_mfma_f32_32x32x2_f32 keeps a SIMD's MFMA pipe 64 clocks; 16 steps of 2 k per stage
        out["mfma_clocks_per_stage"] = 64 * 16 * (4 if entry.endswith("__t128") else 1)
    elif ws:
        # v_mfma_f32_16x16x32_f16 keeps it 16 clocks; BM BN / 1024 of them per stage
        bm, bn = {"__t128x256": (128, 256), "__t128x64": (128, 64), "__t64x64": (64, 64)}.get(
            entry[entry.rindex("__"):], (128, 128))
        out["mfma_clocks_per_stage"] = 16 * bm * bn // 1024
    del a, b, c, stamps
    torch.cuda.empty_cache()
    return out


# --workload loadcost: what a 16-byte-per-lane LDS-DMA load costs the MFMA pipe of a SIMD, the
# measurement behind the fp32 GEMM entries' producer waves.  One workgroup per CU; each MFMA wave
# runs 4 independent v_mfma_f32_32x32x2_f32 chains, 16 MFMAs per iteration (1024 clocks of MFMA
# pipe), and counts its shader clocks (s_memtime).  Modes: 0 MFMAs only; 1 MFMA waves that also
# issue LOADS loads per 16 MFMAs (spread one per MFMA slot); 3 waves NW/2.. issue LOADS loads per
# 16 MFMAs of their sibling with SGPR-only addressing (no VALU); 2 the same with VALU addressing,
# running until the MFMA waves are done (a flag in LDS, bounded).  Every load reads inside a
# 256 MiB buffer (offsets masked) and writes its wave's own 1 KB of LDS.
_LOADCOST_SRC = r"""
typedef float lc_f32x16 __attribute__((ext_vector_type(16)));
typedef int lc_rsrc __attribute__((ext_vector_type(4)));
static __device__ __forceinline__ lc_rsrc lc_make_rsrc(const void* p, unsigned bytes) {
  const unsigned long long a = (unsigned long long)p;
  lc_rsrc r;
  r[0] = (int)(unsigned)a; r[1] = (int)((unsigned)(a >> 32) & 0xffffu); r[2] = (int)bytes; r[3] = 0x00020000;
  return r;
}
static __device__ __forceinline__ void lc_dma(lc_rsrc r, unsigned voff, unsigned lds) {
  asm volatile("buffer_load_dwordx4 %0, %1, 0 offen lds" ::"v"(voff), "s"(r), "{m0}"(lds) : "memory");
}
static __device__ __forceinline__ void lc_dma_s(lc_rsrc r, unsigned voff, unsigned soff, unsigned lds) {
  asm volatile("buffer_load_dwordx4 %0, %1, %2 offen lds" ::"v"(voff), "s"(r), "s"(soff), "{m0}"(lds) : "memory");
}
template <int MODE, int NW, int LOADS>
static __device__ void lc_body(const float* src, unsigned bytes, float* out, unsigned long long* clk, int iters) {
  __shared__ __attribute__((aligned(1024))) float lds[8 * 256];
  __shared__ int done;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  if (threadIdx.x == 0) done = 0;
  __syncthreads();
  const lc_rsrc r = lc_make_rsrc(src, bytes);
  const unsigned ldsw = (unsigned)(size_t)(__attribute__((address_space(3))) float*)lds + wave * 1024;
  const unsigned mask = bytes - 1;  // bytes is a power of two
  unsigned voff = ((blockIdx.x * NW + wave) * 64 + lane) * 16;
  lc_f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  const float a = lane * 1e-3f, b = 1.0f + wave;
  const bool mfma_wave = MODE < 2 || wave < NW / 2;
  int n = 0;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  if (mfma_wave) {
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int m = 0; m < 16; ++m) {
        lc_f32x16& c = (m & 3) == 0 ? c0 : (m & 3) == 1 ? c1 : (m & 3) == 2 ? c2 : c3;
        c = __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
        if (MODE == 1 && (m * LOADS) / 16 != ((m + 1) * LOADS) / 16) {
          lc_dma(r, voff & mask, ldsw);
          voff += 1u << 20;
        }
        if (MODE == 1) __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_s_waitcnt(0);
    if (MODE == 2 && lane == 0) __hip_atomic_fetch_add(&done, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  } else if (MODE == 3) {
    const unsigned v0 = (((blockIdx.x * NW + wave) * 64 + lane) * 16) & ((1u << 21) - 1);
    const int total = iters * LOADS / 8;
    for (int it = 0; it < total; ++it) {
#pragma unroll
      for (int j = 0; j < 8; ++j) lc_dma_s(r, v0, ((unsigned)(it * 8 + j) & 127u) << 21, ldsw);  // < 2^28
      n += 8;
    }
    __builtin_amdgcn_s_waitcnt(0);
  } else {
    for (int it = 0; it < iters * 64; ++it) {  // bounded; ends when every MFMA wave is done
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        lc_dma(r, voff & mask, ldsw);
        voff += 1u << 20;
      }
      n += 8;
      if (__hip_atomic_load(&done, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) >= NW / 2) break;
      __builtin_amdgcn_s_sleep(1);
    }
    __builtin_amdgcn_s_waitcnt(0);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  if (lane == 0) {
    // start, end, loads issued, SIMD id (HW_ID bits 5:4)
    clk[(blockIdx.x * 8 + wave) * 4] = t0;
    clk[(blockIdx.x * 8 + wave) * 4 + 1] = t1;
    clk[(blockIdx.x * 8 + wave) * 4 + 2] = (unsigned long long)n;
    clk[(blockIdx.x * 8 + wave) * 4 + 3] = (unsigned long long)__builtin_amdgcn_s_getreg(4 | (4 << 6) | (1 << 11));
  }
  float s = 0.0f;
#pragma unroll
  for (int e = 0; e < 16; ++e) s += c0[e] + c1[e] + c2[e] + c3[e];
  out[blockIdx.x * 512 + threadIdx.x] = s;
}
#define LC_ENTRY(NAME, MODE, NW, LOADS) \
  extern "C" __global__ __launch_bounds__(512) void NAME(const float* src, unsigned bytes, float* out, \
                                                         unsigned long long* clk, int iters) { \
    lc_body<MODE, NW, LOADS>(src, bytes, out, clk, iters); \
  }
LC_ENTRY(lc_w4_mfma, 0, 4, 0)
LC_ENTRY(lc_w4_loads1, 1, 4, 1)
LC_ENTRY(lc_w4_loads2, 1, 4, 2)
LC_ENTRY(lc_w4_loads4, 1, 4, 4)
LC_ENTRY(lc_w8_mfma, 0, 8, 0)
LC_ENTRY(lc_w8_loads1, 1, 8, 1)
LC_ENTRY(lc_w8_loads2, 1, 8, 2)
LC_ENTRY(lc_w8_salu_producers1, 3, 8, 1)
LC_ENTRY(lc_w8_salu_producers2, 3, 8, 2)
LC_ENTRY(lc_w8_valu_producers, 2, 8, 0)
"""
# (entry, waves per workgroup, what it shows)
_LOADCOST_CASES = (
    ("lc_w4_mfma", 4, "1 wave per SIMD, MFMAs only"),
    ("lc_w4_loads1", 4, "1 wave per SIMD, 1 load per 16 MFMAs"),
    ("lc_w4_loads2", 4, "1 wave per SIMD, 2 loads per 16 MFMAs"),
    ("lc_w4_loads4", 4, "1 wave per SIMD, 4 loads per 16 MFMAs"),
    ("lc_w8_mfma", 8, "2 waves per SIMD, MFMAs only"),
    ("lc_w8_loads1", 8, "2 waves per SIMD, each 1 load per 16 of its MFMAs"),
    ("lc_w8_loads2", 8, "2 waves per SIMD, each 2 loads per 16 of its MFMAs"),
    ("lc_w8_salu_producers1", 8, "MFMA wave + sibling issuing 1 load per 16 of its MFMAs, SGPR addressing"),
    ("lc_w8_salu_producers2", 8, "MFMA wave + sibling issuing 2 loads per 16 of its MFMAs, SGPR addressing"),
    ("lc_w8_valu_producers", 8, "MFMA wave + sibling issuing loads with VALU addressing"),
)


def _loadcost_main(rt, torch, iters: int = 2000) -> int:
    """``--workload loadcost``: for each case of ``_LOADCOST_CASES``, the MFMA pipe's clocks per 16
    MFMAs on each SIMD (median over the 256 workgroups' SIMDs, last of 3 launches; ideal 1024 in
    every case): one MFMA wave on a SIMD counts its own span, two count from the earlier start to
    the later end over both waves' MFMAs.  Also the loads the loading waves issued.  Prints a table
    and one JSON line."""
    import struct

    from easy_as_amd.runtime.hip import compile_code

    mod = rt._mod()
    code = compile_code(mod, _LOADCOST_SRC, "loadcost")
    dev = torch.device("cuda:0")
    nbytes = 1 << 28
    src = torch.zeros(nbytes // 4, dtype=torch.float32, device=dev)
    out = torch.zeros(256 * 512, dtype=torch.float32, device=dev)
    clk = torch.zeros(256 * 8 * 4, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream(0).cuda_stream
    argv = [mod.wrap_pointer(src.data_ptr(), src.nbytes, src), struct.pack("<I", nbytes),
            mod.wrap_pointer(out.data_ptr(), out.nbytes, out), mod.wrap_pointer(clk.data_ptr(), clk.nbytes, clk),
            struct.pack("<i", iters)]
    writable = [False, False, True, True, False]
    rows = []
    for entry, nw, what in _LOADCOST_CASES:
        kern = mod.load(code, entry)
        for _ in range(3):
            clk.zero_()
            torch.cuda.synchronize()
            mod.launch_groups(kern, argv, writable, (256, 1, 1), (64 * nw, 1, 1), stream=stream)
        h = clk.cpu().numpy().reshape(256, 8, 4)[:, :nw].astype(np.float64)
        mfma_waves = nw if "producers" not in entry else nw // 2
        per_simd, shared = [], 0
        for g in range(256):
            for simd in range(4):
                on = [w for w in range(mfma_waves) if int(h[g, w, 3]) == simd]
                if on:
                    span = h[g, on, 1].max() - h[g, on, 0].min()
                    per_simd.append(span / (iters * len(on)))
                    shared += len(on) > 1
        loads = h[:, mfma_waves:nw, 2].reshape(-1)
        row = {"case": what, "entry": entry,
               "simd_clocks_per_16_mfma_median": round(float(np.median(per_simd)), 1),
               "simd_clocks_per_16_mfma_max": round(float(np.max(per_simd)), 1),
               "simds_with_two_mfma_waves": shared}
        if loads.size:
            row["loads_per_16_sibling_mfma"] = round(float(np.median(loads)) / iters, 2)
        rows.append(row)
        _log(f"loadcost: {what}: {row['simd_clocks_per_16_mfma_median']} clocks per 16 MFMAs of a SIMD (ideal 1024)"
             + (f", loading waves issued {row['loads_per_16_sibling_mfma']} loads per 16 sibling MFMAs"
                if loads.size else ""))
    base = rows[0]["simd_clocks_per_16_mfma_median"]
    per_load = round((rows[2]["simd_clocks_per_16_mfma_median"] - base) / 2, 1)
    print(json.dumps({"metric": "MFMA pipe clocks lost per 16-byte-per-lane load issued by the MFMA wave",
                      "value": per_load, "unit": "clocks", "higher_is_better": False, "n_gpus": 1,
                      "config": {"workload": "loadcost microbenchmark (v_mfma_f32_32x32x2_f32 chains + LDS DMA)",
                                 "workgroups": 256, "iterations": iters}, "cases": rows}), flush=True)
    del src, out, clk
    return 0


def _host_info() -> dict:
    """The CPU side of the GPU box: core counts, model, NumPy and its BLAS."""
    import os
    import subprocess

    info: dict = {"os_cpu_count": os.cpu_count(), "numpy": np.__version__,
                  "OPENBLAS_NUM_THREADS": os.environ.get("OPENBLAS_NUM_THREADS"),
                  "OMP_NUM_THREADS": os.environ.get("OMP_NUM_THREADS")}
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=20).stdout
        for line in out.splitlines():
            key, _, val = line.partition(":")
            if key.strip() in ("Model name", "Socket(s)", "Core(s) per socket", "Thread(s) per core"):
                info[key.strip()] = val.strip()
    except Exception as e:  # noqa: BLE001
        info["lscpu"] = f"unavailable: {type(e).__name__}"
    try:
        from threadpoolctl import threadpool_info

        info["blas"] = [f"{p.get('internal_api')} {p.get('version')} ({p.get('architecture')})"
                        for p in threadpool_info() if p.get("user_api") == "blas"]
    except Exception as e:  # noqa: BLE001
        info["blas"] = f"unavailable: {type(e).__name__}"
    return info


def _cpu_threads() -> int:
    """BLAS threads for the matmul baselines: os.cpu_count(), capped at the box's CPU share
    (the GPU box exports OMP_NUM_THREADS for the cores it gives one GPU's job)."""
    import os

    share = int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return min(os.cpu_count() or 1, share) if share > 0 else (os.cpu_count() or 1)


def _median_seconds(fn, warmup: int, repeat: int) -> float:
    for _ in range(warmup):
        fn()
    ts = []
    for _ in range(repeat):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    return sorted(ts)[len(ts) // 2]


def _matmul_cpu_baseline(name: str, ha, hb, m: int, n: int, k: int) -> dict:
    """The reference's CPU expression for this configuration, timed on this host: ``A32 @ B32``
    for the fp32 tiled matmuls (tests/test_matmul_tiled.py:172) and
    ``A16.astype(np.float32) @ B16.astype(np.float32)`` for the f16 (and bf16) MMA matmuls
    (examples/matmul_simdgroup.py:219-222), NumPy/OpenBLAS with the BLAS thread count set."""
    from threadpoolctl import threadpool_limits

    threads = _cpu_threads()
    a2, b2 = np.asarray(ha).reshape(m, k), np.asarray(hb).reshape(k, n)
    tiled = name.startswith("tiled")
    if tiled:
        expr = "A32 @ B32"
        fn = lambda: a2 @ b2  # noqa: E731
    else:
        expr = "A16.astype(np.float32) @ B16.astype(np.float32)"
        fn = lambda: a2.astype(np.float32) @ b2.astype(np.float32)  # noqa: E731
    one_run = 2.0 * m * n * k >= 1e12
    with threadpool_limits(threads):
        s = _median_seconds(fn, 1 if one_run else 3, 1 if one_run else 5)
    return {"value": round(2.0 * m * n * k / s / 1e12, 4), "unit": "TFLOP/s", "cores": threads, "kind": "reference",
            "sample": f"the reference's CPU expression {expr} (NumPy {np.__version__}, OpenBLAS, {threads} threads) "
                      f"at the full {m}x{n}x{k} shape on the configuration's inputs, "
                      + ("one timed run after one warmup" if one_run else "median of 5 runs after 3 warmups")
                      + f": {s:.3f} s per matmul"}


def _cpu_baseline(workload: str, hosts: list[np.ndarray]) -> dict:
    """The reference's CPU expression for the elementwise workload on the configuration's own
    arrays (N = 2^28), timed on this host: ``np.add(a, b, out=c)`` (tests/test_add.py:38,
    tests/test_tensor.py:59) and NumPy ``a*b+c`` as ``np.multiply(a, b, out=t); np.add(t, c,
    out=d)`` (tests/test_fma.py:75; two roundings, so it is a timing baseline, not the fma
    oracle).  NumPy ufuncs run on one thread.  The oracle's C restatement (the fma checker) is
    timed beside it on a 2^26 sample."""
    from oracle import ops

    workload = "fma" if workload == "fma_thread" else workload
    n = hosts[0].size if hosts else N_ELEM
    out = np.empty(n, np.float32)
    tmp = np.empty(n, np.float32) if workload == "fma" else None
    a = hosts[0] if hosts else out
    fns = {"add": (lambda: np.add(hosts[0], hosts[1], out=out), "np.add(a, b, out=c)"),
           "fma": (lambda: (np.multiply(hosts[0], hosts[1], out=tmp), np.add(tmp, hosts[2], out=out)),
                   "np.multiply(a, b, out=t); np.add(t, c, out=d)"),
           "copy": (lambda: np.copyto(out, a), "np.copyto(c, a)"),
           "read": (lambda: float(a.sum()), "a.sum()"),
           "write": (lambda: out.fill(1.0), "c.fill(1.0)")}
    fn, expr = fns[workload]
    s = _median_seconds(fn, 3, 5)
    per = WORKLOADS[workload][2]
    res = {"value": round(per * n / s / 1e9, 2), "unit": "GB/s", "cores": 1, "kind": "reference",
           "sample": f"the reference's CPU expression {expr} (NumPy {np.__version__}, one thread) on the "
                     f"configuration's own N=2^28 float32 arrays, median of 5 runs after 3 warmups: "
                     f"{s * 1e3:.1f} ms per pass",
           "host": _host_info()}
    if workload in ("add", "fma"):
        m = 1 << 26
        sa, sb, sc = (x[:m] for x in (hosts + hosts)[:3])
        ofn = (lambda: ops.add_f32(sa, sb)) if workload == "add" else (lambda: ops.fmaf(sa, sb, sc))
        so = _median_seconds(ofn, 1, 5)
        res["oracle_port"] = {"value": round(per * m / so / 1e9, 2), "unit": "GB/s", "cores": 1,
                              "sample": f"oracle {'add_f32' if workload == 'add' else 'fmaf'} (oracle/fmaf.c, "
                                        f"gcc -O2, one thread) on the first 2^26 elements, median of 5"}
    del out, tmp
    return res


def _expected(workload: str, hosts: list[np.ndarray]) -> np.ndarray | None:
    """Closed-form outputs that NumPy computes exactly (binary32 RNE addition, copies,
    constants); None for fma, whose correctly rounded result only the oracle's fmaf
    gives: that one is checked in the CPU leg (``_fma_check``)."""
    if workload == "add":
        return hosts[0] + hosts[1]
    if workload == "read":
        return np.zeros(N_ELEM, np.float32)
    if workload == "write":
        return np.ones(N_ELEM, np.float32)
    if workload == "copy":
        return hosts[0]
    return None


def _fma_check(got: np.ndarray, hosts: list[np.ndarray]) -> bool:
    """CPU leg, as the checker: the GPU's fma outputs against the oracle's fmaf, bit for bit."""
    from oracle import ops

    return bool(np.array_equal(got.view(np.uint32), ops.fmaf(hosts[0], hosts[1], hosts[2]).view(np.uint32)))


def _f64_rel_err(c: np.ndarray, ref: np.ndarray) -> float:
    """``max|C - R| / max|R|`` (the matmul parity metric) with R a float64 matmul."""
    return float(np.max(np.abs(np.asarray(c, np.float64) - ref))) / (float(np.max(np.abs(ref))) or 1.0)


def main() -> int:
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", choices=sorted(WORKLOADS) + sorted(MATMULS) + ["loadcost"], default="add",
                   help="loadcost: the microbenchmark of what a load costs the MFMA pipe (not a config)")
    p.add_argument("--block", type=int, default=PRIMARY_BLOCK)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--no-extra", action="store_true")
    p.add_argument("--shape", default=None,
                   help="matmul workloads only: M,N,K instead of the configuration's shape (a scaling study, "
                        "not the metric)")
    p.add_argument("--phases", action="store_true",
                   help="matmul workloads on the 8-wave GEMM entry, an f16 smaller-tile entry or an fp32 entry: "
                        "add an in-kernel per-phase time budget of one launch (a stamped copy of the kernel, "
                        "timed after the measurement; the smaller-tile and fp32 entries also give shader clocks "
                        "per K stage)")
    p.add_argument("--data", choices=MATMUL_DATA, default="seeded",
                   help="matmul workloads only: input data (anything but 'seeded' is not the metric's data)")
    args = p.parse_args()
    if args.data != "seeded" and args.workload not in MATMULS:
        print("--data applies to the matmul workloads only", file=sys.stderr)
        return 2
    if args.phases and args.workload not in MATMULS:
        print("--phases applies to the matmul workloads only", file=sys.stderr)
        return 2
    if args.shape is not None:
        if args.workload not in MATMULS:
            print("--shape applies to the matmul workloads only", file=sys.stderr)
            return 2
        dims = tuple(int(x) for x in args.shape.split(","))
        if len(dims) != 3 or min(dims) <= 0:
            print("--shape takes M,N,K (positive)", file=sys.stderr)
            return 2
        SHAPE_OVERRIDE[args.workload] = dims
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported in this build "
              "(the elementwise path would shard N contiguously per GPU with no exchange).", file=sys.stderr)
        return 2

    import torch

    import kernels as K
    from easy_as_amd.runtime import get_runtime

    rt = get_runtime("hip")
    dev = torch.device("cuda:0")
    if args.workload == "loadcost":
        return _loadcost_main(rt, torch)
    if args.workload in MATMULS:
        return _matmul_main(args, rt, torch)
    kname, nin, per_elem = WORKLOADS[args.workload]
    _log(f"device {torch.cuda.get_device_name(0)}; workload {args.workload}; generating inputs N=2^28")
    nin_all = 3 if args.workload == "add" and not args.no_extra else nin
    hosts = _inputs(N_ELEM, tuple(range(nin_all)))
    ins = [torch.from_numpy(h).to(dev) for h in hosts]
    out = torch.zeros(N_ELEM, dtype=torch.float32, device=dev)

    def elementwise(workload: str, block: int) -> dict:
        """Time one elementwise configuration, then check every one of its 2^28 outputs."""
        kn, k_in, per = WORKLOADS[workload]
        kern = getattr(K, kn)
        names = list(kern.sig.parameters)[: k_in + 1]
        rargs = dict(zip(names, ins[:k_in] + [out]))
        rargs["N"] = N_ELEM
        ck = kern.compile(*ins[:k_in], out, N_ELEM, BLOCK=block)
        wall_ms, ev_ms = _time_kernel(rt, ck, rargs, {"BLOCK": block}, args.steps, args.warmup, torch)
        # NaN marks outputs a kernel failed to write; the read kernel writes none, so its
        # output must stay as filled (zeros)
        out.fill_(0.0 if workload == "read" else float("nan"))
        kern(*ins[:k_in], out, N_ELEM, BLOCK=block)
        torch.cuda.synchronize()
        got = out.cpu().numpy()
        want = _expected(workload, hosts)
        if want is not None:
            exact = bool(np.array_equal(got.view(np.uint32), want.view(np.uint32)))
            parity = "bit-exact vs binary32 closed form (all 2^28 outputs)" if exact else "MISMATCH"
        elif not args.no_cpu_baseline:
            exact = _fma_check(got, hosts)
            parity = "bit-exact vs oracle fmaf (all 2^28 outputs)" if exact else "MISMATCH"
        else:
            exact, parity = True, "not checked (--no-cpu-baseline skips the oracle)"
        geo = ck.geometry
        unit = "threadgroup" if ck.launch_mode == "thread" else "program"  # what a group of lanes is
        res = {"ck": ck, "rargs": rargs, "wall_ms": wall_ms, "ev_ms": ev_ms, "GB/s": round(per * N_ELEM / ev_ms / 1e6, 1),
               "frac": round(per * N_ELEM / ev_ms / 1e6 / HBM_PEAK_GBS, 4), "ms_per_launch": round(ev_ms, 5),
               "parity": parity, "parity_ok": exact,
               "launch": f"{geo.wg_size} threads per workgroup, "
                         + (f"{geo.split} workgroups per {unit}" if geo.split > 1
                            else f"{geo.programs_per_wg} {unit}(s) per workgroup")}
        if ck.launch_mode == "thread":
            res["kernel"] = (f"{kn}, thread mode (mk.tid), "
                             + ("emitted as lanes of one program per threadgroup" if geo.params.get("lanes")
                                else "one HIP thread per Metal thread"))
        _log(f"{workload} BLOCK={block}: wall {wall_ms:.4f} ms/step, event {ev_ms:.4f} ms/launch, "
             f"{res['GB/s']} GB/s, {res['launch']}, parity {parity}")
        return res

    prim = elementwise(args.workload, args.block)
    wall_ms, ev_ms, exact, parity = prim["wall_ms"], prim["ev_ms"], prim["parity_ok"], prim["parity"]
    # the workgroups per ns the kernel needs, beside what this box's command processor dispatches
    # (an empty kernel of the same launch shape, this session): a box that dispatches slowly shows
    # here instead of only as a lower bandwidth
    from easy_as_amd.runtime.hip import plan_launch

    kplan = plan_launch(prim["ck"], prim["rargs"])
    need = kplan.grid[0] / (ev_ms * 1e6)
    probe = _dispatch_probe(rt, kplan.grid[0], kplan.block[0])
    dispatch = {"workgroups": kplan.grid[0], "threads_per_workgroup": kplan.block[0],
                "kernel_workgroups_per_ns": round(need, 3), "probe_workgroups_per_ns": round(probe, 3),
                "kernel_over_probe": round(need / probe, 3),
                "probe": "empty kernel, same workgroup count and size, HIP events, median of 5 x 20 launches"}
    _log(f"dispatch: {args.workload} needs {need:.3f} workgroups/ns; an empty kernel of the same shape "
         f"dispatches {probe:.3f}/ns ({100 * need / probe:.1f} %)")
    # vendor comparison on the same device-resident inputs: the torch (ROCm) operation
    tfn = {"add": lambda: torch.add(ins[0], ins[1], out=out),
           "fma": lambda: torch.addcmul(ins[2], ins[0], ins[1], out=out),
           "fma_thread": lambda: torch.addcmul(ins[2], ins[0], ins[1], out=out),
           "copy": lambda: out.copy_(ins[0]), "read": lambda: ins[0].sum(), "write": lambda: out.fill_(1.0)}
    texpr = {"add": "torch.add(a, b, out=c)", "fma": "torch.addcmul(c, a, b, out=d)",
             "fma_thread": "torch.addcmul(c, a, b, out=d)", "copy": "c.copy_(a)",
             "read": "a.sum()", "write": "c.fill_(1.0)"}[args.workload]
    tms = _torch_event_ms(tfn[args.workload], args.steps, args.warmup, torch)
    vendor = {"op": texpr, "GB/s": round(per_elem * N_ELEM / tms / 1e6, 1), "ms_per_launch": round(tms, 5)}
    _log(f"{texpr}: {tms:.4f} ms/launch, {vendor['GB/s']} GB/s")
    extra: dict = {}
    if not args.no_extra and args.workload == "add":
        # configs[1] in full: add at the other BLOCK and fma at both, each timed and checked
        other = 1024 if args.block != 1024 else 256
        for wl, blk in (("add", other), ("fma", 256), ("fma", 1024), ("fma_thread", 256), ("fma_thread", 1024)):
            r = elementwise(wl, blk)
            extra[f"{wl}_block{blk}"] = {k: v for k, v in r.items()
                                         if k not in ("wall_ms", "ev_ms", "parity_ok", "ck", "rargs")}
            exact = exact and r["parity_ok"]
        cpu_fma = None if args.no_cpu_baseline else _cpu_baseline("fma", hosts)
        if cpu_fma is not None:
            cpu_fma.pop("host", None)
            extra["fma_block256"]["cpu_baseline"] = cpu_fma

    if not args.no_extra and args.workload == "add":
        # the plumbing sizes, launch-latency bound.  us_per_call is a whole eas call
        # (binding, specialisation lookup, launch plan, argument packing, async launch) averaged
        # over back-to-back calls; us_per_launch is the GPU time by HIP events.
        for n in (1031, 1 << 20):
            sa, sb = ins[0][:n], ins[1][:n]
            sc = torch.empty(n, dtype=torch.float32, device=dev)
            calls = 2000
            for _ in range(50):
                K.add_kernel(sa, sb, sc, n, BLOCK=PRIMARY_BLOCK, _sync=False)
            rt.synchronize()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(calls):
                K.add_kernel(sa, sb, sc, n, BLOCK=PRIMARY_BLOCK, _sync=False)
            rt.synchronize()
            torch.cuda.synchronize()
            per_call = (time.perf_counter() - t0) / calls
            cks = K.add_kernel.compile(sa, sb, sc, n, BLOCK=PRIMARY_BLOCK)
            sargs = {"a": sa, "b": sb, "c": sc, "N": n}
            ev = sorted(rt.benchmark(cks, sargs, {"BLOCK": PRIMARY_BLOCK}, repeat=200, warmup=20)
                        for _ in range(EVENT_TRIALS))[EVENT_TRIALS // 2]
            ok = bool(np.array_equal(sc.cpu().numpy().view(np.uint32), (hosts[0][:n] + hosts[1][:n]).view(np.uint32)))
            extra[f"add_n{n}"] = {"us_per_call": round(per_call * 1e6, 2), "us_per_launch": round(ev * 1e6, 2),
                                  "GB/s": round(12 * n / ev / 1e9, 1),
                                  "parity": "bit-exact vs binary32 closed form" if ok else "MISMATCH"}
            _log(f"add N={n}: {per_call * 1e6:.2f} us per eas call, {ev * 1e6:.2f} us per launch (events), "
                 f"parity {extra[f'add_n{n}']['parity']}")
            del sc
        del ins, out
        torch.cuda.empty_cache()
        for name in ("mma", "mma_k4100", "mma_bf16", "decode", "prefill", "tiled1024", "tiled2048"):
            # a failing extra is reported in the line; it does not take the primary measurement with it
            try:
                extra[name] = _matmul(name, rt, torch, max(5, min(args.steps, 20)), max(2, min(args.warmup, 5)),
                                      cpu_baseline=not args.no_cpu_baseline)
            except Exception as e:  # noqa: BLE001
                _log(f"{name}: {type(e).__name__}: {e}")
                extra[name] = {"error": f"{type(e).__name__}: {e}"}

    bytes_per_launch = per_elem * N_ELEM
    traffic = None
    pmc = ROOT / "profiles" / f"{args.workload}_f32_n2e28.pmc.json"
    if pmc.exists() and args.block == PRIMARY_BLOCK:
        # HBM bytes per launch from the committed rocprofv3 FETCH_SIZE/WRITE_SIZE passes,
        # each scaled by the reading of a known-size copy (see that file).
        traffic = json.loads(pmc.read_text()).get("traffic_bytes_per_launch")
    value = bytes_per_launch / (wall_ms * 1e-3) / 1e9
    achieved = bytes_per_launch / (ev_ms * 1e-3) / 1e9
    expr = {"add": "c=a+b", "fma": "d=a*b+c (fused, one rounding)", "fma_thread": "d=a*b+c (fused, one rounding)",
            "copy": "c=a", "read": "read a", "write": "c=1"}[args.workload]
    style = ("thread-mode (mk.tid, masked tail)" if args.workload == "fma_thread"
             else "SPMD (mk.arange, masked tail)")
    line = {
        "metric": f"fp32 {args.workload} GB/s @N=2^28 (eas {style.split(' ')[0]} kernel, one MI355X)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": f"synthetic (N(0,1) float32, seeds {list(range(nin))})",
        "config": {"workload": f"fp32 {args.workload} {expr} via @eas.kernel {style}, "
                               f"N=2^28, BLOCK={args.block}",
                   "N": N_ELEM, "BLOCK": args.block, "parallelism": "single GPU"},
        "parity": parity,
        "roofline": {"bound": "hbm", "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic},
        "dispatch": dispatch,
        "cpu_baseline": None if args.no_cpu_baseline else _cpu_baseline(args.workload, hosts[:nin]),
        "vendor": vendor,
        "settle": {"untimed_launches_before_warmup": list(SETTLE_LOG),
                   "rule": f"batches of {SETTLE_BATCH} until two agree within 2%"},
        "extra": extra,
    }
    print(json.dumps(line), flush=True)
    return 0 if exact else 1


def _matmul_main(args, rt, torch) -> int:
    res = _matmul(args.workload, rt, torch, args.steps, args.warmup, args.data,
                  cpu_baseline=not args.no_cpu_baseline)
    _, m, n, k, _, _, desc = _config(args.workload)
    traffic = None
    pmc = ROOT / "profiles" / f"{MATMUL_PROFILES.get(args.workload, args.workload)}.pmc.json"
    if pmc.exists() and args.workload not in SHAPE_OVERRIDE:
        traffic = json.loads(pmc.read_text()).get("traffic_bytes_per_launch")
    tiled = args.workload.startswith("tiled")
    in_dt = "f32" if tiled else ("bf16" if args.workload.endswith("bf16") else "f16")
    wall_tf = res["wall_TFLOP/s"]
    line = {
        "metric": f"{'fp32' if tiled else in_dt} matmul TFLOP/s @{m}x{n}x{k} (eas kernel, one MI355X)",
        "value": wall_tf,
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(2.0 * m * n * k / (wall_tf * 1e12) * 1e3, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": in_dt,
        "data": "synthetic (seeded; see config)" if args.data == "seeded" else
                f"constant inputs ({args.data}): a power probe, not the configs' distribution",
        "config": {"workload": desc, "M": m, "N": n, "K": k, "parallelism": "single GPU"},
        "parity": res["parity"],
        "parity_elementwise_err": res["elementwise_err"], "parity_max_abs_err": res["max_abs_err"],
        "roofline": ({"bound": "hbm", "achieved": res["min_hbm_GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                      "frac": res["frac_of_bound"], "traffic": traffic} if res["bound"] == "hbm" else
                     {"bound": res["bound"], "achieved": res["TFLOP/s"], "peak": res["peak_TFLOP/s"],
                      "unit": "TFLOP/s", "frac": res["frac"], "traffic": traffic}),
        "cpu_baseline": (dict(res["cpu_baseline"], host=_host_info()) if "cpu_baseline" in res else None),
        "vendor": (dict(res["torch_matmul"]) if "torch_matmul" in res else None),
        "settle": {"untimed_launches_before_warmup": list(SETTLE_LOG),
                   "rule": f"batches of {SETTLE_BATCH} until two agree within 2%"},
        "extra": {},
    }
    if args.phases:
        line["phases"] = _gemm_phases(args.workload, rt, torch)
        _log(f"{args.workload}: phases {json.dumps(line['phases'])}")
    print(json.dumps(line), flush=True)
    return 0 if res["parity_ok"] else 1


if __name__ == "__main__":
    sys.exit(main())
