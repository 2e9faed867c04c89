#!/usr/bin/env python3
"""Benchmark of the PSGD-Kron preconditioner update + gradient apply on one MI355X.

Default workload (one line of JSON on stdout): one optimizer step (preconditioner update of every factor, then
precondition + clip + parameter update) over the ViT-B/16 weight set, 12 blocks x {qkv 768x2304, proj 768x768,
fc1 768x3072, fc2 3072x768} = 48 weights, bf16 gradients N(0, 1e-4) resident in HBM, fp32 Kron factors initialised
to the identity, max_size 8192, max_skew inf (every side dense), update probability 1, contractions on the bf16
MFMA path (fp32 accumulate). Synthetic data; weights random-initialised.

    python bench.py [--steps K] [--warmup W] [--precision bf16|fp32] [--skew inf|1] [--no-cpu]
    python bench.py --config syrk      # SYRK / TRMM microbenchmark lines (n = k in 512..4096, fp32 and bf16)
    python bench.py --config ceiling   # hipBLASLt against the library's bf16 GEMM on the optimizer's shapes
    python bench.py --config gemm      # 12 x 3072^3 bf16 GEMM launches (the dominant kernel), for counter runs

`roofline` is measured live: every MFMA-engine launch in the timed steps is bracketed by HIP events on its stream;
the dominant kernel instantiation (largest total time) is reported with its algorithmic TFLOP/s against the bf16
(or fp32) MFMA peak. `traffic` (HBM bytes per launch of that kernel) comes from the committed rocprofv3 counter
summary when present. `sustained_peak` is the bf16 MFMA rate measured live on the same GPU by a kernel of
independent MFMAs with no memory traffic (the ceiling at the box's engine clock under load), and
`frac_of_sustained` the dominant kernel's rate over it; `peak` and `frac` stay the published figures. `cpu_baseline` times the CPU oracle (oracle/psgd_oracle.py, float32, torch CPU threads) on
one ViT-B block (4 of the 48 weights) and scales it to the whole set.
"""
import argparse
import ctypes as C
import json
import math
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

PEAK = {"bf16": 2516.6, "fp32": 157.3}  # TFLOP/s, MI355X dense MFMA
VIT_B = [(768, 2304), (768, 768), (768, 3072), (3072, 768)]
METRIC = "Kron update+apply ms/step & SYRK TFLOP/s (% MFMA peak) at ViT-B shapes, 1 GPU"
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_bf16_vitb16_traffic.txt")


def parse_args():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--precision", choices=["bf16", "fp32"], default="bf16")
    ap.add_argument("--skew", default="inf")
    ap.add_argument("--blocks", type=int, default=12)
    ap.add_argument("--config", choices=["vitb", "syrk", "copy", "llama", "e2e", "ceiling", "gemm"], default="vitb")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--streams", type=int, default=None,
                    help="side streams for independent weight groups (default: KronWhiten's, 3 for up to four groups, "
                         "4 for more)")
    ap.add_argument("--graphs", type=int, default=0,
                    help="must stay 0: replaying the step from a captured HIP graph is switched off")
    ap.add_argument("--fuse", type=int, default=1,
                    help="0: one update call per weight group instead of one call batching all groups' factor work")
    ap.add_argument("--rq16", type=int, default=1, help="0: keep R Q in fp32 between the Procrustes products (option 7)")
    ap.add_argument("--f32kc", type=int, default=1,
                    help="0: fp32 products on the general engine instead of the k-contiguous kernel's fp32 twin (option 8)")
    ap.add_argument("--vmm", type=int, default=-1,
                    help="V A kernel of the norm bounds (option 4): -1 by shape, 0 split-K, 1 column blocks, 2 LDS rows, "
                         "3 upper tiles in tournament-paired rounds")
    ap.add_argument("--tile-cfg", type=int, default=-1,
                    help="bf16 GEMM tile configuration for every launch (library option 1; -1: chosen by size)")
    ap.add_argument("--upd-streams", type=int, default=3,
                    help="side streams of the grouped update inside the library (library option 6)")
    ap.add_argument("--big-batch", type=int, default=64,
                    help="items per batch of the grouped update for factor sides >= 2048 (library option 9)")
    ap.add_argument("--t1q-pg", type=int, default=1,
                    help="0: form term1 Q as the reference writes it, never through Pg (library option 5)")
    ap.add_argument("--r2", type=int, default=0,
                    help="1: the Procrustes step in the reference's r2 form (KronWhiten(r2=True), 3 d^3 instead of 4 d^3)")
    ap.add_argument("--opt", action="append", default=[], metavar="N=V",
                    help="set library option N to V before the run (psgdk_set_option; repeatable)")
    return ap.parse_args()


def read_traffic(kernel):
    """HBM bytes per launch of `kernel` from the committed counter summary (lines `kernel: ...` and
    `bytes_per_launch: ...`), or None."""
    try:
        lines = open(TRAFFIC_FILE).read().splitlines()
    except OSError:
        return None
    k = b = None
    for ln in lines:
        if ln.startswith("kernel:"):
            k = ln.split(":", 1)[1].strip()
        if ln.startswith("bytes_per_launch:"):
            b = float(ln.split(":", 1)[1].strip())
    return b if (k == kernel and b is not None) else None


PEAK_HBM = 8.0  # TB/s, MI355X HBM3E


def mfma_sustained(dev):
    """The bf16 MFMA rate the GPU sustains now (psgdk_mfma_rate: 2 workgroups of 4 waves per CU, each wave issuing
    32 independent 16 x 16 x 32 MFMAs per round with no memory traffic), in TFLOP/s: the ceiling at the box's current
    engine clock under a dense MFMA load."""
    import torch
    from psgd_pro_amd import _lib as L
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    wgs, iters = 2 * cus, 20000
    out = torch.empty(4 * wgs, device=dev)
    st = L.stream_of(out)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    L.check(L.lib().psgdk_mfma_rate(iters, wgs, C.c_void_p(out.data_ptr()), st))
    torch.cuda.synchronize(dev)
    ev[0].record()
    for _ in range(3):
        L.check(L.lib().psgdk_mfma_rate(iters, wgs, C.c_void_p(out.data_ptr()), st))
    ev[1].record()
    torch.cuda.synchronize(dev)
    sec = ev[0].elapsed_time(ev[1]) * 1e-3 / 3
    return 4 * wgs * iters * 32 * 16384 / sec / 1e12


CLOCK_MHZ = 2400.0  # MI355X peak engine clock: the published MFMA and HBM peaks assume it


def read_rates(dev):
    """The read rates this GPU sustains now (psgdk_read_rate, TB/s): HBM (a 2 GiB buffer read once per launch by 2048
    workgroups) and the L2 (a 2 MiB buffer read 4096 times by 1024 workgroups, odd stride), median of 5 launches."""
    import torch
    from psgd_pro_amd import _lib as L
    out = {}
    for name, nbytes, wgs, iters, stride in (("hbm", 2 << 30, 2048, (2 << 30) // 4096 // 2048, 1),
                                             ("l2", 2 << 20, 1024, 4096, 977)):
        buf = torch.ones(nbytes, dtype=torch.uint8, device=dev)
        sink = torch.zeros(wgs, dtype=torch.int32, device=dev)
        st = L.stream_of(buf)
        f = lambda: L.check(L.lib().psgdk_read_rate(C.c_void_p(buf.data_ptr()), nbytes, wgs, iters, stride,
                                                    C.c_void_p(sink.data_ptr()), st))
        f()
        times = []
        for _ in range(5):
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record()
            f()
            ev[1].record()
            torch.cuda.synchronize(dev)
            times.append(ev[0].elapsed_time(ev[1]) * 1e-3)
        out[name] = round(wgs * iters * 4096 / sorted(times)[2] / 1e12, 2)
        del buf, sink
    return out


class ClockSampler:
    """The engine clock over a region of work on `stream`: a one-wave sampler on its own stream records (cycle
    counter, wall counter) pairs about every 4 us (psgdk_clock_sample) while two wall marks on `stream` bracket the
    region; the clock is the cycle increment over the wall increment between the first and last samples inside it."""

    def __init__(self, dev):
        """Create it before any other stream of the process: the runtime spreads streams over a few hardware queues,
        and a sampler whose queue is shared with the timed stream runs before that stream's work instead of beside
        it (then no sample falls inside the region and the result says so)."""
        import torch
        from psgd_pro_amd import _lib as L
        self.L, self.dev = L, dev
        self.side = torch.cuda.Stream(device=dev)
        khz = C.c_int(0)
        L.check(L.lib().psgdk_wall_clock_rate(C.byref(khz)))
        self.khz = khz.value
        probe = torch.zeros(1, dtype=torch.int64, device=dev)  # first use of the stream (queues may bind on use)
        L.check(L.lib().psgdk_wall_mark(C.c_void_p(probe.data_ptr()), C.c_void_p(self.side.cuda_stream)))
        torch.cuda.synchronize(dev)

    def arm(self, stream, est_ms):
        import torch
        self.stream = stream
        self.n = int(min(1 << 22, max(1024, est_ms * 1e3 / 2.5 * 1.5)))
        self.buf = torch.zeros(2 * self.n, dtype=torch.int64, device=self.dev)
        self.marks = torch.zeros(2, dtype=torch.int64, device=self.dev)
        return self

    def start(self):
        raw = lambda st: C.c_void_p(st.cuda_stream)
        self.side.wait_stream(self.stream)
        self.L.check(self.L.lib().psgdk_clock_sample(self.n, C.c_void_p(self.buf.data_ptr()), raw(self.side)))
        self.L.check(self.L.lib().psgdk_wall_mark(C.c_void_p(self.marks.data_ptr()), raw(self.stream)))

    def stop(self):
        self.L.check(self.L.lib().psgdk_wall_mark(C.c_void_p(self.marks.data_ptr() + 8), C.c_void_p(self.stream.cuda_stream)))

    def result(self):
        import torch
        torch.cuda.synchronize()
        s = self.buf.view(-1, 2).cpu()
        m0, m1 = (int(x) for x in self.marks.cpu())
        inside = s[(s[:, 1] >= m0) & (s[:, 1] <= m1)]
        if len(inside) < 2:
            return {"mhz": None, "samples": int(len(inside)), "coverage": 0.0}
        dc = float(inside[-1, 0] - inside[0, 0])
        dw = float(inside[-1, 1] - inside[0, 1])
        return {"mhz": round(dc / dw * self.khz / 1e3, 1), "samples": int(len(inside)),
                "coverage": round(dw / max(1.0, float(m1 - m0)), 3)}


def roof_ms(fl, by, peak):
    """The roofline model's time for a launch: its flops at the MFMA peak or its algorithmic bytes at the HBM peak,
    whichever takes longer (ms)."""
    return max(fl / (peak * 1e12), by / (PEAK_HBM * 1e12)) * 1e3


def aggregate(recs, peak):
    """Per kernel instantiation: launches, total ms, algorithmic flops and bytes, roofline-model ms; plus the SYRK
    subset."""
    agg, syrk = {}, {}
    for r in recs:
        kid, tri, ms, fl, by = r.kernel_id, r.tri, r.ms, r.flops, r.bytes
        for d in (agg, syrk) if tri else (agg,):
            a = d.setdefault(kid, [0, 0.0, 0.0, 0.0, 0.0])
            a[0] += 1
            a[1] += ms
            a[2] += fl
            a[3] += by
            a[4] += roof_ms(fl, by, peak)
    return agg, syrk


def launch_classes(recs, steps, peak, top=12):
    """The most expensive (kernel, problems, shape) classes of MFMA launches, per step, each against its own roof:
    its arithmetic intensity (algorithmic flops / algorithmic bytes) against the ridge (MFMA peak / HBM peak) says
    whether the MFMA peak or the HBM peak bounds it, and roof_frac is the roofline model's time over the measured
    time. shape is [problems, m, n, k] (k: the largest problem's); rounds is the launch's workgroups over the ones
    the GPU holds at once (CUs x per_cu, the kernel's occupancy), so 1.27 means a full round and a 27% tail."""
    import torch
    from psgd_pro_amd import _lib as L
    cus = torch.cuda.get_device_properties(torch.cuda.current_device()).multi_processor_count
    agg = {}
    for r in recs:
        key = (r.kernel_id, r.tri, r.nb, r.m, r.n, r.k, round(r.flops), round(r.bytes), r.workgroups, r.per_cu)
        a = agg.setdefault(key, [0, 0.0])
        a[0] += 1
        a[1] += r.ms
    rows = sorted(agg.items(), key=lambda kv: -kv[1][1])[:top]
    out = []
    for (kid, tri, nb, m, n, k, fl, by, wgs, per_cu), v in rows:
        us = v[1] * 1e3 / v[0]
        ai = fl / by
        out.append({"kernel": kid, "name": L.kernel_name(kid), "syrk": bool(tri), "shape": [nb, m, n, k],
                    "gflop": round(fl / 1e9, 2), "gbyte": round(by / 1e9, 3), "flop_per_byte": round(ai, 1),
                    "bound": "mfma" if ai >= peak / PEAK_HBM else "hbm",
                    "launches_per_step": v[0] / steps, "us": round(us, 1),
                    "tflops": round(fl / (us * 1e-6) / 1e12, 1), "tbps": round(by / (us * 1e-6) / 1e12, 2),
                    "roof_frac": round(roof_ms(fl, by, peak) * 1e3 / us, 3), "workgroups": wgs, "per_cu": per_cu,
                    "rounds": round(wgs / (cus * per_cu), 2) if per_cu else None})
    return out


def cpu_threads():
    """The host threads the CPU leg may use: the CPUs this process may run on, capped by OMP_NUM_THREADS when set
    (the GPU box gives one GPU's job a share of the host, announced there through OMP_NUM_THREADS)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    env = os.environ.get("OMP_NUM_THREADS", "")
    if env.isdigit() and int(env) > 0:
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(precision, skew, seconds):
    """The CPU oracle (float32) on one ViT-B block (4 weights): with every host thread the process may use, 1 warmup
    step, then timed steps until `seconds` of work (median); with one thread, one timed step. Both scaled x12 to
    the 48-weight set (the 12 blocks are identical, and the oracle steps the weights one after another)."""
    import torch
    from oracle import psgd_oracle as O
    threads = cpu_threads()
    gen = torch.Generator().manual_seed(7)
    grads = [(0.01 * torch.randn(s, generator=gen)).to(torch.bfloat16).float() for s in VIT_B]
    eps = torch.finfo(torch.bfloat16).eps if precision == "bf16" else None

    def oracle():
        return O.OracleKron([torch.zeros(s) for s in VIT_B], preconditioner_max_size=8192,
                            preconditioner_max_skew=skew, preconditioner_init_scale=1.0, seed=0, dtype=torch.float32,
                            grad_eps=eps)
    torch.set_num_threads(threads)
    ora = oracle()
    ora.step(grads)
    times = []
    t_start = time.perf_counter()
    while True:
        t0 = time.perf_counter()
        ora.step(grads)
        times.append(time.perf_counter() - t0)
        if time.perf_counter() - t_start > seconds or len(times) >= 20:
            break
    times.sort()
    med = times[len(times) // 2]
    torch.set_num_threads(1)
    ora1 = oracle()
    t0 = time.perf_counter()
    ora1.step(grads)
    one = time.perf_counter() - t0
    torch.set_num_threads(threads)
    return dict(value=round(med * 1e3 * 12, 2), unit="ms/step", cores=threads, kind="port",
                host_cpus=os.cpu_count(), value_1_thread=round(one * 1e3 * 12, 2),
                sample=f"oracle float32 on 1 ViT-B block (4 of 48 weights) x12: median of {len(times)} steps after "
                       f"1 warmup on {threads} threads; 1 step on 1 thread for value_1_thread")


def check_finite(opt, params):
    """Fails the run when any parameter, factor or L is not finite after the timed steps."""
    import torch
    bad = [i for i, p in enumerate(params) if not bool(torch.isfinite(p).all())]
    for i in range(len(params)):
        Qs, Ls = opt.factors(i)
        if not all(bool(torch.isfinite(t).all()) for t in Qs + Ls):
            bad.append(i)
    if bad:
        print(f"bench.py: non-finite parameters or factors after the timed steps (weights {sorted(set(bad))[:8]})",
              file=sys.stderr)
        sys.exit(3)


def bench_vitb(args):
    import torch
    from psgd_pro_amd.flops import flops_2d, is_dense
    from psgd_pro_amd import KronWhiten
    from psgd_pro_amd import _lib as L

    dev = torch.device("cuda:0")
    clock = ClockSampler(dev)  # first stream of the process (see ClockSampler)
    L.check(L.lib().psgdk_set_option(5, args.t1q_pg))
    L.check(L.lib().psgdk_set_option(6, args.upd_streams))
    L.check(L.lib().psgdk_set_option(1, args.tile_cfg))
    L.check(L.lib().psgdk_set_option(7, args.rq16))
    L.check(L.lib().psgdk_set_option(4, args.vmm))
    L.check(L.lib().psgdk_set_option(8, args.f32kc))
    L.check(L.lib().psgdk_set_option(9, args.big_batch))
    skew = math.inf if args.skew == "inf" else float(args.skew)
    shapes = VIT_B * args.blocks
    gen = torch.Generator().manual_seed(0)
    params = [(0.02 * torch.randn(s, generator=gen)).to(dev).requires_grad_(True) for s in shapes]
    grads = [(0.01 * torch.randn(s, generator=gen)).to(torch.bfloat16).to(dev) for s in shapes]
    opt = KronWhiten(params, preconditioner_max_size=8192, preconditioner_max_skew=skew,
                     preconditioner_init_scale=1.0, precision=args.precision, draws="device", seed=0,
                     streams=args.streams, graphs=bool(args.graphs), r2=bool(args.r2), fuse_groups=bool(args.fuse))
    flops_step = sum(flops_2d(m, n, is_dense(m, m * n, 8192, skew), is_dense(n, m * n, 8192, skew), r2=bool(args.r2))
                     for m, n in shapes)
    for _ in range(args.warmup):
        opt.step_math(grads)
    torch.cuda.synchronize()
    stream = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        opt.step_math(grads)
    e1.record(stream)
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    wall_ms = (t1 - t0) * 1e3 / args.steps
    ev_ms = e0.elapsed_time(e1) / args.steps
    check_finite(opt, params)
    # Per-launch figures come from a second pass on one stream, eager, so that each kernel's HIP-event duration is
    # its own and not shared with another group's kernels.
    opt._nstreams = 0
    L.check(L.lib().psgdk_set_option(6, 0))  # the grouped update's side streams too
    opt.step_math(grads)
    torch.cuda.synchronize()
    # the engine clock over this pass: the published peaks assume CLOCK_MHZ, and the GPU lowers its clock under a
    # sustained MFMA and memory load
    clock.arm(stream, est_ms=1.5 * args.steps * ev_ms + 50)
    clock.start()
    L.profile_start()
    for _ in range(args.steps):
        opt.step_math(grads)
    clock.stop()
    torch.cuda.synchronize()
    recs = L.profile_stop()
    clk = clock.result()
    opt._nstreams = args.streams
    L.check(L.lib().psgdk_set_option(6, args.upd_streams))
    streams_used = opt.side_streams()
    sustained = mfma_sustained(dev)
    rates = read_rates(dev)
    peak = PEAK[args.precision]
    agg, syrk = aggregate(recs, peak)
    kid = max(agg, key=lambda k: agg[k][1])
    n_l, ms_tot, fl_tot, by_tot, roof_tot = agg[kid]
    prec_of = "bf16" if (kid >= 5000 or (kid % 1000) // 100 == 1) else "fp32"
    ai = fl_tot / by_tot
    mfma_bound = ai >= PEAK[prec_of] / PEAK_HBM
    achieved = fl_tot / (ms_tot * 1e-3) / 1e12 if mfma_bound else by_tot / (ms_tot * 1e-3) / 1e9
    kname = L.kernel_name(kid)
    traffic = read_traffic(kname)
    s_l = sum(v[0] for v in syrk.values())
    s_ms = sum(v[1] for v in syrk.values())
    s_fl = sum(v[2] for v in syrk.values())
    s_roof = sum(v[4] for v in syrk.values())
    syrk_tf = s_fl / (s_ms * 1e-3) / 1e12 if s_ms else 0.0
    mfma_ms = sum(v[1] for v in agg.values()) / args.steps
    mfma_fl = sum(v[2] for v in agg.values()) / args.steps  # flops the MFMA launches execute (their own shapes)
    out = {
        "metric": METRIC,
        "value": round(wall_ms, 3),
        "unit": "ms/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms, 3),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.precision,
        "data": "synthetic",
        "config": {"workload": "vit-b16-kron-update-apply", "weights": "12 x {768x2304, 768x768, 768x3072, 3072x768}",
                   "cpu_baseline_sample": "one ViT-B block, x12",
                   "blocks": args.blocks, "grad_dtype": "bf16", "factor_dtype": "fp32", "max_size": 8192,
                   "max_skew": args.skew, "update_probability": 1.0, "procrustes": "r2" if args.r2 else "step2",
                   "term1_q": "pg" if args.t1q_pg else "term1", "fuse_groups": bool(args.fuse),
                   "update_side_streams": args.upd_streams,
                   "parallelism": "none"},
        "gpu_ms_per_step": round(ev_ms, 3),
        "streams": streams_used,
        "graphs": bool(args.graphs),
        "profile_pass": "per-launch figures (roofline, kernels, launch_classes) from a separate single-stream pass",
        "algorithmic_tflop_per_step": round(flops_step / 1e12, 4),
        "tflops": round(flops_step / (wall_ms * 1e-3) / 1e12, 2),
        "mfma_ms_per_step": round(mfma_ms, 3),
        "executed_mfma_tflop_per_step": round(mfma_fl / 1e12, 4),
        "executed_tflops": round(mfma_fl / (wall_ms * 1e-3) / 1e12, 2),
        "syrk": {"tflops": round(syrk_tf, 2), "frac": round(syrk_tf / PEAK[args.precision], 4),
                 "roof_frac": round(s_roof / s_ms, 4) if s_ms else None,
                 "launches_per_step": s_l / args.steps, "ms_per_step": round(s_ms / args.steps, 3)},
        "roofline": {"bound": "mfma" if mfma_bound else "hbm", "kernel": kname, "launches_per_step": n_l / args.steps,
                     "avg_launch_us": round(ms_tot * 1e3 / n_l, 2),
                     "flops_per_launch": fl_tot / n_l, "algorithmic_bytes_per_launch": by_tot / n_l,
                     "flop_per_byte": round(ai, 1), "ridge_flop_per_byte": round(PEAK[prec_of] / PEAK_HBM, 1),
                     "achieved": round(achieved, 2), "peak": PEAK[prec_of] if mfma_bound else PEAK_HBM * 1e3,
                     "unit": "TFLOP/s" if mfma_bound else "GB/s",
                     "frac": round(achieved / (PEAK[prec_of] if mfma_bound else PEAK_HBM * 1e3), 4),
                     "roof_frac": round(roof_tot / ms_tot, 4), "traffic": traffic,
                     "sustained_peak": round(sustained, 1) if mfma_bound and prec_of == "bf16" else None,
                     "frac_of_sustained": round(achieved / sustained, 4) if mfma_bound and prec_of == "bf16" else None,
                     "clock_mhz": clk["mhz"],
                     "frac_at_clock": (round(achieved / ((PEAK[prec_of] if mfma_bound else PEAK_HBM * 1e3)
                                                         * clk["mhz"] / CLOCK_MHZ), 4)
                                       if clk["mhz"] and mfma_bound else None)},
        "clock": dict(clk, published_peak_mhz=CLOCK_MHZ, **{"pass": "the single-stream per-launch pass"}),
        "read_rate_tbps": dict(rates, hbm_published=PEAK_HBM),
        "launch_classes": launch_classes(recs, args.steps, peak),
        "kernels": {L.kernel_name(k): {"launches_per_step": v[0] / args.steps, "ms_per_step": round(v[1] / args.steps, 3),
                                       "tflops": round(v[2] / (v[1] * 1e-3) / 1e12, 2),
                                       "roof_frac": round(v[4] / v[1], 4)} for k, v in agg.items()},
    }
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.precision, skew, args.cpu_seconds)
    else:
        out["cpu_baseline"] = None
    return out


def bench_gemm(args):
    """One launch shape of the dominant kernel class, for counter runs: 12 problems of C = A B^T with A, B 3072 x 3072
    bf16 (k contiguous) and fp32 C, launched `steps` times after `warmup`; the engine clock over the timed launches."""
    import torch
    from psgd_pro_amd import _lib as L
    dev = torch.device("cuda:0")
    clock = ClockSampler(dev)
    m = n = k = 3072
    nb = 12
    gen = torch.Generator(device=dev).manual_seed(0)
    A = [torch.randn(m, k, device=dev, generator=gen).to(torch.bfloat16) for _ in range(nb)]
    B = [torch.randn(n, k, device=dev, generator=gen).to(torch.bfloat16) for _ in range(nb)]
    Cs = [torch.empty(m, n, device=dev) for _ in range(nb)]
    stream = torch.cuda.current_stream()
    st = C.c_void_p(stream.cuda_stream)
    f = lambda: L.check(L.lib().psgdk_gemm(1, 0, 1, m, n, k, 1.0, 1, 1, nb, L.ptrs(A), k, L.ptrs(B), k, 0.0,
                                           L.ptrs(Cs), n, st))
    for _ in range(max(1, args.warmup)):
        f()
    torch.cuda.synchronize()
    clock.arm(stream, est_ms=args.steps * 1.2 + 20)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
    clock.start()
    ev[0].record(stream)
    for _ in range(args.steps):
        f()
    ev[1].record(stream)
    clock.stop()
    clk = clock.result()
    us = ev[0].elapsed_time(ev[1]) * 1e3 / args.steps
    tf = 2.0 * m * n * k * nb / (us * 1e-6) / 1e12
    return {"op": "gemm_bf16", "m": m, "n": n, "k": k, "nb": nb, "launches": args.steps, "us": round(us, 1),
            "tflops": round(tf, 1), "frac": round(tf / PEAK["bf16"], 4), "clock_mhz": clk["mhz"],
            "frac_at_clock": round(tf / (PEAK["bf16"] * clk["mhz"] / CLOCK_MHZ), 4) if clk["mhz"] else None}


def bench_syrk(args):
    """SYRK C = triu(A A^T) (A n x k, n = k) and TRMM triu(Q) B microbenchmarks, fp32 and bf16 inputs."""
    import torch
    from psgd_pro_amd import _lib as L
    lines = []
    dev = torch.device("cuda:0")
    st = L.stream_of(torch.empty(1, device=dev))
    for prec, name in ((1, "bf16"), (0, "fp32")):
        dt = torch.bfloat16 if prec else torch.float32
        for n in (512, 1024, 2048, 4096):
            A = torch.randn(n, n, device=dev).to(dt)
            C = torch.empty(n, n, device=dev)
            adt = L.dtype_code(dt)

            def syrk(stream=st):
                L.check(L.lib().psgdk_syrk(prec, 0, L.OUT_UPPER, n, n, adt, 1, L.ptrs([A]), n, L.ptrs([C]), n,
                                           stream))
            for _ in range(3):
                syrk()
            torch.cuda.synchronize()
            reps = max(20, int(2e10 / (n ** 3)))
            # us: back-to-back launches between two events (the per-launch event pairs of the library's profiler,
            # event_us, add a few microseconds of their own to a small launch)
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            ev[0].record()
            for _ in range(reps):
                syrk()
            ev[1].record()
            torch.cuda.synchronize()
            ms = ev[0].elapsed_time(ev[1]) / reps
            L.profile_start()
            for _ in range(reps):
                syrk()
            recs = L.profile_stop()
            ms_ev = sum(r[3] for r in recs) / len(recs)
            tf = n * (n + 1) * n / (ms * 1e-3) / 1e12
            lines.append({"op": "syrk", "n": n, "k": n, "dtype": name, "us": round(ms * 1e3, 2),
                          "tflops": round(tf, 2), "frac": round(tf / PEAK[name], 4), "event_us": round(ms_ev * 1e3, 2)})
            B = torch.randn(n, n, device=dev)
            Af = A.float()
            ws = L.Workspace()

            def trmm():
                L.call_ws(L.lib().psgdk_trmm_ws, prec, n, n, 0, 1, L.ptrs([Af]), n, L.ptrs([B]), n, L.ptrs([C]), n,
                          ws=ws, device=dev, stream=st)
            for _ in range(3):
                trmm()
            torch.cuda.synchronize()
            # back-to-back whole calls (operand copies + product) between two events, and the product alone from the
            # library's per-launch events
            ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]
            L.profile_start()
            ev[0].record()
            for _ in range(reps):
                trmm()
            ev[1].record()
            torch.cuda.synchronize()
            recs = L.profile_stop()
            ms = ev[0].elapsed_time(ev[1]) / reps
            ms_mm = sum(r[3] for r in recs) / len(recs)
            tf = n * n * (n + 1) / (ms * 1e-3) / 1e12
            lines.append({"op": "trmm", "n": n, "dtype": name, "us": round(ms * 1e3, 2), "tflops": round(tf, 2),
                          "frac": round(tf / PEAK[name], 4), "product_us": round(ms_mm * 1e3, 2),
                          "note": "us: whole psgdk_trmm_ws call (triu(Q) and B^T copies + product)"})
    return lines


def bench_llama(args):
    """Llama-class shapes: one 4096 x 4096 and one 4096 x 14336 weight, bf16 gradients, every factor dense
    (max_size 16384, max_skew inf), fp32 factors, bf16 MFMA path, update every step."""
    import torch
    from psgd_pro_amd.flops import flops_2d
    from psgd_pro_amd import KronWhiten
    from psgd_pro_amd import _lib as L
    dev = torch.device("cuda:0")
    shapes = [(4096, 4096), (4096, 14336)]
    gen = torch.Generator().manual_seed(0)
    params = [(0.02 * torch.randn(s, generator=gen)).to(dev).requires_grad_(True) for s in shapes]
    grads = [(0.01 * torch.randn(s, generator=gen)).to(torch.bfloat16).to(dev) for s in shapes]
    opt = KronWhiten(params, preconditioner_max_size=16384, preconditioner_max_skew=math.inf,
                     preconditioner_init_scale=1.0, precision=args.precision, draws="device", seed=0,
                     streams=args.streams, graphs=bool(args.graphs))
    flops_step = sum(flops_2d(m, n, True, True) for m, n in shapes)
    steps, warmup = min(args.steps, 10), min(args.warmup, 3)
    for _ in range(warmup):
        opt.step_math(grads)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        opt.step_math(grads)
    torch.cuda.synchronize()
    ms = (time.perf_counter() - t0) * 1e3 / steps
    check_finite(opt, params)
    opt._nstreams = 0
    L.check(L.lib().psgdk_set_option(6, 0))  # one stream: each launch's event time is its own
    L.profile_start()
    for _ in range(2):
        opt.step_math(grads)
    torch.cuda.synchronize()
    recs = L.profile_stop()
    L.check(L.lib().psgdk_set_option(6, args.upd_streams))
    opt._nstreams = args.streams
    return {"metric": "Kron update+apply ms/step at Llama shapes (4096x4096 + 4096x14336), 1 GPU", "value": round(ms, 3),
            "unit": "ms/step", "steps": steps, "warmup": warmup, "higher_is_better": False, "dtype": args.precision,
            "data": "synthetic", "config": {"workload": "llama-4096x4096+4096x14336-kron-update-apply",
                                            "max_size": 16384, "max_skew": "inf", "streams": opt.side_streams()},
            "algorithmic_tflop_per_step": round(flops_step / 1e12, 3),
            "tflops": round(flops_step / (ms * 1e-3) / 1e12, 2),
            "launch_classes": launch_classes(recs, 2, PEAK[args.precision], top=8)}


def _vit(dim=512, depth=6, heads=8, dim_head=64, mlp=1024, patch=4, image=32, classes=10):
    """A ViT of vit_pro.py's architecture (vit_pro.py:76-226: pre-norm attention and MLP blocks, patch embedding
    with LayerNorms, class token, learned positions, final LayerNorm, class-token head). The attention products
    run in float32 on contiguous operands outside autocast; the Linear layers run under bf16 autocast."""
    import torch
    from torch import nn

    class Attention(nn.Module):
        def __init__(self):
            super().__init__()
            inner = heads * dim_head
            self.norm = nn.LayerNorm(dim)
            self.to_qkv = nn.Linear(dim, 3 * inner, bias=False)
            self.to_out = nn.Linear(inner, dim)

        def forward(self, x):
            b, n, _ = x.shape
            qkv = self.to_qkv(self.norm(x)).reshape(b, n, 3, heads, dim_head).permute(2, 0, 3, 1, 4)
            with torch.autocast("cuda", enabled=False):
                q, k, v = (t.float().contiguous() for t in qkv)
                att = torch.matmul(q, k.transpose(-1, -2).contiguous()) * dim_head ** -0.5
                out = torch.matmul(att.softmax(dim=-1), v)
            return self.to_out(out.permute(0, 2, 1, 3).reshape(b, n, heads * dim_head))

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.attn = Attention()
            self.ff = nn.Sequential(nn.LayerNorm(dim), nn.Linear(dim, mlp), nn.GELU(), nn.Linear(mlp, dim))

        def forward(self, x):
            x = self.attn(x) + x
            return self.ff(x) + x

    class ViT(nn.Module):
        def __init__(self):
            super().__init__()
            pdim = 3 * patch * patch
            self.np = (image // patch) ** 2
            self.embed = nn.Sequential(nn.LayerNorm(pdim), nn.Linear(pdim, dim), nn.LayerNorm(dim))
            self.pos = nn.Parameter(torch.randn(1, self.np + 1, dim))
            self.cls = nn.Parameter(torch.randn(1, 1, dim))
            self.blocks = nn.ModuleList([Block() for _ in range(depth)])
            self.norm = nn.LayerNorm(dim)
            self.head = nn.Linear(dim, classes)

        def forward(self, img):
            b, h = img.shape[0], image // patch
            x = img.reshape(b, 3, h, patch, h, patch).permute(0, 2, 4, 3, 5, 1).reshape(b, h * h, -1)
            x = self.embed(x)
            x = torch.cat([self.cls.expand(b, 1, dim), x], dim=1) + self.pos
            for blk in self.blocks:
                x = blk(x)
            return self.head(self.norm(x)[:, 0])

    return ViT()


def bench_e2e(args):
    """Optimizer share of an end-to-end training step: the ViT above, batch 512 of synthetic 32 x 32 images and
    labels, bf16 autocast, KronWhiten with vit_pro.py's settings (max_skew 2, momentum 0.9, lr 1e-3, update every
    step). t_step = forward + backward + optimizer, t_opt = optimizer; medians of 50 steps after 10 warmup."""
    import statistics
    import torch
    from psgd_pro_amd import KronWhiten
    dev = torch.device("cuda:0")
    torch.manual_seed(0)
    model = _vit().to(dev)
    params = [p for p in model.parameters() if p.requires_grad]
    x = torch.randn(512, 3, 32, 32, device=dev)
    y = torch.randint(0, 10, (512,), device=dev)
    opt = KronWhiten(params, preconditioner_max_skew=2, lr_params=1e-3, preconditioner_update_probability=1.0,
                     momentum=0.9, precision=args.precision, streams=args.streams, graphs=bool(args.graphs))
    ev = [[torch.cuda.Event(enable_timing=True) for _ in range(3)] for _ in range(60)]
    losses = []
    for i in range(60):
        e = ev[i]
        e[0].record()
        with torch.autocast("cuda", dtype=torch.bfloat16):
            loss = torch.nn.functional.cross_entropy(model(x).float(), y)
        grads = torch.autograd.grad(loss, params)
        e[1].record()
        opt.step_math(grads)
        e[2].record()
        losses.append(loss.detach())
    torch.cuda.synchronize()
    t_step = [ev[i][0].elapsed_time(ev[i][2]) for i in range(10, 60)]
    t_opt = [ev[i][1].elapsed_time(ev[i][2]) for i in range(10, 60)]
    ms_step, ms_opt = statistics.median(t_step), statistics.median(t_opt)
    return {"metric": "optimizer share of an end-to-end ViT training step (t_opt / t_step), 1 GPU",
            "value": round(ms_opt / ms_step, 4), "unit": "fraction", "higher_is_better": False,
            "ms_step": round(ms_step, 3), "ms_opt": round(ms_opt, 3), "ms_fwd_bwd": round(ms_step - ms_opt, 3),
            "loss_first_last": [round(float(losses[0]), 4), round(float(losses[-1]), 4)],
            "dtype": args.precision, "data": "synthetic",
            "config": {"workload": "vit-dim512-depth6-heads8-mlp1024-patch4-batch512-e2e", "params": len(params),
                       "max_skew": 2, "momentum": 0.9, "streams": opt.side_streams(), "graphs": bool(args.graphs)}}


def bench_ceiling(args):
    """The bf16 GEMM ceiling of this GPU at the optimizer's shapes: hipBLASLt (torch.matmul, bf16 output) against
    the library's k-contiguous kernel (fp32 output) on the same operands; back-to-back launches between events."""
    import torch
    from psgd_pro_amd import _lib as L
    dev = torch.device("cuda:0")
    st = L.stream_of(torch.empty(1, device=dev))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(2)]

    def timeit(fn, reps=10):
        for _ in range(3):
            fn()
        torch.cuda.synchronize()
        ev[0].record()
        for _ in range(reps):
            fn()
        ev[1].record()
        torch.cuda.synchronize()
        return ev[0].elapsed_time(ev[1]) / reps * 1e3
    lines = []
    for nb, m, n, k in [(12, 3072, 3072, 3072), (16, 3072, 3072, 3072), (12, 768, 3072, 3072), (12, 768, 2304, 2304),
                        (1, 4096, 14336, 4096), (1, 8192, 8192, 8192), (1, 16384, 16384, 8192)]:
        A = torch.randn(nb, m, k, device=dev).to(torch.bfloat16)
        B = torch.randn(nb, n, k, device=dev).to(torch.bfloat16)
        Bt = B.transpose(1, 2).contiguous()  # k x n, as torch.matmul takes it
        C = torch.empty(nb, m, n, device=dev)
        fl = 2.0 * nb * m * n * k
        t_blas = timeit(lambda: torch.matmul(A, Bt))
        t_ours = timeit(lambda: L.check(L.lib().psgdk_gemm(1, 0, 1, m, n, k, 1.0, 1, 1, nb, L.ptrs(list(A)), k,
                                                           L.ptrs(list(B)), k, 0.0, L.ptrs(list(C)), n, st)))
        lines.append({"op": "gemm_bf16", "nb": nb, "m": m, "n": n, "k": k,
                      "hipblaslt_us": round(t_blas, 1), "hipblaslt_tflops": round(fl / t_blas / 1e6, 1),
                      "psgdk_us": round(t_ours, 1), "psgdk_tflops": round(fl / t_ours / 1e6, 1),
                      "psgdk_over_hipblaslt": round(t_blas / t_ours, 3), "peak": PEAK["bf16"]})
        del A, B, Bt, C
        torch.cuda.empty_cache()
    return lines


def bench_copy(args):
    """Calibration for the HBM counters: one device-to-device copy of 256 MiB (read 256 MiB, write 256 MiB)."""
    import torch
    n = 64 * 1024 * 1024
    x = torch.randn(n, device="cuda:0")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(3):
        y.copy_(x)
    torch.cuda.synchronize()
    return {"op": "copy", "bytes_read": 4 * n, "bytes_written": 4 * n, "launches": 3}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: measures one GPU only (--gpus {args.gpus} requested); the preconditioner would shard by "
              f"parameter across GPUs, which is not implemented in psgd_pro_amd.", file=sys.stderr)
        sys.exit(2)
    if args.graphs:
        print("bench.py: --graphs 1 is refused: replaying the step from a captured HIP graph is switched off (a capture "
              "of the step aborted the process and the cause is not established)", file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        sys.exit(1)
    if args.opt:
        from psgd_pro_amd import _lib as L
        for kv in args.opt:
            k, v = kv.split("=")
            L.check(L.lib().psgdk_set_option(int(k), int(v)))
    if args.config == "copy":
        print(json.dumps(bench_copy(args)), flush=True)
        return
    if args.config == "e2e":
        print(json.dumps(bench_e2e(args)), flush=True)
        return
    if args.config == "llama":
        print(json.dumps(bench_llama(args)), flush=True)
        return
    if args.config == "gemm":
        print(json.dumps(bench_gemm(args)), flush=True)
        return
    if args.config == "syrk":
        for ln in bench_syrk(args):
            print(json.dumps(ln), flush=True)
        return
    if args.config == "ceiling":
        for ln in bench_ceiling(args):
            print(json.dumps(ln), flush=True)
        return
    print(json.dumps(bench_vitb(args)), flush=True)


if __name__ == "__main__":
    main()
