#!/usr/bin/env python3
"""Benchmark: SSD prefill tok/s + GFLOP/s at L=8192 H=64 P=64 N=128 G=8 seq=1.

One step = one HELIX scan (Pass A, B, C) over BASELINE.json config 2 with
inputs resident in HBM, on the bf16 path (bf16 Pass C operands; Pass A on
bf16x6 split products, which keeps the carried state and s1 fp32-accurate as
the reference requires; fp32 Pass B). The same workload is also timed on the
fp32 path. Timing follows
the reference protocol (docs/BENCHMARKING.md:48-69): wall-clock warm-up of at
least 800 ms, events on the launch stream, min / median / spread reported.

Prints ONE JSON line. value = tokens/s of the whole job (one GPU).
"""
from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

import torch  # noqa: E402

from helix_amd.abi import Context  # noqa: E402
from helix_amd.desc import (HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA, HELIX_OK,  # noqa: E402
                            algorithmic_bytes, algorithmic_flops)
from helix_amd.scan import make_desc, tensor_arg  # noqa: E402

METRIC = "SSD prefill tok/s + GFLOP/s at L=8192 H=64 P=64 N=128 seq=1; % roofline"
# MI355X published peaks.
PEAK_HBM = 8.0e12           # B/s
PEAK_FP32_MFMA = 157.3e12   # FLOP/s
PEAK_BF16_MFMA = 2516.6e12  # FLOP/s (dense)
# Reference's published number for this metric and path: 3-pass + bf16 Pass C
# on an Apple M5 Max (reference README.md:96-98).
REF_TOKS = 1315051.0

CFG = dict(L=8192, S=1, H=64, P=64, N=128, G=8)
ARENA_BYTES = 4 << 30   # the headline workload's inputs, outputs and scratch fit
Y_PLACES, Y_STEP = 4, 1 << 20   # y placements timed for the headline (1 MiB apart)
COLD_FLUSH_BYTES = 1 << 30      # a copy of this size evicts the 256 MB Infinity Cache

# BASELINE.json's configurations (config 4 in its two head-dim variants): shape,
# the paths each is quoted on, and the distributions that differ from the common
# ones (h0 standard deviation, dt_raw mean and standard deviation).
CONFIGS = [
    dict(name="0", L=256, S=1, H=8, P=64, N=64, G=1, paths=("fp32",)),
    dict(name="1", L=2048, S=1, H=64, P=64, N=128, G=8, paths=("fp32",)),
    dict(name="2", L=8192, S=1, H=64, P=64, N=128, G=8, paths=("bf16", "fp32")),
    dict(name="3", L=1000, S=4, H=32, P=128, N=128, G=1, paths=("fp32",), s0_sigma=0.1,
         dt_mu=-2.0, dt_sigma=1.0),
    dict(name="4a", L=4096, S=8, H=80, P=64, N=128, G=1, paths=("bf16",), s0_sigma=0.1),
    dict(name="4b", L=4096, S=8, H=27, P=192, N=128, G=1, paths=("bf16",), s0_sigma=0.1),
]


def make_inputs(seed: int, dev, cfg=None):
    """BASELINE.json distributions at a config's shape (config 2 by default),
    generated on the device."""
    cfg = cfg or dict(CFG)
    L, S, H, P, N, G = (cfg[k] for k in "LSHPNG")
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    x = torch.randn((S, L, H, P), generator=g, device=dev)
    dt = cfg.get("dt_mu", -1.0) + cfg.get("dt_sigma", 0.5) * torch.randn((S, L, H), generator=g, device=dev)
    A = -torch.exp(math.log(1.0) + (math.log(16.0) - math.log(1.0))
                   * torch.rand((H,), generator=g, device=dev))
    B = torch.randn((S, L, G, N), generator=g, device=dev) / math.sqrt(N)
    C = torch.randn((S, L, G, N), generator=g, device=dev) / math.sqrt(N)
    s0 = cfg.get("s0_sigma", 0.0) * torch.randn((S, H, P, N), generator=g, device=dev)
    return x, dt, A, B, C, s0


def as_storage(tensors, dtype):
    """x, B and C rounded to a 16-bit storage type (io_dtype); dt, A, s0 stay fp32."""
    x, dt, A, B, C, s0 = tensors
    return x.to(dtype), dt, A, B.to(dtype), C.to(dtype), s0


class Variant:
    def __init__(self, name, ctx, backend, tensors, env=None, multipass=True):
        self.name = name
        self.env = env or {}
        self.multipass = multipass
        saved = self._push()
        # A context reads its tuning knobs when it is created: a variant with
        # its own environment gets its own context.
        self.ctx = Context(torch.cuda.current_device()) if self.env else ctx
        ctx = self.ctx
        x, dt, A, B, C, s0 = tensors
        self.y = torch.empty_like(x)
        self.s1 = torch.empty_like(s0)
        self.d = make_desc(x, dt, B, C, s0, self.y, A, multipass=multipass)
        self.d.backend = backend
        assert ctx.supported(self.d), ctx.backend_desc(self.d)
        self.kernel = ctx.backend_desc(self.d)
        self.plan = ctx.plan_info(self.d)
        self.scratch = torch.empty(max(1, ctx.scratch_size(self.d)), dtype=torch.uint8,
                                   device=x.device)
        self.args = [tensor_arg(t) for t in (s0, x, dt, A, B, C)]
        self._pop(saved)

    def _push(self):
        saved = {k: os.environ.get(k) for k in self.env}
        os.environ.update(self.env)
        return saved

    def _pop(self, saved):
        for k, v in saved.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v

    def encode(self, stream):
        s0, x, dt, A, B, C = self.args
        rc = self.ctx.encode(stream.cuda_stream, self.d, s0, x, dt, A, B, C, tensor_arg(None),
                             tensor_arg(self.y), tensor_arg(self.s1), tensor_arg(self.scratch))
        if rc != HELIX_OK:
            raise RuntimeError(f"{self.name}: encode failed {rc}: {self.ctx.last_error()}")


def time_variant(v: Variant, steps: int, stream, only: str | None = None):
    """Per-step event times (ms) of `steps` encodes; HELIX_ONLY_PASS=only if set."""
    if only:
        os.environ["HELIX_ONLY_PASS"] = only
    try:
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in range(steps)]
        torch.cuda.synchronize()
        for a, b in evs:
            a.record(stream)
            v.encode(stream)
            b.record(stream)
        torch.cuda.synchronize()
        return [a.elapsed_time(b) for a, b in evs]
    finally:
        os.environ.pop("HELIX_ONLY_PASS", None)


def time_placements(v: Variant, steps: int, stream, ys):
    """Per-step event times (ms) of `steps` whole scans, step i writing y at
    ys[i % len(ys)] (the same output at other addresses). Returns the per-step
    times and, per placement, the times of its steps."""
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    y0 = v.y
    try:
        torch.cuda.synchronize()
        for i, (a, b) in enumerate(evs):
            v.y = ys[i % len(ys)]
            a.record(stream)
            v.encode(stream)
            b.record(stream)
        torch.cuda.synchronize()
    finally:
        v.y = y0
    ts = [a.elapsed_time(b) for a, b in evs]
    return ts, [ts[k::len(ys)] for k in range(len(ys))]


def time_cold(v: Variant, steps: int, stream, flush_bytes: int):
    """Per-step event times (ms) of `steps` whole scans, each preceded, outside
    its events, by a device copy of `flush_bytes` that evicts the 256 MB
    Infinity Cache: the scan then reads its inputs from HBM, as a first call
    on them would."""
    src = torch.empty(flush_bytes, dtype=torch.uint8, device=v.y.device)
    dst = torch.empty_like(src)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    torch.cuda.synchronize()
    for a, b in evs:
        dst.copy_(src)
        a.record(stream)
        v.encode(stream)
        b.record(stream)
    torch.cuda.synchronize()
    return [a.elapsed_time(b) for a, b in evs]


def time_passes(v: Variant, steps: int, stream):
    """Per-pass event times (ms): each step encodes Pass A, B and C as three
    single-pass encodes in a row (HELIX_ONLY_PASS), each between two events
    on the launch stream, so every pass runs in the same order, and on the
    same cache state, as inside a whole scan. A fourth, empty encode
    (HELIX_ONLY_PASS=X launches nothing) between two events measures what
    the event pair itself adds ('X'); pass_us() subtracts it."""
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in "ABCX"]
           for _ in range(steps)]
    try:
        torch.cuda.synchronize()
        for step in evs:
            for k, (a, b) in zip("ABCX", step):
                os.environ["HELIX_ONLY_PASS"] = k
                a.record(stream)
                v.encode(stream)
                b.record(stream)
        torch.cuda.synchronize()
    finally:
        os.environ.pop("HELIX_ONLY_PASS", None)
    return {k: [step[i][0].elapsed_time(step[i][1]) for step in evs] for i, k in enumerate("ABCX")}


def time_in_scan(v: Variant, steps: int, stream):
    """Each pass's time inside whole scans (ms per step): every step encodes
    the whole scan and then the scan without one pass (HELIX_ONLY_PASS=BC, AC,
    AB), each between two events, and a pass's time is the difference of the
    two means. Unlike the single-pass split this keeps each pass in the cache
    state the scan leaves it (what rocprofv3's kernel trace of the same run
    averages, since whole scans dominate its calls); it includes the pass's
    launch gap."""
    drop = {"A": "BC", "B": "AC", "C": "AB"}
    live = [k for k in "ABC" if k != "B" or v.plan.kernel_b]
    evs = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(2)]
           for _ in range(steps * len(live))]
    try:
        torch.cuda.synchronize()
        i = 0
        for _ in range(steps):
            for k in live:
                for j, only in enumerate((None, drop[k])):
                    if only:
                        os.environ["HELIX_ONLY_PASS"] = only
                    else:
                        os.environ.pop("HELIX_ONLY_PASS", None)
                    a, b = evs[i][j]
                    a.record(stream)
                    v.encode(stream)
                    b.record(stream)
                i += 1
        torch.cuda.synchronize()
    finally:
        os.environ.pop("HELIX_ONLY_PASS", None)
    out = {}
    for n, k in enumerate(live):
        pairs = evs[n::len(live)]
        full = statistics.fmean(p[0][0].elapsed_time(p[0][1]) for p in pairs)
        part = statistics.fmean(p[1][0].elapsed_time(p[1][1]) for p in pairs)
        out[k] = (full - part) * 1e3
    return out


def pass_us(passes, stat="median"):
    """Per-pass kernel time (us): the pass's event-bracketed time less that
    of an empty encode between the same two events."""
    x = dist(passes["X"])[stat]
    return {k: max(0.0, dist(ts)[stat] - x) * 1e3 for k, ts in passes.items() if k != "X"}


def pass_algorithmic_bytes(plan):
    """Bytes each pass must move once at config 2 on the bf16 path (the
    scratch it writes or reads included, since the pass cannot avoid it)."""
    L, S, H, P, N, G = (CFG[k] for k in "LSHPNG")
    x = y = S * L * H * P * 4
    dt = S * L * H * 4
    bc = S * L * G * N * 4
    state = S * H * P * N * 4
    # With bf16 copies of B and C, Pass A also reads C and writes both copies,
    # and Pass C reads the copies instead.
    cp = plan.bccopy_bytes
    # With Pass B run by the walking Pass C (no kernel_b), Pass C also reads s0
    # and writes s1; the segment aggregates are read once either way. Pass A
    # writes the per-token decay records, which Pass C reads instead of dt.
    fused = not plan.kernel_b
    rec = plan.rec_bytes
    # Pass B stores, and a walking Pass C reads, the start states of the walks
    # only (one per walk_len chunks); off the walk, every segment's.
    starts = state * plan.walks_per_group if plan.walk_len != plan.seg_len else plan.s_seg_bytes
    return {
        "A": x + dt + bc + plan.s_local_bytes + plan.s_seg_bytes + ((bc + cp) if cp else 0) + rec,
        "B": 0 if fused else plan.s_seg_bytes + starts + 2 * state,
        "C": x + (rec if rec else dt) + (cp if cp else 2 * bc) + plan.s_local_bytes
             + (plan.s_seg_bytes if fused else starts) + y + (2 * state if fused else 0),
    }


def profiled_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 summary
    (FETCH_SIZE + WRITE_SIZE, calibrated against a plain copy), or None when
    the summary has no row for it."""
    path = os.path.join(ROOT, "profiles", "kernels_cfg2.md")
    try:
        with open(path) as fh:
            for line in fh:
                cells = [c.strip() for c in line.strip().strip("|").split("|")]
                if len(cells) >= 5 and cells[0] == kernel:
                    return (float(cells[3]) + float(cells[4])) * 2**20
    except (OSError, ValueError):
        pass
    return None


def dist(ts):
    s = sorted(ts)
    return {"min": s[0], "median": s[len(s) // 2], "mean": statistics.fmean(s), "max": s[-1],
            "spread": s[-1] / s[0]}


def cpu_baseline(budget_s: float = 20.0):
    """fp64 sequential scan on the host cores, on a bounded head sample of the
    same workload (heads are independent, so per-head cost scales exactly).
    Prefers the reference's own build (oracle/_ref, 1 thread, like its
    ref::scan); also times this repo's C port on all host cores."""
    import numpy as np  # noqa: F401
    from oracle import pyoracle as po

    L, S, H, P, N, G = (CFG[k] for k in "LSHPNG")
    out = {}
    # One head of config 2 (same per-head work as the full problem).
    p1 = po.problem_gauss(L, S, 1, P, N, 1, 1002)
    n_heads = 0
    t_tot = 0.0
    use_ref = po.ref_lib() is not None
    while t_tot < budget_s * 0.5 and n_heads < H:
        t0 = time.perf_counter()
        if use_ref:
            po.ref_scan(p1)
        else:
            po.scan(p1)
        t_tot += time.perf_counter() - t0
        n_heads += 1
    per_head = t_tot / n_heads
    F = algorithmic_flops(L, S, H, P, N)
    out["cpu_baseline"] = {
        "value": S * L / (per_head * H), "unit": "tok/s", "cores": 1,
        "gflops": F / (per_head * H) / 1e9,
        "kind": "reference" if use_ref else "port",
        "sample": f"{n_heads} of {H} heads of config 2 (L={L}), fp64 sequential "
                  f"{'ref::scan from oracle/_ref' if use_ref else 'oracle_scan'}, 1 thread, "
                  f"{t_tot:.1f} s; tok/s scaled to all {H} heads",
    }
    ncpu = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else os.cpu_count()
    nh = min(H, max(ncpu, 1) * 2)
    pm = po.problem_gauss(L, S, nh, P, N, 1, 1002)
    t0 = time.perf_counter()
    po.scan(pm, threads=ncpu)
    tm = time.perf_counter() - t0
    out["cpu_baseline_mt"] = {
        "value": S * L / (tm * H / nh), "unit": "tok/s", "cores": ncpu, "kind": "port",
        "gflops": F / (tm * H / nh) / 1e9,
        "sample": f"{nh} of {H} heads of config 2, fp64 sequential oracle_scan_mt on "
                  f"{ncpu} threads (os.sched_getaffinity), {tm:.1f} s; scaled to {H} heads",
        "hardware_concurrency": os.cpu_count(),
    }
    return out


def config_report(ctx, stream, dev, steps: int, warm_ms: float, names=None):
    """Every BASELINE config on each path it is quoted on: tokens/s, GFLOP/s,
    fraction of the op roofline and the per-pass split (medians of `steps`
    event-timed encodes after `warm_ms` of warm-up). The roofline rule is the
    headline's: max(F_A/fp32_peak + F_C/P_C, alg_bytes/8 TB/s), P_C the bf16
    peak on the bf16 path and the fp32 peak on the fp32 path."""
    out = {}
    for i, cfg in enumerate(CONFIGS):
        if names and cfg["name"] not in names:
            continue
        L, S, H, P, N, G = (cfg[k] for k in "LSHPNG")
        tensors = make_inputs(1000 + i, dev, cfg)
        F = algorithmic_flops(L, S, H, P, N)
        F_A = 2.0 * S * H * ((L + 63) // 64) * 64 * N * P
        nbytes = algorithmic_bytes(L, S, H, P, N, G)
        for path in cfg["paths"]:
            v = Variant(path, ctx, HELIX_BACKEND_MPP if path == "bf16" else HELIX_BACKEND_SGMMA, tensors)
            for _ in range(3):
                v.encode(stream)
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            while (time.perf_counter() - t0) * 1e3 < warm_ms:
                v.encode(stream)
                torch.cuda.synchronize()
            ms = dist(time_variant(v, steps, stream))["median"]
            passes = time_passes(v, steps, stream)
            peak_c = PEAK_BF16_MFMA if path == "bf16" else PEAK_FP32_MFMA
            t_roof = max(F_A / PEAK_FP32_MFMA + (F - F_A) / peak_c, nbytes / PEAK_HBM)
            out[f"{cfg['name']}/{path}"] = {
                "shape": f"S={S} L={L} H={H} P={P} N={N} G={G}",
                "tok_s": S * L / (ms * 1e-3), "gflops": F / (ms * 1e-3) / 1e9, "ms": ms,
                "roofline_frac": t_roof / (ms * 1e-3), "t_roof_us": t_roof * 1e6,
                "passes_us": {k: us for k, us in pass_us(passes).items() if k != "B" or v.plan.kernel_b},
                "plan": {"groups": v.plan.n_groups, "seg_len": v.plan.seg_len},
            }
            del v
        del tensors
        torch.cuda.empty_cache()
    return out


IMPLS = {
    # name: (backend, multipass), the reference bench's --impl names
    # (bench/bench_scan.mm:128-140): "3pass" leaves the backend to AUTO (the
    # bf16 path here), the suffixes pin the fp32 (SGMMA) or bf16 (MPP) Pass C.
    "1pass": (HELIX_BACKEND_AUTO, False),
    "3pass": (HELIX_BACKEND_AUTO, True),
    "3pass-sgmma": (HELIX_BACKEND_SGMMA, True),
    "3pass-mpp": (HELIX_BACKEND_MPP, True),
}


def shape_bench(args, dev):
    """The reference bench's per-shape mode (bench/bench_scan.mm:65-240): one
    problem of the given shape (BASELINE.json's distributions, seed 99), each
    implementation in --impl timed interleaved in this process after a
    wall-clock warm-up; per implementation the fastest and median scan,
    tok/s and GFLOP/s at the fastest, the max/min spread and the speed-up
    over 1pass. With --json, one JSON object per implementation."""
    cfg = dict(CFG)
    for k, a in (("L", args.L), ("S", args.n_seq), ("H", args.heads), ("P", args.head_dim), ("N", args.d_state),
                 ("G", args.groups)):
        if a is not None:
            cfg[k] = a
    L, S, H, P, N, G = (cfg[k] for k in "LSHPNG")
    tensors = make_inputs(99, dev, cfg)
    ctx = Context(0)
    stream = torch.cuda.current_stream(dev)
    variants = []
    for name in (args.impl or "1pass,3pass").split(","):
        if name not in IMPLS:
            print(f"bench.py: unknown impl {name!r} (one of {', '.join(IMPLS)})", file=sys.stderr)
            sys.exit(2)
        backend, multipass = IMPLS[name]
        try:
            variants.append(Variant(name, ctx, backend, tensors, multipass=multipass))
        except AssertionError:
            print(f"bench.py: shape unsupported for impl {name!r}", file=sys.stderr)
            sys.exit(1)
    t0 = time.perf_counter()
    rounds = 0
    while (time.perf_counter() - t0) * 1e3 < args.warmup_ms or rounds < 3:
        for v in variants:
            v.encode(stream)
        torch.cuda.synchronize()
        rounds += 1
    times = {v.name: [] for v in variants}
    for _ in range(args.iters):
        for v in variants:
            times[v.name] += time_variant(v, 1, stream)
    F = algorithmic_flops(L, S, H, P, N)
    base = min(times["1pass"]) if "1pass" in times else None
    if not args.json:
        print(f"L={L} H={H} P={P} N={N} G={G} seq={S}")
        print(f"  {'impl':12s} {'ms':>9s} {'median':>9s} {'tok/s':>13s} {'GFLOP/s':>10s} {'spread':>7s} {'vs 1pass':>8s}  kernels")
    for v in variants:
        d = dist(times[v.name])
        sec = d["min"] * 1e-3
        rel = base / d["min"] if base else None
        if args.json:
            print(json.dumps({"impl": v.name, "L": L, "n_seq": S, "heads": H, "head_dim": P, "d_state": N,
                              "n_group": G, "ms": d["min"], "ms_median": d["median"], "spread": d["spread"],
                              "tok_per_s": L * S / sec, "gflops": F / sec * 1e-9, "speedup_vs_1pass": rel,
                              "kernel": v.kernel}), flush=True)
        else:
            print(f"  {v.name:12s} {d['min']:9.4f} {d['median']:9.4f} {L * S / sec:13.0f} {F / sec * 1e-9:10.0f} "
                  f"{d['spread']:6.2f}x {('%.2fx' % rel) if rel else '-':>8s}  {v.kernel}", flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--warmup-ms", type=float, default=800.0)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--cpu-budget", type=float, default=20.0)
    ap.add_argument("--variants", nargs="?", const="all", default=None, metavar="NAMES",
                    help="also time alternative kernel choices (reported under 'variants'); "
                         "a comma list names which (default: all)")
    ap.add_argument("--config-steps", type=int, default=20,
                    help="event-timed encodes per config and path in the per-config report "
                         "(0 skips the report)")
    ap.add_argument("--only-config", default=None, metavar="NAME",
                    help="run only the per-config report of this BASELINE config (0 1 2 3 4a 4b) and "
                         "print it: a process of its own for profiling one configuration")
    ap.add_argument("--cold-steps", type=int, default=0, metavar="K",
                    help="also time K scans of the bf16 and fp32 paths, each after a 1 GiB copy "
                         "that evicts the Infinity Cache (reported as cold_cache)")
    ap.add_argument("--calib-copy", type=int, default=0, metavar="MiB",
                    help="also run a plain device copy of this size (a known-traffic kernel "
                         "that calibrates rocprofv3 FETCH_SIZE / WRITE_SIZE)")
    shape = ap.add_argument_group("per-shape mode (the reference bench's flags; any of them selects it)")
    shape.add_argument("--L", type=int, default=None, help="tokens per sequence")
    shape.add_argument("--n-seq", type=int, default=None)
    shape.add_argument("--heads", type=int, default=None)
    shape.add_argument("--head-dim", type=int, default=None)
    shape.add_argument("--d-state", type=int, default=None)
    shape.add_argument("--groups", type=int, default=None)
    shape.add_argument("--impl", default=None, help=f"comma list of {', '.join(IMPLS)} (default 1pass,3pass)")
    shape.add_argument("--iters", type=int, default=20)
    shape.add_argument("--json", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for --gpus {args.gpus}); "
              "the scan would shard by head or by sequence, with no collectives",
              file=sys.stderr)
        sys.exit(2)

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if any(a is not None for a in (args.L, args.n_seq, args.heads, args.head_dim, args.d_state, args.groups,
                                   args.impl)):
        shape_bench(args, dev)
        return
    ctx = Context(0)
    if args.only_config:
        stream = torch.cuda.current_stream(dev)
        rep = config_report(ctx, stream, dev, max(1, args.config_steps), args.warmup_ms, {args.only_config})
        if not rep:
            print(f"bench.py: no config named {args.only_config!r}", file=sys.stderr)
            sys.exit(2)
        print(json.dumps({"configs": rep}), flush=True)
        return
    # One device allocation for the whole workload, as a serving runtime's
    # arena: torch's caching allocator keeps this block and carves the
    # inputs, outputs and scratch out of it. Separate allocations made the
    # first variant's scan up to 7 us slower than an identical later one
    # (where x and the scratch land decides what stays in the Infinity Cache
    # between Pass A and Pass C); inside one block the two agree to ~1.5 us.
    _arena = torch.empty(ARENA_BYTES, dtype=torch.uint8, device=dev)
    del _arena
    tensors = make_inputs(1002, dev)
    stream = torch.cuda.current_stream(dev)
    # The headline (bf16 path), the fp32 path, and the single pass
    # (multipass = false, the descriptor default: by default the fp32 path's
    # passes with their state tiles in y, no scratch).
    variants = [Variant("bf16", ctx, HELIX_BACKEND_MPP, tensors),
                Variant("fp32", ctx, HELIX_BACKEND_SGMMA, tensors),
                Variant("single-pass", ctx, HELIX_BACKEND_AUTO, tensors, multipass=False)]
    if args.variants:
        # Alternative kernel choices, timed interleaved in the same process
        # (--variants alone: all of them; --variants a,b: those named).
        wanted = None if args.variants == "all" else set(args.variants.split(","))
        n0 = len(variants)
        # The single pass's one-launch kernel (what it falls back to when y
        # overlaps an input).
        variants.append(Variant("single-pass-1launch", ctx, HELIX_BACKEND_AUTO, tensors, multipass=False,
                                env={"HELIX_1PASS_Y": "0"}))
        variants.append(Variant("bf16-storage", ctx, HELIX_BACKEND_MPP, as_storage(tensors, torch.bfloat16)))
        variants.append(Variant("bf16-passA-x3-optin", ctx, HELIX_BACKEND_MPP, tensors,
                                env={"HELIX_PASSA_SPLIT": "3"}))
        variants.append(Variant("bf16-passA-x6", ctx, HELIX_BACKEND_MPP, tensors,
                                env={"HELIX_PASSA_F16": "0"}))
        variants.append(Variant("bf16-copies", ctx, HELIX_BACKEND_MPP, tensors,
                                env={"HELIX_WALK_BCCOPY": "1"}))
        # The fp32 path at d_state 64 (config 2's shape otherwise): the walk
        # (default) against the chunk-parallel Pass C on stored states.
        t64 = make_inputs(1010, dev, dict(CFG, N=64))
        variants.append(Variant("fp32-dstate64-walk", ctx, HELIX_BACKEND_SGMMA, t64))
        variants.append(Variant("fp32-dstate64-chunk", ctx, HELIX_BACKEND_SGMMA, t64,
                                env={"HELIX_F32_WALK": "0"}))
        if wanted is not None:
            unknown = wanted - {v.name for v in variants[n0:]}
            if unknown:
                print(f"bench.py: unknown variant(s) {sorted(unknown)}", file=sys.stderr)
                sys.exit(2)
            variants = variants[:n0] + [v for v in variants[n0:] if v.name in wanted]

    def warm_up(v, ms):
        """W steps, then more until the wall clock has run `ms` (the
        reference's protocol against clock ramps). Each variant is warmed
        right before it is timed, on its own: alternating variants would hand
        each timed pass another variant's cache state."""
        for _ in range(args.warmup):
            v.encode(stream)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        while (time.perf_counter() - t0) * 1e3 < ms:
            v.encode(stream)
            torch.cuda.synchronize()

    L, S, H, P, N, G = (CFG[k] for k in "LSHPNG")
    F = algorithmic_flops(L, S, H, P, N)
    nch = (L + 63) // 64
    F_A = 2.0 * S * H * nch * 64 * N * P
    F_C = F - F_A
    bytes_alg = algorithmic_bytes(L, S, H, P, N, G)
    # Where the caller's y lands in memory is the caller's choice: the timed
    # steps of the two paths write y at Y_PLACES placements 1 MiB apart within
    # one 4 MiB window (the same output tensor shifted), one placement per step
    # in turn, and the reported time is the median over placements of each
    # placement's mean.
    y_bytes = variants[0].y.numel() * 4
    y_pool = torch.empty(y_bytes + (Y_PLACES - 1) * Y_STEP + 4096, dtype=torch.uint8, device=dev)
    ys = [y_pool[k * Y_STEP:k * Y_STEP + y_bytes].view(torch.float32).view(variants[0].y.shape)
          for k in range(Y_PLACES)]
    results = {}
    for i, v in enumerate(variants):
        warm_up(v, args.warmup_ms if i == 0 else min(args.warmup_ms, 200.0))
        # Whole op: K steps bracketed by synchronize; per-step events too.
        torch.cuda.synchronize()
        w0 = time.perf_counter()
        place = None
        if v.name in ("bf16", "fp32"):
            ts, per_place = time_placements(v, args.steps, stream, ys)
            place = [statistics.fmean(t) for t in per_place]
        else:
            ts = time_variant(v, args.steps, stream)
        torch.cuda.synchronize()
        wall = (time.perf_counter() - w0) / args.steps * 1e3
        # Per-pass split (HELIX_ONLY_PASS) exists only for the multipass path.
        passes = time_passes(v, args.steps, stream) if v.multipass else None
        in_scan = time_in_scan(v, args.steps, stream) if v.multipass and v.name == "bf16" else None
        d = dist(ts)
        ms = statistics.median(place) if place else statistics.fmean(ts)
        peak_c = PEAK_BF16_MFMA if v.name == "bf16" else PEAK_FP32_MFMA
        t_roof = max(F_A / PEAK_FP32_MFMA + F_C / peak_c, bytes_alg / PEAK_HBM)
        results[v.name] = dict(ms=ms, d=d, wall_ms=wall, passes=passes, in_scan=in_scan, t_roof=t_roof, place=place,
                               kernel=v.kernel, plan=v.plan)

    # Dominant kernel of the headline (bf16) path and its roofline. Every pass
    # is HBM-bound at this shape (Pass C: ~0.49 GB against ~6 us of bf16 MFMA
    # work; Pass A: ~0.32 GB against ~20 us of bf16x6 MFMA work), so each is
    # priced on its algorithmic bytes: what it must read and write once. The
    # dominant kernel and its duration come from the passes' times inside
    # whole scans (time_in_scan, means), the statistic rocprofv3 --stats
    # averages over a run of this script.
    r = results["bf16"]
    pa = pass_us(r["passes"])                   # median kernel time per pass (split encodes), us
    pin = r["in_scan"]                          # mean time per pass inside whole scans, us
    plan = r["plan"]
    pass_bytes = pass_algorithmic_bytes(plan)
    # Pass B has no kernel of its own when the walking Pass C runs its scan
    # (plan.kernel_b is null): its bytes and time are then Pass C's.
    kernels = {"A": plan.kernel_a, "B": plan.kernel_b, "C": plan.kernel_c}
    live = [k for k in "ABC" if kernels[k]]
    dom = max(live, key=lambda k: pin[k])
    kname = kernels[dom].decode()
    t = pin[dom] * 1e-6
    roof = {"kernel": f"{kname} (Pass {dom})", "bound": "hbm",
            "achieved": pass_bytes[dom] / t / 1e9, "peak": PEAK_HBM / 1e9, "unit": "GB/s",
            "algorithmic_bytes": pass_bytes[dom], "duration_us": pin[dom],
            "duration_stat": "mean time inside whole scans (whole scan less the scan without the pass)"}
    roof["frac"] = roof["achieved"] / roof["peak"]
    roof["traffic"] = profiled_traffic(kname)
    passes_roof = {k: {"kernel": kernels[k].decode(),
                       "us_in_scan": pin[k], "us_split": pa[k], "algorithmic_bytes": pass_bytes[k],
                       "hbm_frac": pass_bytes[k] / (pin[k] * 1e-6) / PEAK_HBM} for k in live}

    ms = r["ms"]
    value = S * L / (ms * 1e-3)
    out = {
        "metric": METRIC,
        "value": value,
        "unit": "tok/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": value / REF_TOKS,
        "dtype": "bf16",
        "data": "synthetic (BASELINE.json distributions; config 2 on torch RNG seed 1002, config i of the per-config report on seed 1000+i)",
        "config": {
            "workload": "config 2: SSD prefill scan S=1 L=8192 H=64 P=64 N=128 G=8 chunk=64, "
                        "bf16 Pass C operands, Pass A on bf16x6 split products (carried state and "
                        "s1 at the fp32 per-element bound), fp32 Pass B, inputs resident in HBM",
            "kernel": r["kernel"],
            "plan": {"groups": plan.n_groups, "seg_len": plan.seg_len, "hblk": plan.hblk,
                     "scratch_MiB": plan.total_bytes / 2**20},
            "vs_baseline_ref": "reference 3-pass + bf16 Pass C on Apple M5 Max, 1,315,051 tok/s",
        },
        "gflops": F / (ms * 1e-3) / 1e9,
        "roofline_op": {"t_roof_us": r["t_roof"] * 1e6, "t_us": ms * 1e3,
                        "frac": r["t_roof"] / (ms * 1e-3),
                        "rule": "max(F_A/fp32_peak + F_C/bf16_peak, alg_bytes/8TB/s)"},
        "roofline": roof,
        "passes_roofline": passes_roof,
        "timing_ms": {k: round(vv, 5) for k, vv in r["d"].items()},
        "y_placements": {"offsets_MiB": [k * Y_STEP / 2**20 for k in range(Y_PLACES)],
                         "ms": [round(t, 5) for t in r["place"]],
                         "spread": max(r["place"]) / min(r["place"]),
                         "value_from": "median over placements of each placement's mean step time"},
        # Per-pass kernel times: event-bracketed single-pass encodes less an
        # empty encode between the same events (event_pair_us), and the
        # passes' times inside whole scans (time_in_scan).
        "passes_us": {k: pa[k] for k in live},
        "passes_in_scan_us": {k: pin[k] for k in live},
        "event_pair_us": dist(r["passes"]["X"])["median"] * 1e3,
        "fp32_path": {
            "tok_s": S * L / (results["fp32"]["ms"] * 1e-3),
            "gflops": F / (results["fp32"]["ms"] * 1e-3) / 1e9,
            "ms_per_step": results["fp32"]["ms"],
            "y_placement_ms": [round(t, 5) for t in results["fp32"]["place"]],
            "roofline_frac": results["fp32"]["t_roof"] / (results["fp32"]["ms"] * 1e-3),
            "passes_us": pass_us(results["fp32"]["passes"]),
            "kernel": results["fp32"]["kernel"],
        },
    }
    sp = results["single-pass"]
    out["single_pass"] = {
        "tok_s": S * L / (sp["ms"] * 1e-3),
        "gflops": F / (sp["ms"] * 1e-3) / 1e9,
        "ms_per_step": sp["ms"],
        "form": ("three launches, state tiles in y (no scratch)" if sp["plan"].state_in_y
                 else "one launch (no scratch)"),
        "kernels": ([k.decode() for k in (sp["plan"].kernel_a, sp["plan"].kernel_b, sp["plan"].kernel_c)]
                    if sp["plan"].state_in_y else [sp["plan"].kernel_1pass.decode()]),
        "kernel": sp["kernel"],
    }
    extra = [v for v in variants if v.name not in ("bf16", "fp32", "single-pass")]
    if extra:
        out["variants"] = {}
        for v in extra:
            rv = results[v.name]
            e = {"ms_per_step": rv["ms"], "kernel": rv["kernel"]}
            if rv["passes"]:
                e["passes_us"] = pass_us(rv["passes"])
            out["variants"][v.name] = e
    if args.cold_steps > 0:
        # Steps that repeat one input find much of it in the 256 MB Infinity
        # Cache (x alone is 128 MiB); these scans start with it evicted.
        cold = {}
        for name in ("bf16", "fp32"):
            v = next(vv for vv in variants if vv.name == name)
            warm_up(v, 100.0)
            tc = statistics.median(time_cold(v, args.cold_steps, stream, COLD_FLUSH_BYTES))
            cold[name] = {"ms_per_step": tc, "tok_s": S * L / (tc * 1e-3), "vs_warm": tc / results[name]["ms"]}
        cold["flush"] = f"a {COLD_FLUSH_BYTES >> 20} MiB device copy before each timed scan, outside its events"
        cold["steps"] = args.cold_steps
        out["cold_cache"] = cold
    if args.config_steps > 0:
        out["configs"] = config_report(ctx, stream, dev, args.config_steps,
                                       min(args.warmup_ms, 100.0))
    if args.calib_copy:
        n = args.calib_copy * (1 << 20) // 4
        src = torch.randn(n, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        out["calib_copy_bytes"] = n * 4
    if not args.no_cpu:
        out.update(cpu_baseline(args.cpu_budget))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
