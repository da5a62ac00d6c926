"""GPU parity against the fp64 sequential oracle.

Mirrors the reference's tests/test_metal_parity.mm:
  * the same 22-shape matrix (:77-104), seed 4242, harness inputs;
  * SHORT and LONG memory (:121-128) and the tiny-scratch mode that forces many
    super-chunk groups (HELIX_SCRATCH_MB=1, :106-110);
  * per-element allclose with the tolerance of the backend that actually ran
    (:163-166); s1 held to the fp32 bound on every default path (:210-218).
    Only the bf16 path's opt-in two-plane Pass A (HELIX_PASSA_SPLIT=3) is held
    to a bound ten times wider (gpu_harness.s1_tolerance).
Both MI355X paths are exercised explicitly (SGMMA -> fp32 path, MPP -> bf16
Pass C) because AUTO resolves to bf16 for every multipass shape here. The
reference's single-pass modes (multipass=false, AUTO backend: the fp32
single-pass kernel) run in SHORT and LONG memory.

Then the BASELINE.json configurations at full size on both paths and the
single pass, in BASELINE's distributions and in LONG memory, gated on
max|dy|/max|y| <= 1e-4 (fp32) / 2e-2 (bf16) and likewise for s1, with the CPU
oracle recomputing every head.
"""
from __future__ import annotations

import functools

import numpy as np
import pytest

from oracle import pyoracle as po
from helix_amd.desc import HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA
from baseline_configs import CONFIGS
from gpu_harness import (BF16_ABS, BF16_GATE, BF16_REL, F32_ABS, F32_GATE, F32_REL, ctx_for, run,
                         s1_tolerance)

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 1, 2, 64, 128, 1, "L=1 ragged only"),
    (7, 1, 2, 64, 128, 1, "L=7 ragged only"),
    (63, 1, 2, 64, 128, 1, "L=63 ragged only"),
    (64, 1, 2, 64, 128, 1, "L=64 one full chunk"),
    (65, 1, 2, 64, 128, 1, "L=65 full + 1 ragged"),
    (127, 1, 2, 64, 128, 1, "L=127 full + ragged"),
    (128, 1, 2, 64, 128, 1, "L=128 two full chunks"),
    (129, 1, 2, 64, 128, 1, "L=129 two full + ragged"),
    (96, 1, 4, 64, 128, 1, "L=96 full + 32 ragged"),
    (160, 1, 4, 64, 128, 1, "L=160 two full + 32 ragged"),
    (300, 1, 8, 64, 128, 2, "L=300 four full + 44 ragged"),
    (256, 1, 4, 64, 64, 1, "d_state=64"),
    (256, 1, 4, 128, 128, 1, "head_dim=128"),
    (256, 1, 4, 128, 256, 1, "d_state=256"),
    (256, 1, 4, 64, 256, 1, "d_state=256 head_dim=64"),
    (300, 1, 4, 128, 256, 1, "d_state=256 ragged tail"),
    (256, 1, 8, 128, 256, 2, "d_state=256 grouped"),
    (256, 1, 4, 192, 128, 1, "head_dim=192 three slabs"),
    # Partial 16-channel blocks and padded state indices (head_dim and
    # d_state need only be multiples of 8).
    (200, 1, 3, 40, 96, 1, "head_dim=40 d_state=96"),
    (150, 1, 2, 72, 40, 1, "head_dim=72 d_state=40"),
    (256, 1, 8, 128, 128, 8, "n_group=8 grouped"),
    (256, 4, 4, 64, 128, 1, "n_seq=4 batched"),
    (1024, 1, 2, 64, 128, 1, "L=1024 sixteen chunks"),
    (2048, 1, 8, 64, 128, 2, "L=2048 realistic prefill"),
]

MODES = [
    # (label, backend, scratch_mb, memory, extra environment, multipass)
    ("1pass", HELIX_BACKEND_AUTO, None, "short", {}, False),
    ("1pass/long", HELIX_BACKEND_AUTO, None, "long", {}, False),
    # The single pass in its one-launch form everywhere (by default the
    # shapes with rows for a state tile run the three passes with the tiles
    # in y, test_gpu_single_y.py).
    ("1pass/1launch/long", HELIX_BACKEND_AUTO, None, "long", {"HELIX_1PASS_Y": "0"}, False),
    ("fp32", HELIX_BACKEND_SGMMA, None, "short", {}, True),
    ("fp32/sm", HELIX_BACKEND_SGMMA, 1, "short", {}, True),
    ("fp32/long", HELIX_BACKEND_SGMMA, None, "long", {}, True),
    ("fp32/sm/long", HELIX_BACKEND_SGMMA, 1, "long", {}, True),
    # The fp32 path's chunk-parallel Pass C on per-chunk states stored by
    # Pass A, which d_state <= 128 replaces with the walk wherever the plan
    # walks more than one chunk.
    ("fp32/chunk/long", HELIX_BACKEND_SGMMA, None, "long", {"HELIX_F32_WALK": "0"}, True),
    # The fp32 walk (pinned: most shapes here plan one-chunk walks) with Pass
    # B launched on its own, with Pass B's segment scan in its prologue, over
    # four-chunk walks, and over several chunk groups carried through s1.
    ("fp32/passB/long", HELIX_BACKEND_SGMMA, None, "long", {"HELIX_F32_WALK": "1", "HELIX_FUSE_B": "0"}, True),
    ("fp32/fuseB/long", HELIX_BACKEND_SGMMA, None, "long", {"HELIX_F32_WALK": "1", "HELIX_FUSE_B": "1"}, True),
    ("fp32/walk4/long", HELIX_BACKEND_SGMMA, None, "long", {"HELIX_F32_WALK": "1", "HELIX_SEG_LEN": "4"}, True),
    ("fp32/walk/sm", HELIX_BACKEND_SGMMA, 1, "short", {"HELIX_F32_WALK": "1"}, True),
    ("fp32/chunk/sm", HELIX_BACKEND_SGMMA, 1, "short", {"HELIX_F32_WALK": "0"}, True),
    ("bf16", HELIX_BACKEND_MPP, None, "short", {}, True),
    ("bf16/sm", HELIX_BACKEND_MPP, 1, "short", {}, True),
    ("bf16/long", HELIX_BACKEND_MPP, None, "long", {}, True),
    ("bf16/sm/long", HELIX_BACKEND_MPP, 1, "long", {}, True),
    # The walk with Pass B launched on its own, and with Pass B's segment scan
    # run in its prologue (by default: single-group plans of at most four
    # segments).
    ("bf16/passB/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_FUSE_B": "0"}, True),
    ("bf16/fuseB/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_FUSE_B": "1"}, True),
    # The walk on the caller's fp32 B and C, and on Pass A's bf16 copies of
    # them (by default only past eight items per group).
    ("bf16/nocopy/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_WALK_BCCOPY": "0"}, True),
    ("bf16/copy/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_WALK_BCCOPY": "1"}, True),
    ("bf16/copy/sm", HELIX_BACKEND_MPP, 1, "short", {"HELIX_WALK_BCCOPY": "1"}, True),
    # d_state 129..256 runs as blocks of at most 128 state indices by default;
    # these pin one launch sequence on the d_state 256 kernels.
    ("fp32/n256/long", HELIX_BACKEND_SGMMA, None, "long", {"HELIX_STATE_BLOCKS": "0"}, True),
    ("bf16/n256/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_STATE_BLOCKS": "0"}, True),
    ("1pass/n256/long", HELIX_BACKEND_AUTO, None, "long", {"HELIX_STATE_BLOCKS": "0", "HELIX_1PASS_Y": "0"}, False),
    # Pass A on two scaled fp16 planes (three products), s1 at the fp32 bound.
    ("bf16/h3", HELIX_BACKEND_MPP, None, "short", {"HELIX_PASSA_F16": "1"}, True),
    ("bf16/h3/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_PASSA_F16": "1"}, True),
    ("bf16/h3/sm/long", HELIX_BACKEND_MPP, 1, "long", {"HELIX_PASSA_F16": "1"}, True),
    ("bf16/h3/copy/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_PASSA_F16": "1", "HELIX_WALK_BCCOPY": "1"}, True),
    # Opt-in: Pass A on two split planes (three products), s1 at the wider bound.
    ("bf16/x3", HELIX_BACKEND_MPP, None, "short", {"HELIX_PASSA_SPLIT": "3"}, True),
    ("bf16/x3/sm/long", HELIX_BACKEND_MPP, 1, "long", {"HELIX_PASSA_SPLIT": "3"}, True),
]


@functools.lru_cache(maxsize=None)
def _reference(shape, memory):
    L, S, H, P, N, G, _ = shape
    p = po.problem_harness(L, S, H, P, N, G, 4242, memory)
    y, s1 = po.scan(p, threads=0)
    return p, y, s1


@pytest.mark.parametrize("mode", MODES, ids=[m[0] for m in MODES])
@pytest.mark.parametrize("shape", SHAPES, ids=[s[-1] for s in SHAPES])
def test_shape_matrix(gpu, shape, mode):
    label, backend, scratch_mb, memory, extra, multipass = mode
    p, y_ref, s_ref = _reference(shape, memory)
    d = p.d.copy()
    d.multipass = multipass
    d.backend = backend
    ctx = ctx_for(gpu, HELIX_SCRATCH_MB=scratch_mb, **extra)
    assert ctx.supported(d), ctx.backend_desc(d)
    is_bf16 = ctx.select_backend(d) == HELIX_BACKEND_MPP
    s_rel, s_abs = s1_tolerance(ctx, d)
    if scratch_mb:
        assert not multipass or ctx.plan_info(d).n_groups > 1 or shape[0] <= 256
    _, y, s1 = run(ctx, p, desc=d)
    rel, ab = (BF16_REL, BF16_ABS) if is_bf16 else (F32_REL, F32_ABS)
    ry = po.allclose_ratio(y, y_ref, rel, ab)
    rs = po.allclose_ratio(s1, s_ref, s_rel, s_abs)
    print(f"{label:13s} {shape[-1]:32s} y ratio {ry:.3f}  s1 ratio {rs:.3f}  "
          f"maxrel {po.max_rel_err(y, y_ref):.2e}", flush=True)
    assert ry <= 1.0, f"y outside tolerance: ratio {ry}"
    assert rs <= 1.0, f"s1 outside tolerance: ratio {rs}"


# ---------------------------------------------------------------------------
# BASELINE.json configurations at full size, every head against the oracle
# ---------------------------------------------------------------------------

@functools.lru_cache(maxsize=None)
def _baseline(name, memory):
    c = CONFIGS[name]
    if memory == "long":
        p = po.problem_harness(*c.shape, c.seed, "long")
        p.ids = None
    else:
        p = po.problem_gauss(*c.shape, c.seed, c.s0_sigma, c.dt_mu, c.dt_sigma)
    y, s1 = po.scan(p, threads=0)
    return p, y, s1


# Both paths and the single pass on every config, in BASELINE's distributions
# ("dist") and in LONG memory; the opt-in two-plane Pass A on the configs BASELINE
# quotes on the bf16 path.
CASES = [(n, path, mem) for n in CONFIGS for mem in ("dist", "long") for path in ("fp32", "bf16", "1pass")]
CASES += [(n, "bf16/x3", "dist") for n, c in CONFIGS.items() if "bf16" in c.paths]
CASES += [(n, "bf16/h3", mem) for n, c in CONFIGS.items() if "bf16" in c.paths for mem in ("dist", "long")]


@pytest.mark.parametrize("name,path,memory", CASES, ids=[f"{n}-{p}-{m}" for n, p, m in CASES])
def test_baseline_config(gpu, name, path, memory):
    p, y_ref, s_ref = _baseline(name, memory)
    d = p.d.copy()
    d.multipass = path != "1pass"
    d.backend = (HELIX_BACKEND_MPP if path.startswith("bf16")
                 else HELIX_BACKEND_AUTO if path == "1pass" else HELIX_BACKEND_SGMMA)
    ctx = ctx_for(gpu, HELIX_PASSA_SPLIT="3" if path == "bf16/x3" else None,
                  HELIX_PASSA_F16="1" if path == "bf16/h3" else None)
    assert ctx.supported(d)
    s_rel, s_abs = s1_tolerance(ctx, d)
    assert (ctx.select_backend(d) == HELIX_BACKEND_MPP) == path.startswith("bf16")
    print(f"[{name} {path} {memory}] {ctx.backend_desc(d)}", flush=True)
    _, y, s1 = run(ctx, p, desc=d)
    is_bf16 = path.startswith("bf16")
    ey = po.max_rel_err(y, y_ref)
    es = po.max_rel_err(s1, s_ref)
    gate = BF16_GATE if is_bf16 else F32_GATE
    print(f"  max|dy|/max|y| = {ey:.3e}   max|ds1|/max|s1| = {es:.3e}   gate {gate:g}", flush=True)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    assert ey <= gate
    assert es <= gate
    if is_bf16:
        assert po.allclose_ratio(y, y_ref, BF16_REL, BF16_ABS) <= 1.0
    else:
        # The fp32 paths are also held to the reference's per-element bound.
        assert po.allclose_ratio(y, y_ref, F32_REL, F32_ABS) <= 1.0
    # The carried state never passes through bf16 on any default path: the
    # fp32 per-element bound (the wider one only for the opt-in bf16x3 Pass A).
    assert po.allclose_ratio(s1, s_ref, s_rel, s_abs) <= 1.0


# ---------------------------------------------------------------------------
# The fp32 path at d_state 64 and full length: the walk over 16-chunk
# segments (the default there), the chunk-parallel Pass C
# (HELIX_F32_WALK=0), and the bf16 path; every head against the oracle.
# ---------------------------------------------------------------------------

D64_SHAPE = (8192, 1, 64, 64, 64, 8)
D64_CASES = [
    ("fp32/walk", HELIX_BACKEND_SGMMA, {}),
    ("fp32/chunk", HELIX_BACKEND_SGMMA, {"HELIX_F32_WALK": "0"}),
    ("bf16", HELIX_BACKEND_MPP, {}),
]


@functools.lru_cache(maxsize=None)
def _d64(memory):
    if memory == "long":
        p = po.problem_harness(*D64_SHAPE, 1010, "long")
        p.ids = None
    else:
        p = po.problem_gauss(*D64_SHAPE, 1010, 0.0, -1.0, 0.5)
    y, s1 = po.scan(p, threads=0)
    return p, y, s1


@pytest.mark.parametrize("memory", ["dist", "long"])
@pytest.mark.parametrize("label,backend,extra", D64_CASES, ids=[c[0] for c in D64_CASES])
def test_dstate64_full_length(gpu, label, backend, extra, memory):
    p, y_ref, s_ref = _d64(memory)
    d = p.d.copy()
    d.multipass = True
    d.backend = backend
    ctx = ctx_for(gpu, **extra)
    assert ctx.supported(d)
    info = ctx.plan_info(d)
    if label == "fp32/walk":
        assert info.kernel_c == b"helix_scan_walk_x6_n64" and info.walk_len > 1
    elif label == "fp32/chunk":
        assert info.kernel_c == b"helix_chunk_out_x6_n64"
    s_rel, s_abs = s1_tolerance(ctx, d)
    print(f"[d_state 64 {label} {memory}] {ctx.backend_desc(d)}", flush=True)
    _, y, s1 = run(ctx, p, desc=d)
    is_bf16 = backend == HELIX_BACKEND_MPP
    gate = BF16_GATE if is_bf16 else F32_GATE
    ey, es = po.max_rel_err(y, y_ref), po.max_rel_err(s1, s_ref)
    print(f"  max|dy|/max|y| = {ey:.3e}   max|ds1|/max|s1| = {es:.3e}   gate {gate:g}", flush=True)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    assert ey <= gate and es <= gate
    rel, ab = (BF16_REL, BF16_ABS) if is_bf16 else (F32_REL, F32_ABS)
    assert po.allclose_ratio(y, y_ref, rel, ab) <= 1.0
    assert po.allclose_ratio(s1, s_ref, s_rel, s_abs) <= 1.0


# ---------------------------------------------------------------------------
# Where Pass B's segment scan runs, at full size: its own launch at config 2
# (the default), also over many super-chunk groups whose walks span two Pass A
# segments (HELIX_SCRATCH_MB=20: fifteen groups, one-chunk segments,
# two-chunk walks, carried through s1); and the walk's prologue at config 4a
# (the default) against its own launch there. Every head against the oracle,
# s1 at the fp32 per-element bound.
# ---------------------------------------------------------------------------

PASS_B_CASES = [
    ("cfg2", "bf16", {"HELIX_SCRATCH_MB": "20"}, "launched", True),
    ("cfg2", "fp32", {"HELIX_SCRATCH_MB": "20"}, "launched", True),
    ("cfg4a", "bf16", {"HELIX_FUSE_B": "0"}, "launched", False),
    ("cfg4a", "bf16", {}, "in_c", False),
]


@pytest.mark.parametrize("name,path,extra,where,multi", PASS_B_CASES,
                         ids=[f"{c[0]}-{c[1]}-" + ("-".join(f"{k[6:]}={v}" for k, v in c[2].items()) or "default")
                              for c in PASS_B_CASES])
def test_pass_b_placement(gpu, name, path, extra, where, multi):
    from helix_amd.abi import PASS_B_IN_C, PASS_B_LAUNCHED
    p, y_ref, s_ref = _baseline(name, "dist")
    d = p.d.copy()
    d.multipass = True
    d.backend = HELIX_BACKEND_MPP if path == "bf16" else HELIX_BACKEND_SGMMA
    ctx = ctx_for(gpu, **extra)
    info = ctx.plan_info(d)
    assert info.pass_b == {"in_c": PASS_B_IN_C, "launched": PASS_B_LAUNCHED}[where]
    if multi:
        assert info.n_groups > 1 and info.walk_len > info.seg_len
    print(f"[{name} {path} {extra}] groups {info.n_groups} seg {info.seg_len} walk {info.walk_len} "
          f"pass_b {info.pass_b}", flush=True)
    _, y, s1 = run(ctx, p, desc=d)
    is_bf16 = path == "bf16"
    ey, es = po.max_rel_err(y, y_ref), po.max_rel_err(s1, s_ref)
    print(f"  max|dy|/max|y| = {ey:.3e}   max|ds1|/max|s1| = {es:.3e}", flush=True)
    assert ey <= (BF16_GATE if is_bf16 else F32_GATE) and es <= F32_GATE
    rel, ab = (BF16_REL, BF16_ABS) if is_bf16 else (F32_REL, F32_ABS)
    assert po.allclose_ratio(y, y_ref, rel, ab) <= 1.0
    assert po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS) <= 1.0


# ---------------------------------------------------------------------------
# A walk length the dispatch model picks (caps.cpp fused_walk_len) on a
# batched shape with two B/C groups: 25-chunk walks, 25 + 7 chunks per
# sequence, Pass B in the walk's prologue, on both paths. Harness inputs in
# LONG memory, every head against the oracle.
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("path", ["bf16", "fp32"])
def test_model_walk_length(gpu, path):
    from helix_amd.abi import PASS_B_IN_C
    p = po.problem_harness(2048, 8, 96, 64, 128, 2, 4848, "long")
    y_ref, s_ref = po.scan(p, threads=0)
    d = p.d.copy()
    d.multipass = True
    d.backend = HELIX_BACKEND_MPP if path == "bf16" else HELIX_BACKEND_SGMMA
    info = gpu.plan_info(d)
    assert (info.n_groups, info.seg_len, info.walk_len, info.segs_per_group, info.pass_b) == (1, 25, 25, 2, PASS_B_IN_C)
    _, y, s1 = run(gpu, p, desc=d)
    is_bf16 = path == "bf16"
    rel, ab = (BF16_REL, BF16_ABS) if is_bf16 else (F32_REL, F32_ABS)
    ry, rs = po.allclose_ratio(y, y_ref, rel, ab), po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS)
    print(f"[model walk {path}] y ratio {ry:.3f}  s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0
