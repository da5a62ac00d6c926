"""GPU parity against the fp64 sequential oracle.

Mirrors the reference's tests/test_metal_parity.mm:
  * the same 22-shape matrix (:77-104), seed 4242, harness inputs;
  * SHORT and LONG memory (:121-128) and the tiny-scratch mode that forces many
    super-chunk groups (HELIX_SCRATCH_MB=1, :106-110);
  * per-element allclose with the tolerance of the backend that actually ran
    (:163-166); s1 held to the fp32 bound (:214-218) on every path whose Pass A
    runs six split products, and to a bound ten times wider on the walking bf16
    path's default three-product Pass A (gpu_harness.s1_tolerance).
Both MI355X paths are exercised explicitly (SGMMA -> fp32 MFMA Pass C, MPP ->
bf16 Pass C) because AUTO resolves to bf16 for every multipass shape here, and
each with its default bf16x6 split-product kernels and with the fp32-MFMA
ones (HELIX_X6=0). The reference's single-pass modes (multipass=false, AUTO
backend: the fp32 single-pass kernel) run in SHORT and LONG memory.

Then the BASELINE.json configurations at full size, gated on
max|dy|/max|y| <= 1e-4 (fp32) / 2e-2 (bf16) and likewise for s1, with the CPU
oracle recomputing a subset of heads (heads are independent, scan_ref.cpp:45).
"""
from __future__ import annotations

import functools

import numpy as np
import pytest

from oracle import pyoracle as po
from helix_amd.desc import HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA
from baseline_configs import CONFIGS
from gpu_harness import (BF16_ABS, BF16_GATE, BF16_REL, F32_ABS, F32_GATE, F32_REL, env, run,
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
    (256, 1, 8, 128, 128, 8, "n_group=8 grouped"),
    (256, 4, 4, 64, 128, 1, "n_seq=4 batched"),
    (1024, 1, 2, 64, 128, 1, "L=1024 sixteen chunks"),
    (2048, 1, 8, 64, 128, 2, "L=2048 realistic prefill"),
]

MODES = [
    # (label, backend, scratch_mb, memory, extra environment, multipass)
    ("1pass", HELIX_BACKEND_AUTO, None, "short", {}, False),
    ("1pass/long", HELIX_BACKEND_AUTO, None, "long", {}, False),
    ("fp32", HELIX_BACKEND_SGMMA, None, "short", {}, True),
    ("fp32/sm", HELIX_BACKEND_SGMMA, 1, "short", {}, True),
    ("fp32/long", HELIX_BACKEND_SGMMA, None, "long", {}, True),
    ("fp32/sm/long", HELIX_BACKEND_SGMMA, 1, "long", {}, True),
    ("bf16", HELIX_BACKEND_MPP, None, "short", {}, True),
    ("bf16/sm", HELIX_BACKEND_MPP, 1, "short", {}, True),
    ("bf16/long", HELIX_BACKEND_MPP, None, "long", {}, True),
    ("bf16/sm/long", HELIX_BACKEND_MPP, 1, "long", {}, True),
    ("bf16walk", HELIX_BACKEND_MPP, None, "short", {"HELIX_BF16_PASSC": "walk"}, True),
    ("bf16walk/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_BF16_PASSC": "walk"}, True),
    ("bf16walk/sm/long", HELIX_BACKEND_MPP, 1, "long", {"HELIX_BF16_PASSC": "walk"}, True),
    # The walk with Pass B launched on its own, and with Pass B's segment scan
    # run in the walk's prologue (by default: single-group plans of at most
    # four segments).
    ("bf16walk/passB/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_BF16_PASSC": "walk", "HELIX_FUSE_B": "0"},
     True),
    ("bf16walk/fuseB/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_BF16_PASSC": "walk", "HELIX_FUSE_B": "1"},
     True),
    # The walk with Pass A on six split products: s1 at the fp32 bound.
    ("bf16walk/x6", HELIX_BACKEND_MPP, None, "short", {"HELIX_BF16_PASSC": "walk", "HELIX_PASSA_SPLIT": "6"},
     True),
    ("bf16walk/x6/sm/long", HELIX_BACKEND_MPP, 1, "long",
     {"HELIX_BF16_PASSC": "walk", "HELIX_PASSA_SPLIT": "6"}, True),
    # The 16 x 16 walk on the caller's fp32 B and C instead of Pass A's bf16
    # copies.
    ("bf16walk/nocopy/long", HELIX_BACKEND_MPP, None, "long", {"HELIX_BF16_PASSC": "walk", "HELIX_WALK_BCCOPY": "0"},
     True),
    # The walk on 32 x 32 tiles (the default walk runs 16 x 16 tiles).
    ("bf16walk32", HELIX_BACKEND_MPP, None, "short", {"HELIX_BF16_PASSC": "walk", "HELIX_WALK": "32"}, True),
    ("bf16walk32/sm/long", HELIX_BACKEND_MPP, 1, "long", {"HELIX_BF16_PASSC": "walk", "HELIX_WALK": "32"}, True),
    # fp32-MFMA kernels instead of bf16x6 split products.
    ("fp32/mma/sm/long", HELIX_BACKEND_SGMMA, 1, "long", {"HELIX_X6": "0"}, True),
    ("fp32/mma", HELIX_BACKEND_SGMMA, None, "short", {"HELIX_X6": "0"}, True),
    ("bf16/mma/sm/long", HELIX_BACKEND_MPP, 1, "long", {"HELIX_X6": "0"}, True),
    ("bf16walk/mma/long", HELIX_BACKEND_MPP, None, "long",
     {"HELIX_X6": "0", "HELIX_BF16_PASSC": "walk"}, True),
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
    with env(HELIX_SCRATCH_MB=scratch_mb, **extra):
        assert gpu.supported(d), gpu.backend_desc(d)
        is_bf16 = gpu.select_backend(d) == HELIX_BACKEND_MPP
        s_rel, s_abs = s1_tolerance(gpu, d)
        _, y, s1 = run(gpu, p, desc=d)
    rel, ab = (BF16_REL, BF16_ABS) if is_bf16 else (F32_REL, F32_ABS)
    ry = po.allclose_ratio(y, y_ref, rel, ab)
    rs = po.allclose_ratio(s1, s_ref, s_rel, s_abs)
    print(f"{label:13s} {shape[-1]:32s} y ratio {ry:.3f}  s1 ratio {rs:.3f}  "
          f"maxrel {po.max_rel_err(y, y_ref):.2e}", flush=True)
    assert ry <= 1.0, f"y outside tolerance: ratio {ry}"
    assert rs <= 1.0, f"s1 outside tolerance: ratio {rs}"


# ---------------------------------------------------------------------------
# BASELINE.json configurations at full size
# ---------------------------------------------------------------------------

@functools.lru_cache(maxsize=None)
def _baseline(name, memory):
    c = CONFIGS[name]
    if memory == "long":
        p = po.problem_harness(*c.shape, c.seed, "long")
        p.ids = None
    else:
        p = po.problem_gauss(*c.shape, c.seed, c.s0_sigma, c.dt_mu, c.dt_sigma)
    mask = np.zeros(c.H, np.uint8)
    mask[list(c.check_heads)] = 1
    y, s1 = po.scan(p, head_mask=mask, threads=0)
    return p, y, s1


CASES = [(n, path, mem) for n, c in CONFIGS.items() for path in c.paths for mem in ("dist", "long")]
CASES += [(n, "bf16walk", "dist") for n, c in CONFIGS.items() if "bf16" in c.paths]
CASES += [(n, "bf16walk/x6", "dist") for n, c in CONFIGS.items() if "bf16" in c.paths]
CASES += [(n, "bf16walk32", "dist") for n, c in CONFIGS.items() if "bf16" in c.paths]
CASES += [(n, path + "/mma", "long") for n, c in CONFIGS.items() for path in c.paths]
CASES += [(n, "1pass", mem) for n in CONFIGS for mem in ("dist", "long")]


@pytest.mark.parametrize("name,path,memory", CASES, ids=[f"{n}-{p}-{m}" for n, p, m in CASES])
def test_baseline_config(gpu, name, path, memory):
    c = CONFIGS[name]
    p, y_ref, s_ref = _baseline(name, memory)
    d = p.d.copy()
    d.multipass = path != "1pass"
    d.backend = (HELIX_BACKEND_MPP if path.startswith("bf16")
                 else HELIX_BACKEND_AUTO if path == "1pass" else HELIX_BACKEND_SGMMA)
    with env(HELIX_BF16_PASSC="walk" if path.startswith("bf16walk") else None,
             HELIX_WALK="32" if path == "bf16walk32" else None,
             HELIX_X6="0" if path.endswith("/mma") else None,
             HELIX_PASSA_SPLIT="6" if path.endswith("/x6") else None):
        assert gpu.supported(d)
        s_rel, s_abs = s1_tolerance(gpu, d)
        assert (gpu.select_backend(d) == HELIX_BACKEND_MPP) == path.startswith("bf16")
        print(f"[{name} {path} {memory}] {gpu.backend_desc(d)}", flush=True)
        _, y, s1 = run(gpu, p, desc=d)
    path = "bf16" if path.startswith("bf16") else "fp32"
    hs = list(c.check_heads)
    ey = po.max_rel_err(y[:, :, hs], y_ref[:, :, hs])
    es = po.max_rel_err(s1[:, hs], s_ref[:, hs])
    gate = BF16_GATE if path == "bf16" else F32_GATE
    print(f"  max|dy|/max|y| = {ey:.3e}   max|ds1|/max|s1| = {es:.3e}   gate {gate:g}", flush=True)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    assert ey <= gate
    assert es <= gate
    if path == "fp32":
        # The fp32 path is also held to the reference's per-element bound.
        assert po.allclose_ratio(y[:, :, hs], y_ref[:, :, hs], F32_REL, F32_ABS) <= 1.0
    # The carried state never passes through bf16 on either path: fp32 bound,
    # or the bf16x3 bound where Pass A runs on two split planes.
    assert po.allclose_ratio(s1[:, hs], s_ref[:, hs], s_rel, s_abs) <= 1.0
