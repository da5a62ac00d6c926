"""Seeded random shapes against the fp64 oracle, on the three paths.

Each case draws a sequence length (ragged chunks included), one to three
sequences, one, two or four B/C groups, up to twelve heads per group, head_dim
and d_state among the multiples of 8 up to 192 and 256 (d_state above 128 runs
as blocks of state indices), SHORT or LONG memory and a nonzero s0; shapes
whose oracle would take more than about a second are drawn again. The bf16
path (Pass A on scaled fp16 planes by default), the fp32 path and the single
pass are held to the reference's per-element bounds (y at the bf16 bound on the
bf16 path, s1 at the fp32 bound everywhere). Every other shape also runs with
x, B, C and y in bf16 and f16 storage on the walk, the fp32 path and the single
pass, against the oracle fed the same inputs rounded to the storage type, to the
bounds of the storage tests (test_gpu_io.check).
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import pyoracle as po
from helix_amd.desc import HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA, HELIX_BF16, HELIX_F16
from gpu_harness import BF16_ABS, BF16_REL, F32_ABS, F32_REL, run
from test_gpu_io import NAME, check, rounded, run_io

pytestmark = pytest.mark.gpu

BUDGET = 1.5e8   # L * S * H * P * N per case


def _shapes(n: int, seed: int):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        L = int(rng.choice([int(rng.integers(1, 130)), int(rng.integers(130, 1500))]))
        S = int(rng.integers(1, 4))
        G = int(rng.choice([1, 2, 4]))
        H = G * int(rng.integers(1, 13))
        P = 8 * int(rng.integers(1, 25))
        N = 8 * int(rng.integers(1, 33))
        if L * S * H * P * N > BUDGET:
            continue
        out.append((L, S, H, P, N, G, "long" if rng.random() < 0.5 else "short", int(rng.integers(1 << 30))))
    return out


CASES = _shapes(24, 20261202)
PATHS = [("bf16", HELIX_BACKEND_MPP, True), ("fp32", HELIX_BACKEND_SGMMA, True), ("single", HELIX_BACKEND_AUTO, False)]


@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
@pytest.mark.parametrize("case", CASES, ids=[f"L{c[0]}-S{c[1]}-H{c[2]}-P{c[3]}-N{c[4]}-G{c[5]}-{c[6]}" for c in CASES])
def test_random_shape(gpu, case, path):
    L, S, H, P, N, G, memory, seed = case
    label, backend, multipass = path
    p = po.problem_harness(L, S, H, P, N, G, seed % 100000, memory)
    p.s0 = (np.random.default_rng(seed).standard_normal(p.s0.shape) * 0.3).astype(np.float32)
    d = p.d.copy()
    d.multipass = multipass
    d.backend = backend
    assert gpu.supported(d), gpu.backend_desc(d)
    y_ref, s_ref = po.scan(p, threads=0)
    _, y, s1 = run(gpu, p, desc=d)
    rel, ab = (BF16_REL, BF16_ABS) if label == "bf16" else (F32_REL, F32_ABS)
    ry = po.allclose_ratio(y, y_ref, rel, ab)
    rs = po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS)
    print(f"{label:6s} L={L} S={S} H={H} P={P} N={N} G={G} {memory}: y {ry:.3f} s1 {rs:.3f} "
          f"[{gpu.backend_desc(d)}]", flush=True)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)


IO_CASES = CASES[::2]
IO_PATHS = [("walk", HELIX_BACKEND_AUTO, True), ("fp32", HELIX_BACKEND_SGMMA, True), ("1pass", HELIX_BACKEND_AUTO, False)]
_io_refs = {}


def _io_problem(case, io):
    """The case's inputs rounded to the storage type and the oracle's result on them (kept per case)."""
    key = (case, io)
    if key not in _io_refs:
        L, S, H, P, N, G, memory, seed = case
        p = rounded(po.problem_harness(L, S, H, P, N, G, seed % 100000, memory), io)
        p.s0 = (np.random.default_rng(seed).standard_normal(p.s0.shape) * 0.3).astype(np.float32)
        _io_refs.clear()
        _io_refs[key] = (p, *po.scan(p, threads=0))
    return _io_refs[key]


@pytest.mark.parametrize("path", IO_PATHS, ids=[p[0] for p in IO_PATHS])
@pytest.mark.parametrize("io", [HELIX_BF16, HELIX_F16], ids=["bf16", "f16"])
@pytest.mark.parametrize("case", IO_CASES, ids=[f"L{c[0]}-S{c[1]}-H{c[2]}-P{c[3]}-N{c[4]}-G{c[5]}-{c[6]}" for c in IO_CASES])
def test_random_shape_storage(gpu, case, io, path):
    label, backend, multipass = path
    p, y_ref, s_ref = _io_problem(case, io)
    desc, y, s1 = run_io(gpu, p, io, backend, multipass)
    assert f"{NAME[io]} storage" in desc
    ey, es = check(io, desc, y, s1, y_ref, s_ref)
    print(f"{NAME[io]} {label} {case[:7]}: y {ey:.2e} s1 {es:.2e}  [{desc}]", flush=True)
