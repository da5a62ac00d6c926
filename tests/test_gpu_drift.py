"""Numerical drift across many chunk boundaries, on the GPU.

Counterpart of the reference's tests/test_drift.mm:38-208. A per-chunk error
that is small says nothing about whether it compounds, so this walks 8192
tokens (128 chunks) and checks the carried state against the fp64 oracle's
snapshots (oracle_scan_snapshots, the reference's scan_with_snapshots) at
every 8th chunk boundary. As in the reference, a boundary state is read
through the public API by re-running the scan truncated to that boundary:
HELIX exposes no intermediate state.

Each boundary is held to the fp32 per-element bound (rel 5e-6, abs 5e-7) on
every path: the carried state never passes through bf16, the bf16 path's
included (only its Pass C narrows operands). The worst late-quarter error
must stay under ten times the worst early-quarter error, so a scheme that
compounds error multiplicatively across chunks fails here.

Modes: the single pass and the multipass scan on the bf16 path (AUTO, as the
reference's default) and on the fp32 path, in SHORT and LONG memory (LONG is
the regime where the inter-chunk carry is numerically visible).
"""
from __future__ import annotations

import functools

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from helix_amd.desc import HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA
from gpu_harness import F32_ABS, F32_REL, run, s1_tolerance, upload

pytestmark = pytest.mark.gpu

TOKENS, CHUNK, HEADS, HEAD_DIM, STATE = 8192, 64, 8, 64, 128
SEED = 20260905

MODES = [
    # (label, multipass, backend, memory)
    ("1pass/short", False, HELIX_BACKEND_AUTO, "short"),
    ("3pass/short", True, HELIX_BACKEND_AUTO, "short"),
    ("3pass-fp32/short", True, HELIX_BACKEND_SGMMA, "short"),
    ("1pass/long", False, HELIX_BACKEND_AUTO, "long"),
    ("3pass/long", True, HELIX_BACKEND_AUTO, "long"),
    ("3pass-fp32/long", True, HELIX_BACKEND_SGMMA, "long"),
]


@functools.lru_cache(maxsize=None)
def _truth(memory):
    p = po.problem_harness(TOKENS, 1, HEADS, HEAD_DIM, STATE, 1, SEED, memory)
    _, _, snaps = po.scan_snapshots(p, CHUNK)
    return p, snaps


@pytest.mark.parametrize("mode", MODES, ids=[m[0] for m in MODES])
def test_drift_bounded(gpu, mode):
    label, multipass, backend, memory = mode
    p, snaps = _truth(memory)
    n_chunks = (TOKENS + CHUNK - 1) // CHUNK
    dev = {k: upload(getattr(p, k)) for k in ("s0", "x", "dt", "A", "B", "C")}
    y_buf = torch.empty(p.y_shape(), device="cuda")
    probes, drift = [], []
    for c in range(7, n_chunks, 8):
        d = p.d.copy()
        d.n_tok = (c + 1) * CHUNK          # the same buffers and strides, truncated
        d.multipass = multipass
        d.backend = backend
        assert gpu.supported(d), f"{label} unsupported at chunk {c}"
        if multipass and backend == HELIX_BACKEND_AUTO:
            assert gpu.select_backend(d) == HELIX_BACKEND_MPP
        assert s1_tolerance(gpu, d) == (F32_REL, F32_ABS)
        s1_buf = torch.full(p.s_shape(), float("nan"), device="cuda")
        sub = po.Problem(d, p.s0, p.x, p.dt, p.A, p.B, p.C, None)
        _, _, s1 = run(gpu, sub, desc=d, s0_gpu=dev["s0"], y_gpu=y_buf, s1_gpu=s1_buf)
        want = snaps[c]
        assert np.all(np.isfinite(s1)), f"{label}: non-finite state at chunk {c}"
        err = np.abs(s1.astype(np.float64) - want)
        ratio = float(np.max(err / (F32_ABS + F32_REL * np.abs(want))))
        probes.append(c)
        drift.append(float(err.max()))
        assert ratio <= 1.0, f"{label}: tolerance exceeded at chunk {c} (ratio {ratio:.3f})"
    for c, e in zip(probes, drift):
        print(f"  {label} chunk {c:3d} (tok {(c + 1) * CHUNK:5d})  max|ds| = {e:.3e}", flush=True)
    q = len(probes) // 4
    early, late = max(drift[:q]), max(drift[-q:])
    growth = late / early if early > 0 else 1.0
    print(f"  {label}: early-quarter max {early:.3e} -> late-quarter max {late:.3e} ({growth:.2f}x)",
          flush=True)
    assert growth < 10.0, f"{label}: drift grows {growth:.2f}x across {n_chunks} chunks"
