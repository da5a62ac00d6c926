"""Diagonal A (A[h][n], HELIX_A_DIAG_PER_CHANNEL) on the GPU against the fp64
oracle, whose diagonal form is pinned bit-exactly to the reference's own
ref::scan (tests/test_oracle.py; reference scan_ref.cpp:26-29).

The reference declines diagonal A (caps.mm:121-123); this build serves it with
the single-pass walk (kernels/pass_single.hip, DIAG), for either value of
multipass, up to d_state 128. Held to the fp32 gates: max|dy|/max|y| <= 1e-4
and the per-element bound of the reference's parity test, SHORT and LONG
memory, with the state-splitting invariant and an ids permutation.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from helix_amd.desc import HELIX_BACKEND_AUTO, HELIX_BACKEND_SGMMA, desc_init
from gpu_harness import F32_ABS, F32_GATE, F32_REL, run

pytestmark = pytest.mark.gpu

SHAPES = [
    (1, 1, 2, 64, 128, 1, "L=1"),
    (63, 1, 2, 64, 128, 1, "L=63 ragged only"),
    (64, 1, 2, 64, 128, 1, "L=64 one chunk"),
    (129, 1, 2, 64, 128, 1, "L=129 two full + ragged"),
    (300, 1, 8, 64, 128, 2, "L=300 grouped"),
    (256, 1, 4, 64, 64, 1, "d_state=64"),
    (256, 1, 4, 64, 16, 1, "d_state=16 (Mamba-1 size)"),
    (200, 1, 4, 64, 40, 2, "d_state=40"),
    (256, 1, 4, 128, 128, 1, "head_dim=128"),
    (256, 1, 4, 192, 128, 1, "head_dim=192 three slabs"),
    (256, 4, 4, 64, 128, 1, "n_seq=4"),
    (1024, 1, 2, 64, 128, 1, "L=1024"),
]
MODES = [("short", False), ("long", False), ("short", True), ("long", True)]


def _check(y, s1, y_ref, s_ref):
    ey, es = po.max_rel_err(y, y_ref), po.max_rel_err(s1, s_ref)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    assert ey <= F32_GATE and es <= F32_GATE, (ey, es)
    assert po.allclose_ratio(y, y_ref, F32_REL, F32_ABS) <= 1.0
    assert po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS) <= 1.0
    return ey, es


@pytest.mark.parametrize("mode", MODES, ids=[f"{m}-{'mp' if mp else '1p'}" for m, mp in MODES])
@pytest.mark.parametrize("shape", SHAPES, ids=[s[-1] for s in SHAPES])
def test_diag_matrix(gpu, shape, mode):
    memory, multipass = mode
    p = po.problem_diag(*shape[:6], 4242, memory)
    p.s0 = np.random.default_rng(1).standard_normal(p.s0.shape).astype(np.float32) * 0.2
    y_ref, s_ref = po.scan(p)
    d = p.d.copy()
    d.multipass = multipass
    d.backend = HELIX_BACKEND_AUTO
    assert gpu.supported(d), gpu.backend_desc(d)
    assert "diagonal A" in gpu.backend_desc(d)
    _, y, s1 = run(gpu, p, desc=d)
    ey, es = _check(y, s1, y_ref, s_ref)
    print(f"diag {memory} {'mp' if multipass else '1p'} {shape[-1]}: y {ey:.2e} s1 {es:.2e}", flush=True)


@pytest.mark.parametrize("split", [64, 700])
def test_diag_state_splitting(gpu, split):
    p = po.problem_diag(1500, 2, 4, 64, 64, 2, 77, "long")
    y_ref, s_ref = po.scan(p, threads=0)
    L, S, H, P, N, G = p.shape

    def part(t0, t1):
        d = desc_init(t1 - t0, S, H, P, N, G)
        d.a_form, d.s_a = p.d.a_form, p.d.s_a
        d.backend = HELIX_BACKEND_SGMMA
        cut = lambda a: np.ascontiguousarray(a[:, t0:t1])
        return po.Problem(d, p.s0, cut(p.x), cut(p.dt), p.A, cut(p.B), cut(p.C), None)

    a, b = part(0, split), part(split, L)
    mid = torch.full(a.s_shape(), float("nan"), device="cuda")
    _, y1, _ = run(gpu, a, desc=a.d, s1_gpu=mid)
    _, y2, s1 = run(gpu, b, desc=b.d, s0_gpu=mid)
    _check(np.concatenate([y1, y2], axis=1), s1, y_ref, s_ref)


def test_diag_ids_permutation(gpu):
    p = po.problem_diag(300, 4, 4, 64, 32, 2, 9, "long")
    p.s0 = np.random.default_rng(2).standard_normal(p.s0.shape).astype(np.float32) * 0.3
    p.ids = np.array([1, 3, 0, 2], np.int32)
    y_ref, s_ref = po.scan(p, use_ids=True)
    d = p.d.copy()
    d.backend = HELIX_BACKEND_AUTO
    _, y, s1 = run(gpu, p, desc=d, use_ids=True)
    _check(y, s1, y_ref, s_ref)
