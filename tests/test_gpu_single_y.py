"""The single pass (multipass = false) run as the fp32 path's three passes with
its state tiles in y: which shapes take that form, parity against the fp64
oracle at the fp32 per-element bound, and the encoder's fallback to the
one-launch kernel when y is misaligned or overlaps an input.

The tiles (Pass A's segment aggregates, then the walks' start states) and the
segment log-decays are written into y's rows of their own segment and the
columns of their own (head, P slab), and read back before the walk overwrites
them with y; shapes whose last segment is too short for a tile keep the
one-launch kernel (tests/test_host.py checks the plans on the CPU).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from helix_amd.desc import HELIX_OK, HELIX_TENSOR_NULL
from gpu_harness import F32_ABS, F32_REL, T, ctx_for, run, upload

pytestmark = pytest.mark.gpu

# (L, S, H, P, N, G, label): every one plans state_in_y.
Y_SHAPES = [
    (1000, 3, 4, 80, 128, 2, "P=80: a 16-channel last slab, 513-row tiles"),
    (2112, 2, 6, 64, 64, 3, "d_state 64, two sequences"),
    (700, 2, 4, 192, 128, 1, "three slabs"),
    (4160, 1, 8, 64, 128, 8, "one head per group, lengthened segments"),
    (2048, 1, 64, 64, 128, 8, "config 1's shape"),
]


def _problem(shape, seed, memory="long"):
    L, S, H, P, N, G, _ = shape
    p = po.problem_harness(L, S, H, P, N, G, seed, memory)
    d = p.d.copy()
    d.multipass = False
    return p, d


def _check(y, s1, y_ref, s_ref, what):
    ry = po.allclose_ratio(y, y_ref, F32_REL, F32_ABS)
    rs = po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS)
    print(f"{what:48s} y ratio {ry:.3f}  s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)


@pytest.mark.parametrize("shape", Y_SHAPES, ids=[s[-1] for s in Y_SHAPES])
def test_state_in_y_parity(gpu, shape):
    p, d = _problem(shape, 4343)
    info = gpu.plan_info(d)
    assert (info.state_in_y, info.launches, info.total_bytes) == (1, 3, 0)
    assert gpu.scratch_size(d) == 0
    y_ref, s_ref = po.scan(p, threads=0)
    _, y, s1 = run(gpu, p, desc=d)
    _check(y, s1, y_ref, s_ref, shape[-1])


def test_state_in_y_ids(gpu):
    # s0 rows picked through ids (a permutation), so s0 is left out of the
    # overlap check and read by Pass B through ids.
    shape = (1500, 3, 4, 64, 128, 2, "ids")
    p, d = _problem(shape, 4344)
    p.s0 = np.random.default_rng(6).standard_normal(p.s0.shape).astype(np.float32) * 0.3
    p.ids = np.array([2, 0, 1], np.int32)
    assert gpu.plan_info(d).state_in_y == 1
    y_ref, s_ref = po.scan(p, use_ids=True)
    _, y, s1 = run(gpu, p, desc=d, use_ids=True)
    _check(y, s1, y_ref, s_ref, "ids permutation")


def test_fallback_y_in_place(gpu):
    # y over x (in place): the tiles would overwrite x before the walk reads
    # it, so the encoder runs the one-launch kernel, which reads each chunk
    # of x before it writes that chunk's y.
    shape = (1100, 1, 4, 64, 128, 2, "in place")
    p, d = _problem(shape, 4345)
    assert gpu.plan_info(d).state_in_y == 1
    assert list(d.s_x) == list(d.s_y) and d.seq_x == d.seq_y
    y_ref, s_ref = po.scan(p, threads=0)
    xy = upload(p.x)
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    dev = {k: upload(getattr(p, k)) for k in ("s0", "dt", "A", "B", "C")}
    rc = gpu.encode(torch.cuda.current_stream().cuda_stream, d, T(dev["s0"]), T(xy), T(dev["dt"]), T(dev["A"]),
                    T(dev["B"]), T(dev["C"]), HELIX_TENSOR_NULL, T(xy), T(s1), HELIX_TENSOR_NULL)
    assert rc == HELIX_OK, gpu.last_error()
    torch.cuda.synchronize()
    _check(xy.cpu().numpy(), s1.cpu().numpy(), y_ref, s_ref, "y over x: one launch")


def test_fallback_y_misaligned(gpu):
    # y 4 bytes past a 16-byte boundary: the 16-byte tile units do not fit,
    # so the one-launch kernel runs; the result is the same scan.
    shape = (1100, 1, 4, 64, 128, 2, "misaligned")
    p, d = _problem(shape, 4346)
    y_ref, s_ref = po.scan(p, threads=0)
    n = int(np.prod(p.y_shape()))
    buf = torch.full((n + 4,), float("nan"), device="cuda")
    y = buf[1:1 + n].view(p.y_shape())
    assert y.data_ptr() % 16 == 4
    _, y_out, s1 = run(gpu, p, desc=d, y_gpu=y)
    _check(y_out, s1, y_ref, s_ref, "y misaligned: one launch")


def test_state_in_y_matches_one_launch(gpu):
    # The two forms of the single pass agree to the fp32 bound on a shape with
    # ragged chunks and two sequences (HELIX_1PASS_Y=0 pins the one launch).
    shape = (3000, 2, 8, 64, 128, 4, "both forms")
    p, d = _problem(shape, 4347)
    one = ctx_for(gpu, HELIX_1PASS_Y="0")
    assert gpu.plan_info(d).state_in_y == 1 and one.plan_info(d).state_in_y == 0
    _, y_a, s_a = run(gpu, p, desc=d)
    _, y_b, s_b = run(one, p, desc=d)
    assert po.allclose_ratio(y_a, y_b, F32_REL, F32_ABS) <= 1.0
    assert po.allclose_ratio(s_a, s_b, F32_REL, F32_ABS) <= 1.0
