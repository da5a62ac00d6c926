"""Blocks of state indices: above d_state 256 the scan runs as blocks of at
most 128 state indices on the fp32 path, and from 129 to 256 (fp32 storage,
scalar A) on whichever path the descriptor asks for; block k reads B, C and
s0 and writes s1 at its first state index and adds its share of y into y
(HelixScanParams::y_acc; the walks of the later blocks load y ahead). On the
bf16 path each block's Pass A writes bf16 copies of its columns of B and C for
its walk.

Parity against the fp64 oracle (pinned at these d_state against the
reference's own ref::scan and for the block decomposition itself in
tests/test_oracle.py) at the fp32 per-element bound, on the multipass plan,
the single pass, a plan of many super-chunk groups carried through s1, ids
with a nonzero s0, and the no-allocation entry point; the encoder's refusal
of a y that overlaps an input above 256, which the blocks would read after an
earlier block had written y, and its fallback to the one-launch single pass
for such a y up to 256.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from helix_amd.desc import (HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA, HELIX_ERR_INVALID_ARG,
                            HELIX_OK, HELIX_TENSOR_NULL)
from gpu_harness import BF16_ABS, BF16_REL, F32_ABS, F32_REL, T, ctx_for, run, upload

pytestmark = pytest.mark.gpu

# (L, S, H, P, N, G, label)
SHAPES = [
    (600, 2, 4, 64, 264, 2, "N=264: three blocks of 88"),
    (1100, 1, 4, 96, 384, 2, "N=384, P=96: a 32-channel last slab"),
    (333, 3, 2, 64, 512, 1, "N=512: four blocks, ragged last chunk"),
]


def _check(y, s1, y_ref, s_ref, what):
    ry = po.allclose_ratio(y, y_ref, F32_REL, F32_ABS)
    rs = po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS)
    print(f"{what:48s} y ratio {ry:.3f}  s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)


def _problem(shape, seed, multipass=True):
    L, S, H, P, N, G, _ = shape
    p = po.problem_harness(L, S, H, P, N, G, seed, "long")
    p.s0 = np.random.default_rng(seed).standard_normal(p.s0.shape).astype(np.float32) * 0.3
    d = p.d.copy()
    d.multipass = multipass
    return p, d


@pytest.mark.parametrize("multipass", [True, False], ids=["multipass", "single"])
@pytest.mark.parametrize("shape", SHAPES, ids=[s[-1] for s in SHAPES])
def test_state_blocks_parity(gpu, shape, multipass):
    p, d = _problem(shape, 5151, multipass)
    info = gpu.plan_info(d)
    assert info.state_blocks > 1 and gpu.select_backend(d) == HELIX_BACKEND_SGMMA
    y_ref, s_ref = po.scan(p, threads=0)
    _, y, s1 = run(gpu, p, desc=d)
    _check(y, s1, y_ref, s_ref, f"{shape[-1]} {'multipass' if multipass else 'single'}")


def test_state_blocks_ids_and_groups(gpu):
    # ids pick s0 rows in reverse; a 1 MiB scratch budget cuts the plan into
    # many super-chunk groups, each block carrying its state columns through s1.
    shape = (900, 3, 4, 64, 320, 2, "ids, many groups")
    p, d = _problem(shape, 5152)
    p.ids = np.array([2, 0, 1], np.int32)
    small = ctx_for(gpu, HELIX_SCRATCH_MB="1")
    info = small.plan_info(d)
    assert info.state_blocks == 3 and info.n_groups > 1
    y_ref, s_ref = po.scan(p, use_ids=True, threads=0)
    _, y, s1 = run(small, p, desc=d, use_ids=True)
    _check(y, s1, y_ref, s_ref, "ids, many groups")


def test_state_blocks_noalloc(gpu):
    # The blocks run one after another in the library's fixed scratch.
    shape = (700, 2, 4, 64, 384, 2, "noalloc")
    p, d = _problem(shape, 5153)
    y_ref, s_ref = po.scan(p, threads=0)
    dev = {k: upload(getattr(p, k)) for k in ("s0", "x", "dt", "A", "B", "C")}
    y = torch.full(p.y_shape(), float("nan"), device="cuda")
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    rc = gpu.encode_noalloc(torch.cuda.current_stream().cuda_stream, d, T(dev["s0"]), T(dev["x"]), T(dev["dt"]),
                            T(dev["A"]), T(dev["B"]), T(dev["C"]), HELIX_TENSOR_NULL, T(y), T(s1))
    assert rc == HELIX_OK, gpu.last_error()
    torch.cuda.synchronize()
    _check(y.cpu().numpy(), s1.cpu().numpy(), y_ref, s_ref, "noalloc")


@pytest.mark.parametrize("multipass", [True, False], ids=["multipass", "single"])
def test_state_blocks_refuse_y_over_x(gpu, multipass):
    # y in place over x: the second block would read x where the first wrote
    # y. Refused before anything is enqueued: x is untouched.
    shape = (300, 1, 2, 64, 264, 1, "in place")
    p, d = _problem(shape, 5154, multipass)
    xy = upload(p.x)
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    dev = {k: upload(getattr(p, k)) for k in ("s0", "dt", "A", "B", "C")}
    n = gpu.scratch_size(d)
    scratch = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
    rc = gpu.encode(torch.cuda.current_stream().cuda_stream, d, T(dev["s0"]), T(xy), T(dev["dt"]), T(dev["A"]),
                    T(dev["B"]), T(dev["C"]), HELIX_TENSOR_NULL, T(xy), T(s1), T(scratch))
    assert rc == HELIX_ERR_INVALID_ARG
    assert "overlaps" in gpu.last_error()
    torch.cuda.synchronize()
    assert np.array_equal(xy.cpu().numpy(), p.x)
    assert torch.isnan(s1).all()


# d_state 129..256: blocks by default, on the path the descriptor asks for.
MID_SHAPES = [
    (600, 2, 4, 64, 256, 2, "N=256: two blocks of 128"),
    (700, 1, 4, 96, 192, 2, "N=192, P=96: two blocks of 96"),
    (333, 2, 2, 64, 160, 1, "N=160: two blocks of 80, ragged last chunk"),
    # 20 heads per group: the bf16 path's Pass A writes bf16 copies of each
    # block's B and C columns for the walks.
    (400, 1, 20, 64, 256, 1, "N=256, 20 heads per group: copies of B and C"),
]
MID_MODES = [("bf16", HELIX_BACKEND_MPP, True), ("fp32", HELIX_BACKEND_SGMMA, True),
             ("single", HELIX_BACKEND_AUTO, False)]


@pytest.mark.parametrize("mode", MID_MODES, ids=[m[0] for m in MID_MODES])
@pytest.mark.parametrize("shape", MID_SHAPES, ids=[s[-1] for s in MID_SHAPES])
def test_blocks_up_to_256_parity(gpu, shape, mode):
    label, backend, multipass = mode
    p, d = _problem(shape, 5161, multipass)
    d.backend = backend
    assert gpu.plan_info(d).state_blocks == 2
    y_ref, s_ref = po.scan(p, threads=0)
    _, y, s1 = run(gpu, p, desc=d)
    rel, ab = (BF16_REL, BF16_ABS) if label == "bf16" else (F32_REL, F32_ABS)
    ry = po.allclose_ratio(y, y_ref, rel, ab)
    rs = po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS)
    print(f"{shape[-1]:44s} {label:6s} y ratio {ry:.3f}  s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)


@pytest.mark.parametrize("backend", [HELIX_BACKEND_AUTO, HELIX_BACKEND_SGMMA], ids=["auto", "fp32"])
def test_blocks_up_to_256_y_over_x_runs_one_launch(gpu, backend):
    # y in place over x at d_state 256: the blocks cannot run (the second would
    # read x where the first wrote y), so the encoder runs the one-launch
    # single pass, which reads each chunk of x before it writes its y and
    # needs no scratch. fp32-accurate, whatever the descriptor's backend.
    shape = (500, 1, 4, 64, 256, 2, "in place")
    p, d = _problem(shape, 5162)
    d.backend = backend
    assert list(d.s_x) == list(d.s_y) and d.seq_x == d.seq_y
    y_ref, s_ref = po.scan(p, threads=0)
    xy = upload(p.x)
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    dev = {k: upload(getattr(p, k)) for k in ("s0", "dt", "A", "B", "C")}
    n = gpu.scratch_size(d)
    scratch = torch.empty(max(n, 1), dtype=torch.uint8, device="cuda")
    rc = gpu.encode(torch.cuda.current_stream().cuda_stream, d, T(dev["s0"]), T(xy), T(dev["dt"]), T(dev["A"]),
                    T(dev["B"]), T(dev["C"]), HELIX_TENSOR_NULL, T(xy), T(s1), T(scratch))
    assert rc == HELIX_OK, gpu.last_error()
    torch.cuda.synchronize()
    _check(xy.cpu().numpy(), s1.cpu().numpy(), y_ref, s_ref, "N=256 y over x: one launch")


def test_blocks_match_one_launch_sequence(gpu):
    # Blocks and the d_state 256 kernels (HELIX_STATE_BLOCKS=0) agree on the
    # fp32 path to the fp32 bound.
    shape = (900, 2, 4, 64, 256, 2, "blocks vs one sequence")
    p, d = _problem(shape, 5163)
    d.backend = HELIX_BACKEND_SGMMA
    native = ctx_for(gpu, HELIX_STATE_BLOCKS="0")
    assert gpu.plan_info(d).state_blocks == 2 and native.plan_info(d).state_blocks == 1
    _, y_a, s_a = run(gpu, p, desc=d)
    _, y_b, s_b = run(native, p, desc=d)
    assert po.allclose_ratio(y_a, y_b, F32_REL, F32_ABS) <= 1.0
    assert po.allclose_ratio(s_a, s_b, F32_REL, F32_ABS) <= 1.0


@pytest.mark.parametrize("heads", [4, 20], ids=["4 heads per group", "20 heads per group"])
def test_blocks_up_to_256_copies_ids_and_groups(gpu, heads):
    # The bf16 path's blocks with copies of B and C: ids pick s0 rows in
    # reverse, and a 1 MiB scratch budget cuts the plan into many super-chunk
    # groups, each group's Pass A copying its chunks' columns of B and C for
    # that group's walks, the state carried through s1's columns of the block.
    G = 2 if heads == 4 else 1
    shape = (900, 3, heads * G, 64, 256, G, "copies, ids, many groups")
    p, d = _problem(shape, 5164)
    d.backend = HELIX_BACKEND_MPP
    p.ids = np.array([2, 0, 1], np.int32)
    small = ctx_for(gpu, HELIX_SCRATCH_MB="1")
    info = small.plan_info(d)
    assert info.state_blocks == 2 and info.n_groups > 1 and info.bccopy_bytes > 0
    y_ref, s_ref = po.scan(p, use_ids=True, threads=0)
    _, y, s1 = run(small, p, desc=d, use_ids=True)
    ry = po.allclose_ratio(y, y_ref, BF16_REL, BF16_ABS)
    rs = po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS)
    print(f"{heads} heads per group: y ratio {ry:.3f}  s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)


def test_blocks_up_to_256_noalloc(gpu):
    # The bf16 path's blocks, copies included, in the library's fixed scratch.
    shape = (700, 2, 4, 64, 256, 2, "noalloc, N=256")
    p, d = _problem(shape, 5165)
    d.backend = HELIX_BACKEND_MPP
    assert gpu.plan_info(d).bccopy_bytes > 0
    y_ref, s_ref = po.scan(p, threads=0)
    dev = {k: upload(getattr(p, k)) for k in ("s0", "x", "dt", "A", "B", "C")}
    y = torch.full(p.y_shape(), float("nan"), device="cuda")
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    rc = gpu.encode_noalloc(torch.cuda.current_stream().cuda_stream, d, T(dev["s0"]), T(dev["x"]), T(dev["dt"]),
                            T(dev["A"]), T(dev["B"]), T(dev["C"]), HELIX_TENSOR_NULL, T(y), T(s1))
    assert rc == HELIX_OK, gpu.last_error()
    torch.cuda.synchronize()
    ry = po.allclose_ratio(y.cpu().numpy(), y_ref, BF16_REL, BF16_ABS)
    rs = po.allclose_ratio(s1.cpu().numpy(), s_ref, F32_REL, F32_ABS)
    print(f"noalloc N=256 bf16: y ratio {ry:.3f}  s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)
