"""helix_scan_encode_noalloc on the GPU, through the C ABI.

The entry point runs helix_scan_encode's plan and kernels on the library's
fixed scratch array instead of a caller's buffer, so its outputs must be
bitwise equal to helix_scan_encode's on the same inputs (the scan is
deterministic), and within the oracle's tolerance. Two calls in a row, the
second on a smaller problem, so the second runs on what the first left in the
array. A scan whose plan would need more than the array is planned for it
(more super-chunk groups): bitwise equal to helix_scan_encode under the same
budget. One that does not fit at one chunk per group is refused and writes
nothing.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from helix_amd import abi
from helix_amd.desc import (HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA,
                            HELIX_ERR_SCRATCH_TOO_SMALL, HELIX_OK, HELIX_TENSOR_NULL)
from gpu_harness import BF16_GATE, F32_GATE, T, ctx_for, upload

pytestmark = pytest.mark.gpu

PATHS = [("bf16", HELIX_BACKEND_MPP, True), ("fp32", HELIX_BACKEND_SGMMA, True),
         ("1pass", HELIX_BACKEND_AUTO, False)]
# (shape L, S, H, P, N, G), larger first
CALLS = [(2048, 2, 8, 64, 128, 2), (300, 1, 4, 64, 128, 1)]


def _encode(gpu, p, d, noalloc):
    dev = {k: upload(getattr(p, k)) for k in ("s0", "x", "dt", "A", "B", "C")}
    y = torch.full(p.y_shape(), float("nan"), device="cuda")
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    args = [T(dev[k]) for k in ("s0", "x", "dt", "A", "B", "C")]
    if noalloc:
        rc = gpu.encode_noalloc(stream, d, *args, HELIX_TENSOR_NULL, T(y), T(s1))
    else:
        need = gpu.scratch_size(d)
        scratch = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        rc = gpu.encode(stream, d, *args, HELIX_TENSOR_NULL, T(y), T(s1), T(scratch))
    assert rc == HELIX_OK, gpu.last_error()
    torch.cuda.synchronize()
    return y.cpu().numpy(), s1.cpu().numpy()


@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
def test_noalloc_matches_encode(gpu, path):
    label, backend, multipass = path
    for i, shape in enumerate(CALLS):
        p = po.problem_harness(*shape, 900 + i, "long")
        d = p.d.copy()
        d.backend = backend
        d.multipass = multipass
        assert gpu.scratch_size(d) <= abi.NOALLOC_SCRATCH_BYTES
        print(f"[noalloc {label}] call {i + 1} shape {shape} scratch {gpu.scratch_size(d)} B", flush=True)
        y_a, s_a = _encode(gpu, p, d, noalloc=False)
        y_b, s_b = _encode(gpu, p, d, noalloc=True)
        assert y_a.tobytes() == y_b.tobytes() and s_a.tobytes() == s_b.tobytes(), (label, shape)
        y_ref, s_ref = po.scan(p, threads=0)
        gate = BF16_GATE if label == "bf16" else F32_GATE
        assert po.max_rel_err(y_b, y_ref) <= gate and po.max_rel_err(s_b, s_ref) <= F32_GATE


def test_noalloc_refuses_oversized_plan(gpu):
    # d_state 256 on the fp32 path, 4096 heads: Pass A stores every chunk's
    # state, 256 MiB for one chunk, so not even one chunk per group fits.
    p = po.problem_harness(64, 1, 4096, 64, 256, 1, 5, "short")
    d = p.d.copy()
    d.backend = HELIX_BACKEND_SGMMA
    d.multipass = True
    assert gpu.scratch_size(d) > abi.NOALLOC_SCRATCH_BYTES
    dev = {k: upload(getattr(p, k)) for k in ("s0", "x", "dt", "A", "B", "C")}
    y = torch.full(p.y_shape(), float("nan"), device="cuda")
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    args = [T(dev[k]) for k in ("s0", "x", "dt", "A", "B", "C")]
    rc = gpu.encode_noalloc(torch.cuda.current_stream().cuda_stream, d, *args, HELIX_TENSOR_NULL, T(y), T(s1))
    assert rc == HELIX_ERR_SCRATCH_TOO_SMALL
    assert "HELIX_NOALLOC_SCRATCH_BYTES" in gpu.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(y).all() and torch.isnan(s1).all()


def test_noalloc_headline_shape(gpu):
    # BASELINE config 2 on the bf16 path: its plan fits the fixed scratch.
    p = po.problem_gauss(8192, 1, 64, 64, 128, 8, 1002)
    d = p.d.copy()
    d.backend = HELIX_BACKEND_MPP
    d.multipass = True
    assert gpu.scratch_size(d) <= abi.NOALLOC_SCRATCH_BYTES
    y_a, s_a = _encode(gpu, p, d, noalloc=False)
    y_b, s_b = _encode(gpu, p, d, noalloc=True)
    assert np.array_equal(y_a, y_b) and np.array_equal(s_a, s_b)


def test_noalloc_config4a(gpu):
    # BASELINE config 4a on the bf16 path: 76 MiB of scratch, within the
    # fixed array; the same plan and kernels as helix_scan_encode, bitwise.
    p = po.problem_gauss(4096, 8, 80, 64, 128, 1, 1004, 0.1)
    d = p.d.copy()
    d.backend = HELIX_BACKEND_MPP
    d.multipass = True
    assert 0 < gpu.scratch_size(d) <= abi.NOALLOC_SCRATCH_BYTES
    y_a, s_a = _encode(gpu, p, d, noalloc=False)
    y_b, s_b = _encode(gpu, p, d, noalloc=True)
    assert y_a.tobytes() == y_b.tobytes() and s_a.tobytes() == s_b.tobytes()


def test_noalloc_capped_plan(gpu):
    # Config 4a's shape with fourteen sequences on the bf16 path: 168 MiB of
    # scratch under the default budget, so the entry point plans it for its
    # 128 MiB array in several groups carried through s1, as
    # helix_scan_encode does with HELIX_SCRATCH_MB=128 (bitwise), and close to
    # the default plan's result.
    p = po.problem_gauss(4096, 14, 80, 64, 128, 1, 1004, 0.1)
    d = p.d.copy()
    d.backend = HELIX_BACKEND_MPP
    d.multipass = True
    assert gpu.scratch_size(d) > abi.NOALLOC_SCRATCH_BYTES
    capped = ctx_for(gpu, HELIX_SCRATCH_MB=abi.NOALLOC_SCRATCH_BYTES >> 20)
    assert capped.plan_info(d).n_groups > 1
    y_n, s_n = _encode(gpu, p, d, noalloc=True)
    y_c, s_c = _encode(capped, p, d, noalloc=False)
    assert y_n.tobytes() == y_c.tobytes() and s_n.tobytes() == s_c.tobytes()
    y_d, s_d = _encode(gpu, p, d, noalloc=False)
    assert po.max_rel_err(y_n, y_d) <= BF16_GATE and po.max_rel_err(s_n, s_d) <= F32_GATE
