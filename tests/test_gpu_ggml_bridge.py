"""The ggml HIP-backend bridge on the GPU: SSM_SCAN operands laid out as ggml
hands them over (tests/ggml_fake.py over device buffers), encoded through
ggml_hip_op_ssm_scan_helix, and dst = [y | final state] checked against the
fp64 oracle. Counterpart of the reference's integration/ggml/
ggml-helix.cpp:286-361. Covers the default fp32 path and GGML_HELIX_MPP=1,
scratch from the caller's pool and from the bridge's own buffer, ids, padded
token rows, and the fall-through (nothing written) for a declined op.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from ggml_fake import SsmScanOp, bridge
from gpu_harness import BF16_GATE, F32_ABS, F32_GATE, F32_REL, env, upload

pytestmark = pytest.mark.gpu


def _problem(L, S, H, P, N, G, seed, ids=None):
    p = po.problem_harness(L, S, H, P, N, G, seed, "long")
    p.s0 = np.random.default_rng(seed).standard_normal(p.s0.shape).astype(np.float32) * 0.2
    p.ids = None if ids is None else np.asarray(ids, np.int32)
    return p


def _run(p, pool_scratch=True, x_row_pad=0, mpp=False):
    L, S, H, P, N, G = p.shape
    dev = {k: upload(getattr(p, k)) for k in ("s0", "dt", "A", "B", "C")}
    if x_row_pad:
        xb = torch.full((S, L, H * P + x_row_pad), float("nan"), device="cuda")
        xb[:, :, :H * P] = upload(p.x).reshape(S, L, H * P)
        dev["x"] = xb
    else:
        dev["x"] = upload(p.x)
    if p.ids is not None:
        dev["ids"] = upload(p.ids)
    n_y, n_s = S * L * H * P, S * H * P * N
    dst = torch.full((n_y + n_s,), float("nan"), device="cuda")
    ptrs = {k: t.data_ptr() for k, t in dev.items()}
    ptrs["dst"] = dst.data_ptr()
    op = SsmScanOp(L, S, H, P, N, G, ptrs=ptrs, x_row_pad=x_row_pad)
    B = bridge()
    stream = torch.cuda.current_stream()
    with env(GGML_HELIX_MPP="1" if mpp else None):
        need = ctypes.c_size_t(0)
        served = B.ggml_hip_ssm_scan_helix_plan(0, op.ref(), ctypes.byref(need))
        scratch = None
        if served and pool_scratch and need.value:
            scratch = torch.empty(need.value, dtype=torch.uint8, device="cuda")
        ok = B.ggml_hip_op_ssm_scan_helix(ctypes.c_void_p(stream.cuda_stream), 0, op.ref(),
                                          ctypes.c_void_p(scratch.data_ptr() if scratch is not None else 0),
                                          need.value if scratch is not None else 0)
    torch.cuda.synchronize()
    out = dst.cpu().numpy()
    return served, ok, out[:n_y].reshape(S, L, H, P), out[n_y:].reshape(S, H, P, N)


CASES = [
    # (label, shape, ids, pool scratch, x_row_pad, mpp)
    ("fp32 ragged", (300, 2, 8, 64, 128, 2), None, True, 0, False),
    ("fp32 ids, own scratch", (300, 4, 4, 64, 128, 2), [2, 0, 3, 1], False, 0, False),
    ("fp32 padded x rows", (200, 2, 4, 64, 128, 1), None, True, 16, False),
    ("fp32 d_state 256", (256, 1, 4, 128, 256, 1), None, True, 0, False),
    ("bf16 (GGML_HELIX_MPP=1)", (1000, 1, 8, 64, 128, 2), None, True, 0, True),
    ("bf16 ids, own scratch", (300, 4, 4, 64, 128, 2), [3, 2, 1, 0], False, 0, True),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_bridge_parity(gpu, case):
    label, shape, ids, pool, pad, mpp = case
    p = _problem(*shape, 4242, ids)
    y_ref, s_ref = po.scan(p, use_ids=ids is not None)
    served, ok, y, s1 = _run(p, pool_scratch=pool, x_row_pad=pad, mpp=mpp)
    assert served and ok, label
    gate = BF16_GATE if mpp else F32_GATE
    ey, es = po.max_rel_err(y, y_ref), po.max_rel_err(s1, s_ref)
    print(f"{label}: y {ey:.2e} s1 {es:.2e}", flush=True)
    assert ey <= gate and es <= F32_GATE
    if not mpp:
        # The default path meets the fp32 per-element bound (ggml's op test is
        # an fp32 bar; reference integration/ggml/README.md:43-55).
        assert po.allclose_ratio(y, y_ref, F32_REL, F32_ABS) <= 1.0
    # The carried state stays at the fp32 per-element bound on both paths.
    assert po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS) <= 1.0


def test_declined_op_writes_nothing(gpu):
    p = _problem(40, 1, 4, 64, 128, 1, 7)       # shorter than GGML_HELIX_MIN_TOKENS
    served, ok, y, s1 = _run(p)
    assert not served and not ok
    assert np.all(np.isnan(y)) and np.all(np.isnan(s1))
    with env(GGML_HELIX_MIN_TOKENS="1"):
        served, ok, y, s1 = _run(p)
    y_ref, s_ref = po.scan(p, use_ids=False)
    assert served and ok and po.max_rel_err(y, y_ref) <= F32_GATE
