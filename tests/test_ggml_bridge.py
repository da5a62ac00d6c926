"""The ggml HIP-backend bridge (helix_amd/integration/ggml), without a GPU.

Counterpart of the reference's integration/ggml/ggml-helix.cpp:157-280
(build_desc). The bridge is compiled against a test-only stand-in of ggml.h
(tests/ggml_stub), since llama.cpp is absent offline: the ne/nb -> element
stride mapping, the dst = [y | state] packing and the gates (K == 1, all
f32, GGML_HELIX_MIN_TOKENS, the A form, GGML_HELIX_MPP, GGML_HELIX_DISABLE)
are checked here; its encode is checked on the GPU against the oracle
(tests/test_gpu_ggml_bridge.py). Against a real ggml build the bridge stays
"parity unpinned".
"""
from __future__ import annotations

import ctypes
import math

import pytest

from helix_amd import abi
from helix_amd.desc import (HELIX_A_DIAG_PER_CHANNEL, HELIX_A_SCALAR_PER_HEAD, HELIX_BACKEND_AUTO,
                            HELIX_BACKEND_SGMMA, HelixScanDesc, desc_init)
from ggml_fake import GGML_TYPE_F16, SsmScanOp, bridge, tensor
from gpu_harness import env


def build(op):
    d = HelixScanDesc()
    ok = bridge().helix_ggml_build_desc(op.ref(), ctypes.byref(d))
    return ok, d


def test_dense_mapping_equals_desc_init():
    L, S, H, P, N, G = 300, 2, 8, 64, 128, 2
    ok, d = build(SsmScanOp(L, S, H, P, N, G))
    assert ok
    want = desc_init(L, S, H, P, N, G)
    want.multipass = True
    want.backend = HELIX_BACKEND_SGMMA
    want.dt_min, want.dt_max = 0.0, math.inf
    assert bytes(d) == bytes(want)
    host = abi.Context(host_only=True)
    try:
        assert host.supported(d)
        assert host.backend_desc(d).startswith("mfma fp32")
    finally:
        host.close()


def test_padded_x_rows_map_to_element_strides():
    L, S, H, P, N, G = 200, 2, 4, 64, 128, 1
    ok, d = build(SsmScanOp(L, S, H, P, N, G, x_row_pad=16))
    assert ok
    assert list(d.s_x) == [H * P + 16, P, 1] and d.seq_x == (H * P + 16) * L
    # y stays dense in x's logical shape: it is the leading region of dst.
    assert list(d.s_y) == [H * P, P, 1] and d.seq_y == H * P * L


def test_mpp_switch_selects_auto():
    with env(GGML_HELIX_MPP="1"):
        ok, d = build(SsmScanOp(256, 1, 8, 64, 128, 2))
    assert ok and d.backend == HELIX_BACKEND_AUTO
    ok, d = build(SsmScanOp(256, 1, 8, 64, 128, 2))
    assert ok and d.backend == HELIX_BACKEND_SGMMA


def test_a_forms():
    ok, d = build(SsmScanOp(256, 1, 4, 64, 128, 1))
    assert ok and d.a_form == HELIX_A_SCALAR_PER_HEAD and d.s_a == 1
    ok, d = build(SsmScanOp(256, 1, 4, 64, 128, 1, a_diag=True))
    assert ok and d.a_form == HELIX_A_DIAG_PER_CHANNEL and d.s_a == 128
    op = SsmScanOp(256, 1, 4, 64, 128, 1)
    op.A = tensor((3, 4), (4, 12))
    op.relink()
    assert not build(op)[0]


def test_min_tokens_gate():
    assert not build(SsmScanOp(63, 1, 4, 64, 128, 1))[0]
    assert build(SsmScanOp(64, 1, 4, 64, 128, 1))[0]
    with env(GGML_HELIX_MIN_TOKENS="1"):
        assert build(SsmScanOp(1, 1, 4, 64, 128, 1))[0]
    with env(GGML_HELIX_MIN_TOKENS="512"):
        assert not build(SsmScanOp(300, 1, 4, 64, 128, 1))[0]


@pytest.mark.parametrize("why,mutate", [
    ("K = 2 snapshots", lambda op: op.dst.op_params.__setitem__(0, 2)),
    ("K = 0", lambda op: op.dst.op_params.__setitem__(0, 0)),
    ("f16 x", lambda op: setattr(op.x, "type", GGML_TYPE_F16)),
    ("f16 dst", lambda op: setattr(op.dst, "type", GGML_TYPE_F16)),
    ("heads not a multiple of groups", lambda op: op.B.ne.__setitem__(1, 3)),
    ("padded state rows", lambda op: op.s.nb.__setitem__(1, 4 * 128 + 16)),
    ("byte stride not whole elements", lambda op: op.x.nb.__setitem__(2, 4 * 8 * 64 + 2)),
    ("missing C", lambda op: op.dst.src.__setitem__(5, ctypes.POINTER(type(op.C))())),
])
def test_gates_decline(why, mutate):
    op = SsmScanOp(256, 2, 8, 64, 128, 2)
    assert build(op)[0]
    mutate(op)
    assert not build(op)[0], why


def test_plan_declines_without_a_device_and_when_disabled():
    op = SsmScanOp(256, 1, 4, 64, 128, 1)
    n = ctypes.c_size_t(123)
    with env(GGML_HELIX_DISABLE="1"):
        assert not bridge().ggml_hip_ssm_scan_helix_plan(0, op.ref(), ctypes.byref(n))
    try:
        import torch
        has_gpu = torch.cuda.is_available()
    except Exception:
        has_gpu = False
    if not has_gpu:
        # No HIP device: the context cannot be created and the op falls back.
        assert not bridge().ggml_hip_ssm_scan_helix_plan(0, op.ref(), ctypes.byref(n))
        assert not bridge().ggml_hip_op_ssm_scan_helix(None, 0, op.ref(), None, 0)
