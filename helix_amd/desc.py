"""ctypes mirror of the HELIX C ABI types (include/helix/helix.h).

Field order, types and enum values are those of the reference ABI
(reference include/helix/helix.h:42-131, HELIX_ABI_VERSION 1); tests check the
layout against the C library and against the reference's own header.

`desc_init` restates the reference's dense-stride defaults
(reference src/runtime/desc.cpp:9-46) for Python callers; the C library's
`helix_scan_desc_init` is the authoritative copy and tests hold the two equal.
"""
from __future__ import annotations

import ctypes
import math
from ctypes import c_bool, c_float, c_int, c_int32, c_int64, c_uint64, c_void_p

HELIX_ABI_VERSION = 1

# helix_status
HELIX_OK = 0
HELIX_ERR_UNSUPPORTED_SHAPE = 1
HELIX_ERR_NO_DEVICE = 2
HELIX_ERR_SCRATCH_TOO_SMALL = 3
HELIX_ERR_INVALID_ARG = 4
HELIX_ERR_PIPELINE = 5

STATUS_NAMES = {
    HELIX_OK: "HELIX_OK",
    HELIX_ERR_UNSUPPORTED_SHAPE: "HELIX_ERR_UNSUPPORTED_SHAPE",
    HELIX_ERR_NO_DEVICE: "HELIX_ERR_NO_DEVICE",
    HELIX_ERR_SCRATCH_TOO_SMALL: "HELIX_ERR_SCRATCH_TOO_SMALL",
    HELIX_ERR_INVALID_ARG: "HELIX_ERR_INVALID_ARG",
    HELIX_ERR_PIPELINE: "HELIX_ERR_PIPELINE",
}

# helix_dtype
HELIX_F32 = 0
HELIX_F16 = 1
HELIX_BF16 = 2

# helix_a_form
HELIX_A_SCALAR_PER_HEAD = 0
HELIX_A_DIAG_PER_CHANNEL = 1

# helix_backend
HELIX_BACKEND_AUTO = 0
HELIX_BACKEND_SGMMA = 1
HELIX_BACKEND_MPP = 2
HELIX_BACKEND_REF = 3


class HelixScanDesc(ctypes.Structure):
    """helix_scan_desc: logical shape, element strides and algorithm knobs."""

    _fields_ = [
        ("n_tok", c_int32),
        ("n_seq", c_int32),
        ("n_head", c_int32),
        ("head_dim", c_int32),
        ("d_state", c_int32),
        ("n_group", c_int32),
        ("s_x", c_int64 * 3),
        ("s_b", c_int64 * 3),
        ("s_c", c_int64 * 3),
        ("s_dt", c_int64 * 2),
        ("s_s", c_int64 * 3),
        ("s_y", c_int64 * 3),
        ("s_a", c_int64),
        ("seq_x", c_int64),
        ("seq_b", c_int64),
        ("seq_c", c_int64),
        ("seq_dt", c_int64),
        ("seq_s", c_int64),
        ("seq_y", c_int64),
        ("chunk", c_int32),
        ("a_form", c_int),
        ("io_dtype", c_int),
        ("compute_dtype", c_int),
        ("backend", c_int),
        ("multipass", c_bool),
        ("dt_min", c_float),
        ("dt_max", c_float),
    ]

    def copy(self) -> "HelixScanDesc":
        out = HelixScanDesc()
        ctypes.memmove(ctypes.byref(out), ctypes.byref(self), ctypes.sizeof(self))
        return out

    def as_dict(self) -> dict:
        d = {}
        for name, _ in self._fields_:
            v = getattr(self, name)
            d[name] = list(v) if isinstance(v, ctypes.Array) else v
        return d


class HelixTensor(ctypes.Structure):
    """helix_tensor: device pointer plus a byte offset."""

    _fields_ = [("buf", c_void_p), ("offset", c_uint64)]


HELIX_TENSOR_NULL = HelixTensor(None, 0)


def desc_init(n_tok: int, n_seq: int, n_head: int, head_dim: int, d_state: int,
              n_group: int) -> HelixScanDesc:
    """Dense strides and defaults; reference src/runtime/desc.cpp:9-46."""
    d = HelixScanDesc()
    d.n_tok, d.n_seq, d.n_head = n_tok, n_seq, n_head
    d.head_dim, d.d_state, d.n_group = head_dim, d_state, n_group
    L, H, P, N, G = n_tok, n_head, head_dim, d_state, n_group
    d.s_x[0], d.s_x[1], d.s_x[2], d.seq_x = H * P, P, 1, L * H * P
    d.s_y[0], d.s_y[1], d.s_y[2], d.seq_y = H * P, P, 1, L * H * P
    d.s_b[0], d.s_b[1], d.s_b[2], d.seq_b = G * N, N, 1, L * G * N
    d.s_c[0], d.s_c[1], d.s_c[2], d.seq_c = G * N, N, 1, L * G * N
    d.s_dt[0], d.s_dt[1], d.seq_dt = H, 1, L * H
    d.s_s[0], d.s_s[1], d.s_s[2], d.seq_s = P * N, N, 1, H * P * N
    d.s_a = 1
    d.chunk = 0
    d.a_form = HELIX_A_SCALAR_PER_HEAD
    d.io_dtype = HELIX_F32
    d.compute_dtype = HELIX_F32
    d.backend = HELIX_BACKEND_AUTO
    d.multipass = False
    d.dt_min = 0.0
    d.dt_max = math.inf
    return d


def algorithmic_flops(n_tok: int, n_seq: int, n_head: int, head_dim: int, d_state: int,
                      chunk: int = 64) -> float:
    """The reference's FLOP count for one scan (bench/bench_scan.mm:205-209):
    2*S*H*n_chunks*(tri*N + tri*P + 2*CS*N*P), tri = CS*(CS+1)/2."""
    n_chunks = (n_tok + chunk - 1) // chunk
    tri = 0.5 * chunk * (chunk + 1)
    return 2.0 * n_seq * n_head * n_chunks * (tri * d_state + tri * head_dim
                                              + 2.0 * chunk * d_state * head_dim)


def algorithmic_bytes(n_tok: int, n_seq: int, n_head: int, head_dim: int, d_state: int,
                      n_group: int) -> float:
    """Every input read once and every output written once, fp32:
    4*(2*S*L*H*P + S*L*H + 2*S*L*G*N + 2*S*H*P*N + H)."""
    S, L, H, P, N, G = n_seq, n_tok, n_head, head_dim, d_state, n_group
    return 4.0 * (2 * S * L * H * P + S * L * H + 2 * S * L * G * N + 2 * S * H * P * N + H)
