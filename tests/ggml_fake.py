"""ctypes mirror of the test-only ggml.h stand-in (tests/ggml_stub/ggml.h) and
helpers that lay a HELIX problem out as the GGML_OP_SSM_SCAN operands the
ggml HIP backend hands the bridge (reference integration/ggml/
ggml-helix.cpp:14-27): ne[] element counts and nb[] byte strides, fastest
dimension first; dst = [y | final state].
"""
from __future__ import annotations

import ctypes
import os

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BRIDGE_PATH = os.path.join(ROOT, "helix_amd", "integration", "ggml", "libggml_helix_stub.so")

GGML_TYPE_F32, GGML_TYPE_F16, GGML_TYPE_I32 = 0, 1, 26


class GgmlTensor(ctypes.Structure):
    pass


GgmlTensor._fields_ = [
    ("type", ctypes.c_int),
    ("ne", ctypes.c_int64 * 4),
    ("nb", ctypes.c_size_t * 4),
    ("op_params", ctypes.c_int32 * 16),
    ("src", ctypes.POINTER(GgmlTensor) * 10),
    ("data", ctypes.c_void_p),
]

_lib = None


def bridge():
    """The bridge compiled against the stand-in header (loads libhelix.so too)."""
    global _lib
    if _lib is None:
        from helix_amd import abi
        abi.lib()   # libhelix.so first, so the bridge binds to the same copy
        L = ctypes.CDLL(BRIDGE_PATH)
        from helix_amd.desc import HelixScanDesc
        L.helix_ggml_build_desc.argtypes = [ctypes.POINTER(GgmlTensor), ctypes.POINTER(HelixScanDesc)]
        L.helix_ggml_build_desc.restype = ctypes.c_bool
        L.ggml_hip_ssm_scan_helix_plan.argtypes = [ctypes.c_int, ctypes.POINTER(GgmlTensor),
                                                   ctypes.POINTER(ctypes.c_size_t)]
        L.ggml_hip_ssm_scan_helix_plan.restype = ctypes.c_bool
        L.ggml_hip_op_ssm_scan_helix.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.POINTER(GgmlTensor),
                                                 ctypes.c_void_p, ctypes.c_size_t]
        L.ggml_hip_op_ssm_scan_helix.restype = ctypes.c_bool
        _lib = L
    return _lib


def tensor(ne, nb, data=0, type_=GGML_TYPE_F32) -> GgmlTensor:
    t = GgmlTensor()
    t.type = type_
    ne = list(ne) + [1] * (4 - len(ne))
    nb = list(nb)
    while len(nb) < 4:
        nb.append(nb[-1] * ne[len(nb) - 1])
    for i in range(4):
        t.ne[i] = ne[i]
        t.nb[i] = nb[i]
    t.data = data
    return t


class SsmScanOp:
    """The SSM_SCAN node and its sources. Keeps every GgmlTensor alive."""

    def __init__(self, L, S, H, P, N, G, ptrs=None, a_diag=False, K=1, x_row_pad=0):
        p = ptrs or {}
        f = 4
        self.s = tensor((N, P, H, S), (f, f * N, f * N * P, f * N * P * H), p.get("s0", 0))
        xr = H * P + x_row_pad                   # token-row stride of x, elements
        self.x = tensor((P, H, L, S), (f, f * P, f * xr, f * xr * L), p.get("x", 0))
        self.dt = tensor((H, L, S), (f, f * H, f * H * L), p.get("dt", 0))
        an = N if a_diag else 1
        self.A = tensor((an, H), (f, f * an), p.get("A", 0))
        self.B = tensor((N, G, L, S), (f, f * N, f * N * G, f * N * G * L), p.get("B", 0))
        self.C = tensor((N, G, L, S), (f, f * N, f * N * G, f * N * G * L), p.get("C", 0))
        self.ids = tensor((S,), (4,), p.get("ids", 0), GGML_TYPE_I32) if p.get("ids") else None
        n_y = P * H * L * S
        n_s = N * P * H * S
        self.dst = tensor((n_y + n_s,), (f,), p.get("dst", 0))
        self.dst.op_params[0] = K
        for i, t in enumerate((self.s, self.x, self.dt, self.A, self.B, self.C, self.ids)):
            if t is not None:
                self.dst.src[i] = ctypes.pointer(t)
        self.n_y = n_y

    def ref(self):
        return ctypes.byref(self.dst)

    def relink(self):
        """Re-point dst.src after a source tensor was replaced."""
        for i, t in enumerate((self.s, self.x, self.dt, self.A, self.B, self.C, self.ids)):
            self.dst.src[i] = ctypes.pointer(t) if t is not None else ctypes.POINTER(GgmlTensor)()
