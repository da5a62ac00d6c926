"""ctypes bindings for libhelix.so (include/helix/helix.h, include/helix/helix_host.h).

The library is opened on first use. There is no fallback: if libhelix.so is
missing the call raises, so a GPU run can never silently compute on the CPU.
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_bool, c_char_p, c_int, c_int32, c_size_t, c_uint64, c_void_p

from .desc import (HELIX_OK, STATUS_NAMES, HelixScanDesc, HelixTensor)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "csrc", "libhelix.so")

# Every symbol include/helix/helix.h and helix_host.h declare.
ABI_SYMBOLS = (
    "helix_scan_desc_init",
    "helix_ctx_create",
    "helix_ctx_free",
    "helix_ctx_last_error",
    "helix_ctx_select_backend",
    "helix_ctx_backend_desc",
    "helix_scan_supported",
    "helix_scan_scratch_size",
    "helix_scan_encode",
    "helix_scan_encode_into",
)
HOST_SYMBOLS = ("helix_ctx_create_host", "helix_scan_plan_info", "helix_scan_encode_noalloc")
# include/helix/helix_host.h HELIX_PASS_B_*: where Pass B's segment scan runs
PASS_B_LAUNCHED, PASS_B_IN_C = 0, 1
# include/helix/helix_host.h HELIX_NOALLOC_SCRATCH_BYTES
NOALLOC_SCRATCH_BYTES = 128 << 20


class HelixPlanInfo(ctypes.Structure):
    _fields_ = [
        ("n_chunks", c_int32),
        ("chunks_per_group", c_int32),
        ("n_groups", c_int32),
        ("seg_len", c_int32),
        ("segs_per_group", c_int32),
        ("hblk", c_int32),
        ("n_hblk", c_int32),
        ("bf16_state", c_int32),
        ("total_bytes", c_uint64),
        ("s_local_bytes", c_uint64),
        ("s_seg_bytes", c_uint64),
        ("launches", c_int32),
        ("np", c_int32),
        ("kernel_a", ctypes.c_char_p),
        ("kernel_b", ctypes.c_char_p),
        ("kernel_c", ctypes.c_char_p),
        ("kernel_1pass", ctypes.c_char_p),
        ("bccopy_bytes", c_uint64),
        ("rec_bytes", c_uint64),
        ("walk_len", c_int32),
        ("walks_per_group", c_int32),
        ("pass_b", c_int32),
        ("state_in_y", c_int32),
        ("state_blocks", c_int32),
    ]


class HelixError(RuntimeError):
    def __init__(self, status: int, msg: str):
        super().__init__(f"{STATUS_NAMES.get(status, status)}: {msg}")
        self.status = status


_lib = None


def lib():
    """Open libhelix.so (once) and declare every prototype."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"libhelix.so not built at {LIB_PATH}; run __graft_entry__.build()")
    L = ctypes.CDLL(LIB_PATH)
    dp = POINTER(HelixScanDesc)
    T = HelixTensor
    L.helix_scan_desc_init.argtypes = [dp] + [c_int32] * 6
    L.helix_scan_desc_init.restype = None
    L.helix_ctx_create.argtypes = [POINTER(c_void_p), c_void_p, c_char_p]
    L.helix_ctx_create.restype = c_int
    L.helix_ctx_create_host.argtypes = [POINTER(c_void_p)]
    L.helix_ctx_create_host.restype = c_int
    L.helix_ctx_free.argtypes = [c_void_p]
    L.helix_ctx_free.restype = None
    L.helix_ctx_last_error.argtypes = [c_void_p]
    L.helix_ctx_last_error.restype = c_char_p
    L.helix_ctx_select_backend.argtypes = [c_void_p, dp]
    L.helix_ctx_select_backend.restype = c_int
    L.helix_ctx_backend_desc.argtypes = [c_void_p, dp]
    L.helix_ctx_backend_desc.restype = c_char_p
    L.helix_scan_supported.argtypes = [c_void_p, dp]
    L.helix_scan_supported.restype = c_bool
    L.helix_scan_scratch_size.argtypes = [c_void_p, dp]
    L.helix_scan_scratch_size.restype = c_size_t
    enc = [c_void_p, c_void_p, dp] + [T] * 10
    L.helix_scan_encode.argtypes = enc
    L.helix_scan_encode.restype = c_int
    L.helix_scan_encode_into.argtypes = enc
    L.helix_scan_encode_into.restype = c_int
    L.helix_scan_encode_noalloc.argtypes = [c_void_p, c_void_p, dp] + [T] * 9
    L.helix_scan_encode_noalloc.restype = c_int
    L.helix_scan_plan_info.argtypes = [c_void_p, dp, POINTER(HelixPlanInfo)]
    L.helix_scan_plan_info.restype = c_int
    _lib = L
    return L


def desc_init_c(n_tok, n_seq, n_head, head_dim, d_state, n_group) -> HelixScanDesc:
    d = HelixScanDesc()
    lib().helix_scan_desc_init(ctypes.byref(d), n_tok, n_seq, n_head, head_dim, d_state, n_group)
    return d


class Context:
    """Owns one helix_ctx. `device` is a HIP ordinal (None = current device);
    host_only=True makes a device-less planning context."""

    def __init__(self, device: int | None = None, code_object: str | None = None,
                 host_only: bool = False):
        L = lib()
        h = c_void_p()
        if host_only:
            st = L.helix_ctx_create_host(ctypes.byref(h))
        else:
            dev = c_int(device) if device is not None else None
            st = L.helix_ctx_create(ctypes.byref(h), ctypes.byref(dev) if dev is not None else None,
                                    code_object.encode() if code_object else None)
        if st != HELIX_OK:
            raise HelixError(st, L.helix_ctx_last_error(None).decode())
        self.handle = h
        self.host_only = host_only

    def close(self):
        if self.handle:
            lib().helix_ctx_free(self.handle)
            self.handle = c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def last_error(self) -> str:
        return lib().helix_ctx_last_error(self.handle).decode()

    def supported(self, d: HelixScanDesc) -> bool:
        return bool(lib().helix_scan_supported(self.handle, ctypes.byref(d)))

    def scratch_size(self, d: HelixScanDesc) -> int:
        return int(lib().helix_scan_scratch_size(self.handle, ctypes.byref(d)))

    def select_backend(self, d: HelixScanDesc) -> int:
        return int(lib().helix_ctx_select_backend(self.handle, ctypes.byref(d)))

    def backend_desc(self, d: HelixScanDesc) -> str:
        return lib().helix_ctx_backend_desc(self.handle, ctypes.byref(d)).decode()

    def plan_info(self, d: HelixScanDesc) -> HelixPlanInfo:
        info = HelixPlanInfo()
        st = lib().helix_scan_plan_info(self.handle, ctypes.byref(d), ctypes.byref(info))
        if st != HELIX_OK:
            raise HelixError(st, "descriptor declined")
        return info

    def encode_noalloc(self, stream: int, d: HelixScanDesc, s0, x, dt, A, B, C, ids, y, s1) -> int:
        """helix_scan_encode_noalloc: the scan on the library's fixed scratch."""
        return int(lib().helix_scan_encode_noalloc(self.handle, c_void_p(stream), ctypes.byref(d), s0, x, dt,
                                                   A, B, C, ids, y, s1))

    def encode(self, stream: int, d: HelixScanDesc, s0, x, dt, A, B, C, ids, y, s1, scratch,
               into: bool = False) -> int:
        """Enqueue the scan. Tensor arguments are HelixTensor; stream is a raw
        hipStream_t handle (0 = null stream). Returns the helix_status."""
        fn = lib().helix_scan_encode_into if into else lib().helix_scan_encode
        return int(fn(self.handle, c_void_p(stream), ctypes.byref(d), s0, x, dt, A, B, C, ids, y,
                      s1, scratch))
