"""ctypes bindings for the CPU oracle. TEST INFRASTRUCTURE.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg import
this module, and only as the checker. It binds two libraries built by
oracle/Makefile:

  liboracle.so              this repository's C restatement (helix_oracle.c)
  _ref/libhelix_refimpl.so  the reference's own oracle and harness generator,
                            present only where the reference tree was
                            available at build time (None otherwise)
"""
from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, c_double, c_float, c_int, c_int32, c_uint8, c_uint64, c_void_p
from dataclasses import dataclass, field

import numpy as np

from helix_amd.desc import HelixScanDesc, desc_init

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_REF_PATH = os.path.join(_HERE, "_ref", "libhelix_refimpl.so")

_fp = POINTER(c_float)
_ip = POINTER(c_int32)
_dp = POINTER(c_double)
_u8p = POINTER(c_uint8)
_descp = POINTER(HelixScanDesc)

_lib = None
_ref = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            raise RuntimeError(f"oracle library missing: {_LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(_LIB_PATH)
        scan_args = [_descp, _fp, _fp, _fp, _fp, _fp, _fp, _ip, _fp, _fp]
        L.oracle_scan.argtypes = scan_args + [_u8p]
        L.oracle_scan.restype = None
        L.oracle_scan_mt.argtypes = scan_args + [_u8p, c_int]
        L.oracle_scan_mt.restype = None
        L.oracle_scan_chunked.argtypes = scan_args
        L.oracle_scan_chunked.restype = None
        L.oracle_scan_snapshots.argtypes = scan_args + [c_int32, _dp]
        L.oracle_scan_snapshots.restype = None
        L.oracle_problem_harness.argtypes = [c_int32] * 6 + [c_uint64, c_int] + [_fp] * 6
        L.oracle_problem_harness.restype = None
        L.oracle_problem_gauss.argtypes = ([c_int32] * 6 + [c_uint64] + [c_double] * 5
                                           + [_fp] * 6)
        L.oracle_problem_gauss.restype = None
        _lib = L
    return _lib


def ref_lib():
    """The reference's own oracle, or None where oracle/_ref was not built."""
    global _ref
    if _ref is None and os.path.exists(_REF_PATH):
        R = ctypes.CDLL(_REF_PATH)
        R.ref_desc_size.restype = ctypes.c_size_t
        R.ref_desc_init.argtypes = [_descp] + [c_int32] * 6
        scan_args = [_descp, _fp, _fp, _fp, _fp, _fp, _fp, _ip, _fp, _fp]
        R.ref_scan.argtypes = scan_args
        R.ref_scan_chunked.argtypes = scan_args
        R.ref_scan_with_snapshots.argtypes = scan_args + [c_int32, _dp]
        R.ref_problem_make.argtypes = ([c_int32] * 7 + [c_uint64, c_int] + [_fp] * 6
                                       + [_descp])
        _ref = R
    return _ref


def _f(a):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_fp)


def _i(a):
    if a is None:
        return None
    assert a.dtype == np.int32 and a.flags.c_contiguous
    return a.ctypes.data_as(_ip)


@dataclass
class Problem:
    """One self-consistent problem instance in the dense helix.h layouts."""

    d: HelixScanDesc
    s0: np.ndarray
    x: np.ndarray
    dt: np.ndarray
    A: np.ndarray
    B: np.ndarray
    C: np.ndarray
    ids: np.ndarray | None = None
    label: str = ""
    meta: dict = field(default_factory=dict)

    @property
    def shape(self):
        d = self.d
        return d.n_tok, d.n_seq, d.n_head, d.head_dim, d.d_state, d.n_group

    def y_shape(self):
        d = self.d
        return (d.n_seq, d.n_tok, d.n_head, d.head_dim)

    def s_shape(self):
        d = self.d
        return (d.n_seq, d.n_head, d.head_dim, d.d_state)


def _alloc(L, S, H, P, N, G):
    return (np.zeros((S, H, P, N), np.float32), np.zeros((S, L, H, P), np.float32),
            np.zeros((S, L, H), np.float32), np.zeros((H,), np.float32),
            np.zeros((S, L, G, N), np.float32), np.zeros((S, L, G, N), np.float32))


def problem_harness(L, S, H, P, N, G, seed, memory="short", chunk=0) -> Problem:
    """The reference harness's Problem::make (tests/harness.hpp:151-186)."""
    s0, x, dt, A, B, C = _alloc(L, S, H, P, N, G)
    lib().oracle_problem_harness(L, S, H, P, N, G, seed, 1 if memory == "long" else 0,
                                 _f(s0), _f(x), _f(dt), _f(A), _f(B), _f(C))
    d = desc_init(L, S, H, P, N, G)
    d.chunk = chunk
    ids = np.arange(S, dtype=np.int32)
    return Problem(d, s0, x, dt, A, B, C, ids, label=f"harness seed={seed} {memory}")


def problem_diag(L, S, H, P, N, G, seed, memory="long") -> Problem:
    """A harness problem with a diagonal A (A[h][n], helix.h HELIX_A_DIAG_PER_CHANNEL,
    reference scan_ref.cpp:26-29): per-(head, state) decays drawn like the
    harness draws the scalar ones, A = -exp(U(-0.5, 1)) for LONG memory and
    A = -exp(U(0, ln 16)) for SHORT, from numpy's generator seeded with `seed`."""
    p = problem_harness(L, S, H, P, N, G, seed, memory)
    rng = np.random.default_rng(seed)
    lo, hi = (-0.5, 1.0) if memory == "long" else (0.0, float(np.log(16.0)))
    p.A = (-np.exp(rng.uniform(lo, hi, (H, N)))).astype(np.float32).ravel()
    p.d.a_form = 1          # HELIX_A_DIAG_PER_CHANNEL
    p.d.s_a = N
    p.label = f"diag-A harness seed={seed} {memory}"
    return p


def problem_gauss(L, S, H, P, N, G, seed, s0_sigma=0.0, dt_mu=-1.0, dt_sigma=0.5,
                  a_lo=1.0, a_hi=16.0) -> Problem:
    """The BASELINE.json generator (Gaussian; see helix_oracle.h)."""
    s0, x, dt, A, B, C = _alloc(L, S, H, P, N, G)
    lib().oracle_problem_gauss(L, S, H, P, N, G, seed, s0_sigma, dt_mu, dt_sigma, a_lo, a_hi,
                               _f(s0), _f(x), _f(dt), _f(A), _f(B), _f(C))
    d = desc_init(L, S, H, P, N, G)
    return Problem(d, s0, x, dt, A, B, C, None, label=f"gauss seed={seed}")


def _outs(p: Problem):
    return np.zeros(p.y_shape(), np.float32), np.zeros(p.s_shape(), np.float32)


def host_threads() -> int:
    """Threads for the parallel oracle: the cores this process may run on, at
    most 16 (the host-CPU share of one GPU on the GPU boxes)."""
    n = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return max(1, min(16, n))


def scan(p: Problem, head_mask=None, threads=1, use_ids=True):
    """fp64 sequential oracle; threads > 1 (or 0 = host_threads()) uses oracle_scan_mt."""
    if threads == 0:
        threads = host_threads()
    y, s1 = _outs(p)
    ids = p.ids if use_ids else None
    mask = None
    if head_mask is not None:
        mask = np.ascontiguousarray(np.asarray(head_mask, dtype=np.uint8))
    mptr = mask.ctypes.data_as(_u8p) if mask is not None else None
    if threads == 1:
        lib().oracle_scan(ctypes.byref(p.d), _f(p.s0), _f(p.x), _f(p.dt), _f(p.A), _f(p.B),
                          _f(p.C), _i(ids), _f(y), _f(s1), mptr)
    else:
        lib().oracle_scan_mt(ctypes.byref(p.d), _f(p.s0), _f(p.x), _f(p.dt), _f(p.A),
                             _f(p.B), _f(p.C), _i(ids), _f(y), _f(s1), mptr, threads)
    return y, s1


def scan_chunked(p: Problem, use_ids=True):
    y, s1 = _outs(p)
    ids = p.ids if use_ids else None
    lib().oracle_scan_chunked(ctypes.byref(p.d), _f(p.s0), _f(p.x), _f(p.dt), _f(p.A),
                              _f(p.B), _f(p.C), _i(ids), _f(y), _f(s1))
    return y, s1


def scan_snapshots(p: Problem, chunk=64, use_ids=True):
    y, s1 = _outs(p)
    ids = p.ids if use_ids else None
    d = p.d
    n_chunks = (d.n_tok + chunk - 1) // chunk
    snaps = np.zeros((n_chunks,) + p.s_shape(), np.float64)
    lib().oracle_scan_snapshots(ctypes.byref(d), _f(p.s0), _f(p.x), _f(p.dt), _f(p.A),
                                _f(p.B), _f(p.C), _i(ids), _f(y), _f(s1), chunk,
                                snaps.ctypes.data_as(_dp))
    return y, s1, snaps


# ---- the reference's own oracle (oracle/_ref) ------------------------------

def ref_problem(L, S, H, P, N, G, seed, memory="short", chunk=0) -> Problem:
    R = ref_lib()
    if R is None:
        raise RuntimeError("oracle/_ref not built (reference tree absent)")
    s0, x, dt, A, B, C = _alloc(L, S, H, P, N, G)
    d = HelixScanDesc()
    R.ref_problem_make(L, S, H, P, N, G, chunk, seed, 1 if memory == "long" else 0,
                       _f(s0), _f(x), _f(dt), _f(A), _f(B), _f(C), ctypes.byref(d))
    ids = np.arange(S, dtype=np.int32)
    return Problem(d, s0, x, dt, A, B, C, ids, label=f"ref harness seed={seed} {memory}")


def ref_scan(p: Problem, use_ids=True):
    y, s1 = _outs(p)
    ids = p.ids if use_ids else None
    ref_lib().ref_scan(ctypes.byref(p.d), _f(p.s0), _f(p.x), _f(p.dt), _f(p.A), _f(p.B),
                       _f(p.C), _i(ids), _f(y), _f(s1))
    return y, s1


def ref_scan_chunked(p: Problem, use_ids=True):
    y, s1 = _outs(p)
    ids = p.ids if use_ids else None
    ref_lib().ref_scan_chunked(ctypes.byref(p.d), _f(p.s0), _f(p.x), _f(p.dt), _f(p.A),
                               _f(p.B), _f(p.C), _i(ids), _f(y), _f(s1))
    return y, s1


def ref_scan_snapshots(p: Problem, chunk=64, use_ids=True):
    y, s1 = _outs(p)
    ids = p.ids if use_ids else None
    d = p.d
    n_chunks = (d.n_tok + chunk - 1) // chunk
    snaps = np.zeros((n_chunks,) + p.s_shape(), np.float64)
    ref_lib().ref_scan_with_snapshots(ctypes.byref(d), _f(p.s0), _f(p.x), _f(p.dt), _f(p.A),
                                      _f(p.B), _f(p.C), _i(ids), _f(y), _f(s1), chunk,
                                      snaps.ctypes.data_as(_dp))
    return y, s1, snaps


# ---- error metrics ---------------------------------------------------------

def allclose_ratio(got, ref, rel_tol, abs_tol):
    """max over elements of |a-b| / (abs_tol + rel_tol*|b|); the reference
    harness's per-element criterion (tests/harness.hpp:63-83). inf if any
    value is non-finite."""
    a = np.asarray(got, np.float64).ravel()
    b = np.asarray(ref, np.float64).ravel()
    if not (np.all(np.isfinite(a)) and np.all(np.isfinite(b))):
        return float("inf")
    if a.size == 0:
        return 0.0
    return float(np.max(np.abs(a - b) / (abs_tol + rel_tol * np.abs(b))))


def max_rel_err(got, ref):
    """max|got-ref| / max|ref|: the BASELINE.json parity gate."""
    a = np.asarray(got, np.float64)
    b = np.asarray(ref, np.float64)
    if not (np.all(np.isfinite(a)) and np.all(np.isfinite(b))):
        return float("inf")
    den = float(np.max(np.abs(b))) if b.size else 0.0
    num = float(np.max(np.abs(a - b))) if b.size else 0.0
    if den == 0.0:
        return num
    return num / den
