"""Pins the CPU oracle before anything is checked against it.

Four independent anchors, chosen so that a plausible mistake in the C
restatement (a dropped term, a wrong sign or index, a transposed operand, the
softplus shortcut or the clamp mishandled, ids applied to the wrong tensor)
fails at least one of them:

1. bit-exactness against the reference's own fp64 oracle and harness
   generator, compiled from /root/reference into oracle/_ref
   (src/reference/scan_ref.cpp, scan_chunked_ref.cpp, tests/harness.hpp);
2. golden vectors written by that reference build (tests/golden/);
3. closed forms of the recurrence (reference.hpp:24-34): L=1, pure decay,
   zero input, the softplus > 20 shortcut, the dt clamp, and a brute-force
   pure-Python recurrence at tiny sizes;
4. invariants: linearity, superposition in s0, state splitting (which pins
   the carry), chunk-size invariance of the chunked form, ids permutation,
   head symmetry within a B/C group.
"""
from __future__ import annotations

import glob
import hashlib
import json
import math
import os

import numpy as np
import pytest

from oracle import pyoracle as po

HAVE_REF = po.ref_lib() is not None
needs_ref = pytest.mark.skipif(not HAVE_REF, reason="oracle/_ref not built (no reference tree)")

# The reference's test_algebra shapes (tests/test_algebra.cpp:28-44).
ALGEBRA_SHAPES = [
    (1, 1, 1, 64, 128, 1, 64), (7, 1, 2, 64, 128, 1, 64), (63, 1, 2, 64, 128, 1, 64),
    (64, 1, 2, 64, 128, 1, 64), (65, 1, 2, 64, 128, 1, 64), (127, 1, 2, 64, 128, 1, 64),
    (128, 1, 2, 64, 128, 1, 64), (129, 1, 2, 64, 128, 1, 64), (256, 1, 4, 64, 64, 1, 64),
    (256, 1, 4, 128, 128, 1, 64), (256, 1, 8, 128, 128, 8, 64), (256, 4, 4, 64, 128, 1, 64),
    (512, 1, 2, 64, 128, 1, 32), (512, 1, 2, 64, 128, 1, 128), (1024, 1, 2, 64, 128, 1, 64),
]


def bits(a):
    return np.ascontiguousarray(a).view(np.uint32 if a.dtype == np.float32 else np.uint64)


# ---------------------------------------------------------------------------
# 1. against the reference build
# ---------------------------------------------------------------------------

@needs_ref
@pytest.mark.parametrize("memory", ["short", "long"])
@pytest.mark.parametrize("shape", ALGEBRA_SHAPES[:12], ids=lambda s: "L%d_S%d_H%d_P%d_N%d_G%d" % s[:6])
def test_generator_matches_reference_harness(shape, memory):
    L, S, H, P, N, G, ck = shape
    mine = po.problem_harness(L, S, H, P, N, G, 12345, memory, chunk=ck)
    ref = po.ref_problem(L, S, H, P, N, G, 12345, memory, chunk=ck)
    for k in ("s0", "x", "dt", "A", "B", "C"):
        assert np.array_equal(bits(getattr(mine, k)), bits(getattr(ref, k))), k
    assert bytes(mine.d) == bytes(ref.d)


@needs_ref
@pytest.mark.parametrize("shape", [(70, 2, 2, 16, 264, 1), (130, 1, 2, 8, 512, 2)],
                         ids=lambda s: "L%d_S%d_H%d_P%d_N%d_G%d" % s)
def test_scan_bitexact_vs_reference_above_256(shape):
    # d_state above 256: the reference gate takes any multiple of 8
    # (caps.mm:129); its ref::scan is the same loop at every d_state.
    L, S, H, P, N, G = shape
    p = po.problem_harness(L, S, H, P, N, G, 778, "long")
    y, s1 = po.scan(p)
    yr, sr = po.ref_scan(p)
    assert np.array_equal(bits(y), bits(yr)) and np.array_equal(bits(s1), bits(sr))


def test_state_blocks_sum_to_the_scan():
    # What the encoder relies on above d_state 256: each state index evolves
    # on its own (h_n <- a h_n + B_n dt x) and y sums C_n h_n over n, so the
    # scans of blocks of state indices give s1 by concatenation and y by
    # summation. Checked on the oracle for the blocks the encoder would use
    # at d_state 264 (three of 88).
    L, S, H, P, N, G = 150, 2, 4, 16, 264, 2
    p = po.problem_harness(L, S, H, P, N, G, 779, "long")
    p.s0 = np.random.default_rng(7).standard_normal(p.s0.shape).astype(np.float32) * 0.3
    y, s1 = po.scan(p)
    y_sum = np.zeros(y.shape, np.float64)
    for n0 in (0, 88, 176):
        sl = slice(n0, n0 + 88)
        q = po.Problem(po.desc_init(L, S, H, P, 88, G), np.ascontiguousarray(p.s0[..., sl]), p.x, p.dt, p.A,
                       np.ascontiguousarray(p.B[..., sl]), np.ascontiguousarray(p.C[..., sl]), p.ids)
        yq, sq = po.scan(q)
        assert np.array_equal(bits(sq), bits(np.ascontiguousarray(s1[..., sl]))), n0
        y_sum += yq
    # y of each block is rounded to fp32 once; the full scan rounds the sum once.
    assert np.allclose(y_sum, y, rtol=1e-6, atol=1e-7)
    # A dropped block is not within that bound.
    assert not np.allclose(y_sum - yq, y, rtol=1e-6, atol=1e-7)


@needs_ref
@pytest.mark.parametrize("memory", ["short", "long"])
@pytest.mark.parametrize("shape", ALGEBRA_SHAPES, ids=lambda s: "L%d_S%d_H%d_P%d_N%d_G%d_c%d" % s)
def test_scan_bitexact_vs_reference(shape, memory):
    L, S, H, P, N, G, ck = shape
    p = po.problem_harness(L, S, H, P, N, G, 777, memory, chunk=ck)
    p.ids = np.arange(S, dtype=np.int32)[::-1].copy()   # exercise the ids gather
    y, s1 = po.scan(p)
    yr, sr = po.ref_scan(p)
    assert np.array_equal(bits(y), bits(yr)) and np.array_equal(bits(s1), bits(sr))
    yc, sc = po.scan_chunked(p)
    ycr, scr = po.ref_scan_chunked(p)
    assert np.array_equal(bits(yc), bits(ycr)) and np.array_equal(bits(sc), bits(scr))


@needs_ref
def test_snapshots_bitexact_vs_reference():
    p = po.problem_harness(300, 2, 3, 64, 64, 1, 20260905, "long")
    y, s1, snaps = po.scan_snapshots(p, 64)
    yr, sr, snr = po.ref_scan_snapshots(p, 64)
    assert np.array_equal(bits(y), bits(yr)) and np.array_equal(bits(s1), bits(sr))
    assert np.array_equal(bits(snaps), bits(snr))


def test_threaded_equals_sequential():
    p = po.problem_harness(200, 2, 6, 64, 64, 2, 5, "long")
    y, s1 = po.scan(p)
    ym, sm = po.scan(p, threads=4)
    assert np.array_equal(bits(y), bits(ym)) and np.array_equal(bits(s1), bits(sm))
    mask = np.array([1, 0, 0, 1, 0, 1], np.uint8)
    yh, sh = po.scan(p, head_mask=mask, threads=3)
    hs = [0, 3, 5]
    assert np.array_equal(bits(yh[:, :, hs]), bits(y[:, :, hs]))
    assert np.array_equal(bits(sh[:, hs]), bits(s1[:, hs]))


# ---------------------------------------------------------------------------
# 2. golden vectors written by the reference build (tests/golden/make_golden.py)
# ---------------------------------------------------------------------------

GOLDEN = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def _golden_problem(meta):
    if meta["gen"] == "harness":
        p = po.problem_harness(*meta["shape"], meta["seed"], meta["memory"])
    else:
        p = po.problem_gauss(*meta["shape"], meta["seed"], *meta["gauss"])
    p.ids = np.asarray(meta["ids"], np.int32) if meta["ids"] is not None else None
    p.d.dt_min, p.d.dt_max = meta["dt_min"], meta["dt_max"]
    return p


def _input_hash(p):
    h = hashlib.sha256()
    for k in ("s0", "x", "dt", "A", "B", "C"):
        h.update(np.ascontiguousarray(getattr(p, k)).tobytes())
    return h.hexdigest()


def test_golden_fixtures_present():
    assert len(GOLDEN) >= 6, "tests/golden/*.npz missing; run tests/golden/make_golden.py"


@pytest.mark.parametrize("path", GOLDEN, ids=[os.path.basename(g) for g in GOLDEN])
def test_oracle_matches_golden(path):
    z = np.load(path, allow_pickle=False)
    meta = json.loads(str(z["meta"]))
    p = _golden_problem(meta)
    assert _input_hash(p) == meta["input_sha256"], "generator drifted from the fixture"
    y, s1 = po.scan(p)
    assert np.array_equal(bits(y), bits(z["y"])), "y differs from the reference build"
    assert np.array_equal(bits(s1), bits(z["s1"])), "s1 differs from the reference build"
    if "snap" in z.files:
        _, _, snaps = po.scan_snapshots(p, 64)
        assert np.array_equal(bits(snaps), bits(z["snap"]))


# ---------------------------------------------------------------------------
# 3. closed forms
# ---------------------------------------------------------------------------

def softplus64(v):
    v = np.asarray(v, np.float64)
    return np.where(v > 20.0, v, np.log1p(np.exp(np.minimum(v, 20.0))))


def test_single_token_closed_form():
    # L=1: s1 = exp(A dt) s0 + dt x B ; y = C . s1  (reference.hpp:24-34)
    p = po.problem_harness(1, 2, 3, 8, 16, 1, 99, "short")
    y, s1 = po.scan(p)
    dt = softplus64(p.dt[:, 0, :])                            # [S, H]
    dA = np.exp(p.A.astype(np.float64)[None, :] * dt)         # [S, H]
    x = p.x[:, 0].astype(np.float64)                          # [S, H, P]
    B = p.B[:, 0, 0].astype(np.float64)                       # [S, N]
    C = p.C[:, 0, 0].astype(np.float64)
    s = dA[:, :, None, None] * p.s0 + (dt[:, :, None] * x)[..., None] * B[:, None, None, :]
    np.testing.assert_allclose(s1, s, rtol=1e-6, atol=1e-9)
    np.testing.assert_allclose(y[:, 0], np.einsum("shpn,sn->shp", s, C), rtol=1e-6, atol=1e-9)


def test_pure_decay_closed_form():
    # B = 0: s1 = exp(A sum dt) s0, y_t = exp(A sum_{j<=t} dt) C_t . s0
    p = po.problem_harness(50, 1, 2, 4, 8, 1, 3, "long")
    p.B[:] = 0.0
    y, s1 = po.scan(p)
    dt = softplus64(p.dt[0])                                  # [L, H]
    cum = np.cumsum(p.A.astype(np.float64)[None, :] * dt, axis=0)
    np.testing.assert_allclose(s1[0], np.exp(cum[-1])[:, None, None] * p.s0[0], rtol=1e-6, atol=1e-12)
    cs0 = np.einsum("ln,hpn->lhp", p.C[0, :, 0].astype(np.float64), p.s0[0].astype(np.float64))
    np.testing.assert_allclose(y[0], np.exp(cum)[:, :, None] * cs0, rtol=1e-6, atol=1e-9)


def test_zero_input_zero_state_gives_zero():
    p = po.problem_harness(70, 2, 2, 8, 8, 1, 4, "short")
    p.x[:] = 0.0
    p.s0[:] = 0.0
    y, s1 = po.scan(p)
    assert not np.any(y) and not np.any(s1)


def test_softplus_shortcut_and_clamp():
    # dt_raw > 20 is used as-is; dt_min/dt_max clamp softplus(dt) (scan_ref.cpp:13-24).
    p = po.problem_harness(1, 1, 1, 1, 1, 1, 8, "short")
    p.s0[:] = 0.0
    p.x[:] = 1.0
    p.B[:] = 1.0
    p.C[:] = 1.0
    p.dt[:] = 25.0
    y, s1 = po.scan(p)
    assert s1.ravel()[0] == np.float32(25.0) and y.ravel()[0] == np.float32(25.0)
    p.dt[:] = 0.5
    p.d.dt_min, p.d.dt_max = 0.0, 0.25
    y, s1 = po.scan(p)
    assert s1.ravel()[0] == np.float32(0.25)
    p.d.dt_min, p.d.dt_max = 3.0, math.inf
    y, s1 = po.scan(p)
    assert s1.ravel()[0] == np.float32(3.0)


def _brute(p):
    """Pure-Python recurrence, one multiply and add at a time."""
    S, L, H, P = p.x.shape
    G, N = p.B.shape[2], p.B.shape[3]
    y = np.zeros((S, L, H, P))
    s1 = np.zeros((S, H, P, N))
    for s in range(S):
        for h in range(H):
            g = h // (H // G)
            for q in range(P):
                st = [float(p.s0[s, h, q, n]) for n in range(N)]
                for t in range(L):
                    v = float(p.dt[s, t, h])
                    dt = v if v > 20 else math.log1p(math.exp(v))
                    acc = 0.0
                    for n in range(N):
                        a_hn = p.A[h * p.d.s_a + (n if p.d.a_form == 1 else 0)]
                        a = math.exp(float(a_hn) * dt)
                        st[n] = a * st[n] + dt * float(p.B[s, t, g, n]) * float(p.x[s, t, h, q])
                        acc += float(p.C[s, t, g, n]) * st[n]
                    y[s, t, h, q] = acc
                s1[s, h, q] = st
    return y, s1


@pytest.mark.parametrize("shape", [(9, 1, 1, 1, 1, 1), (12, 2, 4, 3, 2, 2), (5, 1, 2, 2, 4, 1)])
def test_brute_force_small(shape):
    p = po.problem_harness(*shape, 31, "long")
    y, s1 = po.scan(p)
    yb, sb = _brute(p)
    np.testing.assert_allclose(y, yb, rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(s1, sb, rtol=1e-6, atol=1e-12)


def test_tiny_decay_is_a_prefix_sum():
    # A -> 0: s_t = s0 + sum_{j<=t} dt_j x_j B_j exactly up to exp(~0) = 1.
    p = po.problem_harness(40, 1, 1, 2, 3, 1, 6, "long")
    p.A[:] = -1e-12
    y, s1 = po.scan(p)
    dt = softplus64(p.dt[0, :, 0])
    inc = dt[:, None, None] * p.x[0, :, 0, :, None].astype(np.float64) * p.B[0, :, 0, None, :]
    s = p.s0[0, 0].astype(np.float64) + np.cumsum(inc, axis=0)
    np.testing.assert_allclose(s1[0, 0], s[-1], rtol=1e-6, atol=1e-10)
    np.testing.assert_allclose(y[0, :, 0], np.einsum("lpn,ln->lp", s, p.C[0, :, 0]), rtol=1e-6, atol=1e-10)


# ---------------------------------------------------------------------------
# 4. invariants
# ---------------------------------------------------------------------------

def test_linearity_in_x_and_superposition_in_s0():
    p = po.problem_harness(130, 1, 2, 8, 16, 1, 11, "long")
    q = po.problem_harness(130, 1, 2, 8, 16, 1, 12, "long")
    q.dt[:], q.A[:], q.B[:], q.C[:] = p.dt, p.A, p.B, p.C
    y1, s1a = po.scan(p)
    y2, s2a = po.scan(q)
    r = po.problem_harness(130, 1, 2, 8, 16, 1, 11, "long")
    r.x[:] = 2.0 * p.x - 0.5 * q.x
    r.s0[:] = 2.0 * p.s0 - 0.5 * q.s0
    y3, s3 = po.scan(r)
    np.testing.assert_allclose(y3, 2.0 * y1.astype(np.float64) - 0.5 * y2, rtol=1e-5, atol=1e-6)
    np.testing.assert_allclose(s3, 2.0 * s1a.astype(np.float64) - 0.5 * s2a, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("split", [1, 63, 64, 100])
def test_state_splitting(split):
    # scan(L1 + L2) == scan(L2, s0 = scan(L1).s1): pins the carry.
    L = 200
    p = po.problem_harness(L, 2, 2, 16, 32, 1, 21, "long")
    y, s1 = po.scan(p)
    a = po.problem_harness(split, 2, 2, 16, 32, 1, 21, "long")
    b = po.problem_harness(L - split, 2, 2, 16, 32, 1, 21, "long")
    for k in ("x", "dt", "B", "C"):
        getattr(a, k)[:] = getattr(p, k)[:, :split]
        getattr(b, k)[:] = getattr(p, k)[:, split:]
    a.s0[:], a.A[:], b.A[:] = p.s0, p.A, p.A
    ya, sa = po.scan(a)
    b.s0[:] = sa
    yb, sb = po.scan(b)
    np.testing.assert_allclose(np.concatenate([ya, yb], axis=1), y, rtol=1e-5, atol=1e-7)
    np.testing.assert_allclose(sb, s1, rtol=1e-5, atol=1e-7)


def test_chunk_invariance():
    # tests/test_algebra.cpp:77-93: the chunked form must not depend on chunk.
    base = None
    for ck in (16, 32, 64, 128, 256):
        p = po.problem_harness(509, 1, 4, 64, 128, 1, 777, "short", chunk=ck)
        y, s1 = po.scan_chunked(p)
        if base is None:
            base = (y, s1)
            continue
        assert po.allclose_ratio(y, base[0], 1e-6, 1e-9) <= 1.0
        assert po.allclose_ratio(s1, base[1], 1e-6, 1e-9) <= 1.0


@pytest.mark.parametrize("shape", ALGEBRA_SHAPES, ids=lambda s: "L%d_S%d_H%d_P%d_N%d_G%d_c%d" % s)
def test_chunked_equals_sequential(shape):
    # tests/test_algebra.cpp:57-75 at its tolerances (rel 1e-6, abs 1e-9).
    L, S, H, P, N, G, ck = shape
    p = po.problem_harness(L, S, H, P, N, G, 12345, "short", chunk=ck)
    y, s1 = po.scan(p)
    yc, sc = po.scan_chunked(p)
    assert po.allclose_ratio(yc, y, 1e-6, 1e-9) <= 1.0
    assert po.allclose_ratio(sc, s1, 1e-6, 1e-9) <= 1.0


def test_ids_permutes_source_states():
    p = po.problem_harness(40, 3, 2, 8, 8, 1, 5, "long")
    p.ids = np.array([2, 0, 1], np.int32)
    y, s1 = po.scan(p)
    q = po.problem_harness(40, 3, 2, 8, 8, 1, 5, "long")
    q.s0[:] = p.s0[[2, 0, 1]]
    q.ids = None
    yq, sq = po.scan(q, use_ids=False)
    assert np.array_equal(y, yq) and np.array_equal(s1, sq)


def test_heads_in_a_group_share_b_and_c():
    # Two heads of one group with identical A, dt, x and s0 give identical output.
    p = po.problem_harness(70, 1, 4, 8, 16, 2, 13, "long")
    p.A[1], p.dt[..., 1], p.x[:, :, 1], p.s0[:, 1] = p.A[0], p.dt[..., 0], p.x[:, :, 0], p.s0[:, 0]
    y, s1 = po.scan(p)
    assert np.array_equal(y[:, :, 0], y[:, :, 1]) and np.array_equal(s1[:, 0], s1[:, 1])
    # ...and a head of the other group (same per-head inputs) differs.
    p.A[2], p.dt[..., 2], p.x[:, :, 2], p.s0[:, 2] = p.A[0], p.dt[..., 0], p.x[:, :, 0], p.s0[:, 0]
    y, s1 = po.scan(p)
    assert not np.array_equal(y[:, :, 0], y[:, :, 2])


def test_gauss_generator_moments():
    p = po.problem_gauss(2048, 1, 16, 64, 128, 2, 1234, s0_sigma=0.1, dt_mu=-1.0, dt_sigma=0.5)
    assert abs(p.x.mean()) < 0.01 and abs(p.x.std() - 1.0) < 0.01
    assert abs(p.dt.mean() + 1.0) < 0.02 and abs(p.dt.std() - 0.5) < 0.02
    assert abs(p.B.std() * math.sqrt(128) - 1.0) < 0.02
    assert abs(p.s0.std() - 0.1) < 0.005
    assert np.all(p.A <= -1.0) and np.all(p.A >= -16.0)
    z = po.problem_gauss(16, 1, 2, 8, 8, 1, 1, s0_sigma=0.0)
    assert not np.any(z.s0)


# ---------------------------------------------------------------------------
# Diagonal A (A[h][n]; reference scan_ref.cpp:26-29, helix.h HELIX_A_DIAG_PER_CHANNEL)
# ---------------------------------------------------------------------------

@needs_ref
@pytest.mark.parametrize("memory", ["short", "long"])
@pytest.mark.parametrize("shape", [(1, 1, 1, 8, 8, 1), (130, 2, 4, 64, 64, 2), (300, 1, 2, 64, 128, 1)])
def test_diag_bitexact_vs_reference(shape, memory):
    p = po.problem_diag(*shape, 404, memory)
    p.ids = np.arange(p.d.n_seq, dtype=np.int32)[::-1].copy()
    y, s1 = po.scan(p)
    yr, sr = po.ref_scan(p)
    assert np.array_equal(bits(y), bits(yr)) and np.array_equal(bits(s1), bits(sr))


def test_diag_with_equal_rows_is_the_scalar_form():
    # Every state row of a head decaying at A_h is exactly the scalar-A scan.
    p = po.problem_diag(200, 2, 4, 16, 24, 2, 8, "long")
    q = po.problem_harness(200, 2, 4, 16, 24, 2, 8, "long")
    A = np.repeat(q.A[:, None], 24, axis=1).astype(np.float32)
    p.A = A.ravel()
    y, s1 = po.scan(p)
    yq, sq = po.scan(q)
    assert np.array_equal(bits(y), bits(yq)) and np.array_equal(bits(s1), bits(sq))


@pytest.mark.parametrize("shape", [(9, 1, 1, 1, 3, 1), (12, 2, 4, 3, 2, 2)])
def test_diag_brute_force_small(shape):
    p = po.problem_diag(*shape, 33, "long")
    assert len(set(p.A.tolist())) == p.A.size        # the rows really differ
    y, s1 = po.scan(p)
    yb, sb = _brute(p)
    np.testing.assert_allclose(y, yb, rtol=1e-6, atol=1e-12)
    np.testing.assert_allclose(s1, sb, rtol=1e-6, atol=1e-12)
