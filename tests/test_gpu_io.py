"""16-bit storage of x, B, C and y (io_dtype BF16 / F16) on the GPU.

helix.h:122 defines io_dtype as the storage of x/B/C/y; dt, A and the states
stay fp32 (the reference declines anything but F32, caps.mm:126). The fp64
oracle has no storage type, so it is fed the same inputs rounded to the
storage type (round to nearest even), and the device's y is widened back:
- on the bf16 path (walking Pass C, bf16 operands) y meets the bf16 gates;
- on the single pass (fp32 compute) the only extra error is y's own rounding
  to the storage type, at most the unit roundoff u (2^-8 for bf16, 2^-11 for
  f16) relative, so the per-element bound is the fp32 one plus u:
  |dy| <= F32_ABS + (F32_REL + u)|y|, and max|dy|/max|y| <= F32_GATE + u;
- s1 is fp32 and held to the fp32 bound everywhere, since the state is
  computed from the very values the oracle sees.
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import pyoracle as po
from helix_amd.desc import (HELIX_BACKEND_AUTO, HELIX_BACKEND_SGMMA, HELIX_BF16, HELIX_F16,
                            HELIX_OK, HELIX_TENSOR_NULL)
from baseline_configs import CONFIGS
from gpu_harness import BF16_ABS, BF16_GATE, BF16_REL, F32_ABS, F32_GATE, F32_REL, X3_ABS, X3_REL, T, ctx_for

pytestmark = pytest.mark.gpu

TORCH = {HELIX_BF16: torch.bfloat16, HELIX_F16: torch.float16}
NAME = {HELIX_BF16: "bf16", HELIX_F16: "f16"}
# Unit roundoff of the storage type: y is rounded once to it (single pass).
U = {HELIX_BF16: 2.0 ** -8, HELIX_F16: 2.0 ** -11}


def round_to(a: np.ndarray, io: int) -> np.ndarray:
    """fp32 values rounded to the storage type (RNE), as fp32."""
    a = np.ascontiguousarray(a, dtype=np.float32)
    if io == HELIX_F16:
        return a.astype(np.float16).astype(np.float32)
    u = a.view(np.uint32)
    r = ((u >> 16) & 1) + np.uint32(0x7FFF)
    return ((u + r) & np.uint32(0xFFFF0000)).view(np.float32)


def rounded(p: po.Problem, io: int) -> po.Problem:
    q = po.Problem(p.d.copy(), p.s0, round_to(p.x, io), p.dt, p.A, round_to(p.B, io), round_to(p.C, io),
                   p.ids, label=p.label)
    return q


def run_io(gpu, p: po.Problem, io: int, backend: int, multipass: bool, use_ids=False):
    d = p.d.copy()
    d.io_dtype = io
    d.backend = backend
    d.multipass = multipass
    assert gpu.supported(d), gpu.backend_desc(d)
    dt = TORCH[io]
    dev = {k: torch.from_numpy(np.ascontiguousarray(getattr(p, k))).cuda() for k in ("s0", "dt", "A")}
    for k in ("x", "B", "C"):
        dev[k] = torch.from_numpy(np.ascontiguousarray(getattr(p, k))).cuda().to(dt)
    ids = torch.from_numpy(p.ids).cuda() if (use_ids and p.ids is not None) else None
    y = torch.full(p.y_shape(), float("nan"), device="cuda", dtype=dt)
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    need = gpu.scratch_size(d)
    scratch = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    rc = gpu.encode(torch.cuda.current_stream().cuda_stream, d, T(dev["s0"]), T(dev["x"]), T(dev["dt"]),
                    T(dev["A"]), T(dev["B"]), T(dev["C"]), T(ids) if ids is not None else HELIX_TENSOR_NULL,
                    T(y), T(s1), T(scratch))
    assert rc == HELIX_OK, gpu.last_error()
    torch.cuda.synchronize()
    return gpu.backend_desc(d), y.float().cpu().numpy(), s1.cpu().numpy()


def check(io, desc, y, s1, y_ref, s_ref):
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    ey, es = po.max_rel_err(y, y_ref), po.max_rel_err(s1, s_ref)
    if "bf16 pass C" in desc:
        assert ey <= BF16_GATE and po.allclose_ratio(y, y_ref, BF16_REL, BF16_ABS) <= 1.0, ey
    else:
        assert ey <= F32_GATE + U[io], ey
        assert po.allclose_ratio(y, y_ref, F32_REL + U[io], F32_ABS) <= 1.0
    # s1 at the fp32 bound (the wider bound only for the opt-in three-product
    # Pass A, which no test here selects).
    s_rel, s_abs = (X3_REL, X3_ABS) if "pass A bf16x3" in desc else (F32_REL, F32_ABS)
    assert es <= F32_GATE and po.allclose_ratio(s1, s_ref, s_rel, s_abs) <= 1.0, es
    return ey, es


SHAPES = [
    (300, 2, 8, 64, 128, 2, "L=300 grouped ragged"),
    (64, 1, 2, 64, 128, 1, "L=64 one chunk"),
    (256, 1, 4, 64, 64, 1, "d_state=64"),
    (256, 1, 4, 128, 256, 1, "d_state=256"),
    (256, 1, 4, 192, 128, 1, "head_dim=192 three slabs"),
    (1100, 1, 4, 64, 128, 2, "L=1100 two segments"),
]
PATHS = [("walk", HELIX_BACKEND_AUTO, True), ("1pass", HELIX_BACKEND_AUTO, False),
         ("fp32", HELIX_BACKEND_SGMMA, True), ("walk/x6", HELIX_BACKEND_AUTO, True)]
IOS = [HELIX_BF16, HELIX_F16]


@pytest.mark.parametrize("io", IOS, ids=["bf16", "f16"])
@pytest.mark.parametrize("path", PATHS, ids=[p[0] for p in PATHS])
@pytest.mark.parametrize("shape", SHAPES, ids=[s[-1] for s in SHAPES])
def test_storage_matrix(gpu, shape, path, io):
    label, backend, multipass = path
    p = rounded(po.problem_harness(*shape[:6], 4242, "long"), io)
    p.s0 = np.random.default_rng(3).standard_normal(p.s0.shape).astype(np.float32) * 0.2
    y_ref, s_ref = po.scan(p, use_ids=False)
    # walk/x6: Pass A on six bf16 split products instead of two fp16 planes.
    ctx = ctx_for(gpu, HELIX_PASSA_F16="0") if label == "walk/x6" else gpu
    desc, y, s1 = run_io(ctx, p, io, backend, multipass)
    assert f"{NAME[io]} storage" in desc
    assert ("chunk walk" in desc) == label.startswith("walk")
    ey, es = check(io, desc, y, s1, y_ref, s_ref)
    print(f"{NAME[io]} {label} {shape[-1]}: y {ey:.2e} s1 {es:.2e}  [{desc}]", flush=True)


@pytest.mark.parametrize("io", IOS, ids=["bf16", "f16"])
@pytest.mark.parametrize("path", PATHS[:2], ids=[p[0] for p in PATHS[:2]])
def test_storage_ids(gpu, path, io):
    label, backend, multipass = path
    p = rounded(po.problem_harness(300, 4, 4, 64, 128, 2, 77, "long"), io)
    p.s0 = np.random.default_rng(4).standard_normal(p.s0.shape).astype(np.float32) * 0.3
    p.ids = np.array([3, 1, 0, 2], np.int32)
    y_ref, s_ref = po.scan(p, use_ids=True)
    desc, y, s1 = run_io(gpu, p, io, backend, multipass, use_ids=True)
    check(io, desc, y, s1, y_ref, s_ref)


RANGES = ["rows spread", "channels spread", "spikes"]


@pytest.mark.parametrize("kind", RANGES)
@pytest.mark.parametrize("io", IOS, ids=["bf16", "f16"])
def test_storage_ranges(gpu, io, kind):
    """16-bit storage on the bf16 path, where Pass A keeps one fp16 plane of B
    (the scaled bf16 or f16 value is exact in it): B's state indices spread
    over eight decades, x's channels over six, or single-token spikes late in
    a segment, within the storage type's range; s1 at the fp32 bound (its
    absolute term scaled with the largest reference value)."""
    p = po.problem_harness(1100, 2, 8, 64, 128, 2, 91, "long")
    rng = np.random.default_rng(91)
    if kind == "rows spread":
        p.B *= (10.0 ** rng.uniform(-4, 4, p.B.shape[-1])).astype(np.float32)
    elif kind == "channels spread":
        p.x *= (10.0 ** rng.uniform(-3, 3, p.x.shape[-1])).astype(np.float32)
    else:
        p.x[:, 300, :, 5] *= np.float32(2e3)
        p.B[:, 200, :, 11] *= np.float32(2e3)
    p = rounded(p, io)
    p.s0 = (rng.standard_normal(p.s0.shape) * 0.3).astype(np.float32)
    y_ref, s_ref = po.scan(p, use_ids=False)
    desc, y, s1 = run_io(gpu, p, io, HELIX_BACKEND_AUTO, True)
    assert "fp16x3" in desc
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    ry = po.allclose_ratio(y, y_ref, BF16_REL, BF16_ABS * max(1.0, float(np.max(np.abs(y_ref)))))
    rs = po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS * max(1.0, float(np.max(np.abs(s_ref)))))
    print(f"{NAME[io]} {kind}: y ratio {ry:.3f} s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)


@pytest.mark.parametrize("io", IOS, ids=["bf16", "f16"])
@pytest.mark.parametrize("name", ["cfg2", "cfg4a"])
def test_storage_baseline_config(gpu, name, io):
    """The BASELINE bf16-path configurations at full size with 16-bit storage,
    checked on the oracle's head subset (heads are independent)."""
    c = CONFIGS[name]
    p = rounded(po.problem_gauss(*c.shape, c.seed, c.s0_sigma, c.dt_mu, c.dt_sigma), io)
    mask = np.zeros(c.H, np.uint8)
    mask[list(c.check_heads)] = 1
    y_ref, s_ref = po.scan(p, head_mask=mask, threads=0)
    desc, y, s1 = run_io(gpu, p, io, HELIX_BACKEND_AUTO, True)
    hs = list(c.check_heads)
    ey, es = check(io, desc, y[:, :, hs], s1[:, hs], y_ref[:, :, hs], s_ref[:, hs])
    print(f"[{name} {NAME[io]} storage] {desc}: y {ey:.2e} s1 {es:.2e}", flush=True)


@pytest.mark.parametrize("pad", [8, 2])
@pytest.mark.parametrize("backend", ["bf16", "fp32"])
def test_ssd_scan_padded_rows(gpu, backend, pad):
    """The torch operator with bf16 tensors: io_dtype comes from x.dtype, and B/C
    are views into rows padded by `pad` elements (an even stride; with pad 2
    the rows are only 4-byte aligned)."""
    from helix_amd.scan import ssd_scan
    io = HELIX_BF16
    p = rounded(po.problem_harness(200, 2, 4, 64, 64, 2, 5, "long"), io)
    p.s0 = np.random.default_rng(6).standard_normal(p.s0.shape).astype(np.float32) * 0.2
    y_ref, s_ref = po.scan(p, use_ids=False)
    S, L, G, N = p.B.shape

    def padded(a):
        t = torch.zeros((S, L, G, N + pad), dtype=torch.bfloat16, device="cuda")
        t[..., :N] = torch.from_numpy(a).cuda().to(torch.bfloat16)
        return t[..., :N]

    up = lambda a: torch.from_numpy(np.ascontiguousarray(a)).cuda()
    B, C = padded(p.B), padded(p.C)
    assert B.stride(2) == N + pad
    y, s1 = ssd_scan(up(p.x).to(torch.bfloat16), up(p.dt), up(p.A), B, C, up(p.s0), backend=backend)
    torch.cuda.synchronize()
    assert y.dtype == torch.bfloat16 and s1.dtype == torch.float32
    desc = "mfma bf16 pass C" if backend == "bf16" else "single pass"
    check(io, desc, y.float().cpu().numpy(), s1.cpu().numpy(), y_ref, s_ref)


def test_misaligned_rows_rejected(gpu):
    """16-bit B or C rows are loaded as 32-bit words: a base that is only 2-byte
    aligned is an INVALID_ARG from the host, with nothing enqueued."""
    from helix_amd.desc import HELIX_ERR_INVALID_ARG, HelixTensor
    p = rounded(po.problem_harness(128, 1, 2, 64, 64, 1, 8), HELIX_BF16)
    d = p.d.copy()
    d.io_dtype = HELIX_BF16
    d.backend = HELIX_BACKEND_AUTO
    assert gpu.supported(d)
    up = lambda a, t=torch.float32: torch.from_numpy(np.ascontiguousarray(a)).cuda().to(t)
    x, B, C = (up(a, torch.bfloat16) for a in (p.x, p.B, p.C))
    s0, dt, A = up(p.s0), up(p.dt), up(p.A)
    Bbig = torch.zeros(B.numel() + 1, dtype=torch.bfloat16, device="cuda")
    y = torch.full(p.y_shape(), float("nan"), device="cuda", dtype=torch.bfloat16)
    s1 = torch.full(p.s_shape(), float("nan"), device="cuda")
    scratch = torch.empty(max(gpu.scratch_size(d), 1), dtype=torch.uint8, device="cuda")
    for which in ("B", "C"):
        args = {"B": T(B), "C": T(C)}
        args[which] = HelixTensor(Bbig.data_ptr(), 2)       # 2-byte offset
        rc = gpu.encode(torch.cuda.current_stream().cuda_stream, d, T(s0), T(x), T(dt), T(A),
                        args["B"], args["C"], HELIX_TENSOR_NULL, T(y), T(s1), T(scratch))
        assert rc == HELIX_ERR_INVALID_ARG, (which, rc)
        assert "align" in gpu.last_error(), gpu.last_error()
    torch.cuda.synchronize()
    assert torch.isnan(y.float()).all() and torch.isnan(s1).all()
