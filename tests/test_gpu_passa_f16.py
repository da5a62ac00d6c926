"""Pass A on two scaled fp16 planes (HELIX_PASSA_F16=1, helix_chunk_state_hb_h3agg_*).

The operands are scaled by powers of two into fp16's range: per state index
for B, per channel for the weighted x, set by the first chunk with a nonzero
value and replaced (with the accumulated row or column rescaled) when a later
chunk's values would leave fp16's range. These cases drive the scales where the
BASELINE distributions do not: inputs far above and below fp16's range, state
indices whose magnitudes spread over twelve decades, single-token spikes that
force a mid-segment rescale, rows that stay zero for many chunks, and strong
decay. s1 is held to the reference's fp32 per-element bound and y to the bf16
path's, against the fp64 oracle, on the walk's plan with and without the bf16
copies of B and C; the absolute terms of both bounds scale with the largest
reference value (the reference's bounds are for values of order one). The
six-product bf16 Pass A runs the same cases to the same bounds.
"""
from __future__ import annotations

import numpy as np
import pytest

from oracle import pyoracle as po
from helix_amd.desc import HELIX_BACKEND_MPP
from gpu_harness import BF16_ABS, BF16_REL, F32_ABS, F32_REL, ctx_for, run

pytestmark = pytest.mark.gpu

L, S, H, P, N, G = 1100, 2, 8, 64, 128, 2


def _scaled(kind: str, seed: int) -> po.Problem:
    p = po.problem_harness(L, S, H, P, N, G, seed, "long")
    rng = np.random.default_rng(seed)
    if kind == "x 1e6":
        p.x *= np.float32(1e6)
    elif kind == "x 1e-8":
        p.x *= np.float32(1e-8)
    elif kind == "B 1e5":
        p.B *= np.float32(1e5)
    elif kind == "B 1e-9":
        p.B *= np.float32(1e-9)
    elif kind == "rows spread":
        p.B *= (10.0 ** rng.uniform(-6, 6, N)).astype(np.float32)[None, None, None, :]
    elif kind == "spikes":
        # Late tokens of a segment come first in Pass A's backward walk: the
        # spikes arrive after the scales are set.
        p.x[:, 300, :, 5] *= np.float32(3e4)
        p.B[:, 200, :, 11] *= np.float32(3e4)
        p.x[:, 1000, 3, :] *= np.float32(1e-20)
    elif kind == "zero rows":
        p.B[:, 512:, :, :16] = 0.0      # zero in the chunks Pass A visits first
        p.B[:, :512, :, 16:32] = 0.0
        p.x[:, 600:700, :, :8] = 0.0
    elif kind == "strong decay":
        p.dt[:] = np.float32(3.0)
    else:
        raise ValueError(kind)
    p.s0 = (rng.standard_normal(p.s0.shape) * 0.3).astype(np.float32)
    return p


KINDS = ["x 1e6", "x 1e-8", "B 1e5", "B 1e-9", "rows spread", "spikes", "zero rows", "strong decay"]


@pytest.mark.parametrize("passa", ["h3", "x6"])
@pytest.mark.parametrize("copies", ["0", "1"], ids=["caller rows", "copies"])
@pytest.mark.parametrize("kind", KINDS)
def test_f16_planes_ranges(gpu, kind, copies, passa):
    p = _scaled(kind, 6161)
    d = p.d.copy()
    d.multipass = True
    d.backend = HELIX_BACKEND_MPP
    ctx = ctx_for(gpu, HELIX_PASSA_F16="1" if passa == "h3" else "0", HELIX_WALK_BCCOPY=copies)
    assert (b"_h3agg" in ctx.plan_info(d).kernel_a) == (passa == "h3")
    y_ref, s_ref = po.scan(p, threads=0)
    _, y, s1 = run(ctx, p, desc=d)
    assert np.all(np.isfinite(y)) and np.all(np.isfinite(s1))
    ry = po.allclose_ratio(y, y_ref, BF16_REL, BF16_ABS * max(1.0, float(np.max(np.abs(y_ref)))))
    rs = po.allclose_ratio(s1, s_ref, F32_REL, F32_ABS * max(1.0, float(np.max(np.abs(s_ref)))))
    print(f"{passa} {kind:14s} copies={copies}: y ratio {ry:.3f}  s1 ratio {rs:.3f}", flush=True)
    assert ry <= 1.0 and rs <= 1.0, (ry, rs)
