"""Writes tests/golden/*.npz: outputs of the REFERENCE's own fp64 oracle.

Run in a container that has /root/reference, after `make -C oracle ref` has
compiled the reference's src/reference/scan_ref.cpp (and its harness) into
oracle/_ref/libhelix_refimpl.so. Each fixture stores the problem recipe
(generator, shape, seed, ids, dt clamp), a sha256 of the regenerated inputs,
and the reference build's y, s1 (and chunk snapshots). No reference source is
stored; these are data.

    python tests/golden/make_golden.py
"""
from __future__ import annotations

import hashlib
import json
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import pyoracle as po  # noqa: E402

FIXTURES = [
    # name, gen, shape (L,S,H,P,N,G), seed, memory / gauss params, ids, dt_min, dt_max, snapshots
    ("harness_L1", "harness", (1, 1, 2, 64, 128, 1), 4242, "short", None, 0.0, math.inf, False),
    ("harness_L7", "harness", (7, 1, 2, 64, 128, 1), 4242, "short", None, 0.0, math.inf, False),
    ("harness_L65_grouped_ids", "harness", (65, 2, 8, 16, 24, 4), 4242, "long", [1, 0], 0.0,
     math.inf, False),
    ("harness_L129_snapshots", "harness", (129, 1, 2, 16, 40, 1), 20260905, "long", None, 0.0,
     math.inf, True),
    ("harness_L100_clamped", "harness", (100, 1, 2, 16, 32, 1), 99, "short", None, 0.01, 0.5, False),
    ("gauss_cfg0_2heads", "gauss", (256, 1, 2, 64, 64, 1), 1000, [0.0, -1.0, 0.5, 1.0, 16.0], None,
     0.0, math.inf, False),
    ("gauss_cfg3_ragged", "gauss", (1000, 1, 1, 16, 16, 1), 1003, [0.1, -2.0, 1.0, 1.0, 16.0], None,
     0.0, math.inf, True),
]


def main():
    if po.ref_lib() is None:
        raise SystemExit("oracle/_ref/libhelix_refimpl.so missing: run make -C oracle ref")
    for name, gen, shape, seed, dist, ids, dt_min, dt_max, snaps in FIXTURES:
        if gen == "harness":
            p = po.problem_harness(*shape, seed, dist)
        else:
            p = po.problem_gauss(*shape, seed, *dist)
        p.ids = np.asarray(ids, np.int32) if ids is not None else None
        p.d.dt_min, p.d.dt_max = dt_min, dt_max
        h = hashlib.sha256()
        for k in ("s0", "x", "dt", "A", "B", "C"):
            h.update(np.ascontiguousarray(getattr(p, k)).tobytes())
        meta = {"gen": gen, "shape": list(shape), "seed": seed, "ids": ids, "dt_min": dt_min,
                "dt_max": dt_max, "input_sha256": h.hexdigest()}
        if gen == "harness":
            meta["memory"] = dist
        else:
            meta["gauss"] = dist
        out = {}
        if snaps:
            y, s1, sn = po.ref_scan_snapshots(p, 64)
            out["snap"] = sn
        else:
            y, s1 = po.ref_scan(p)
        out.update(y=y, s1=s1, meta=np.array(json.dumps(meta)))
        path = os.path.join(HERE, name + ".npz")
        np.savez_compressed(path, **out)
        print(f"wrote {path} ({os.path.getsize(path)} bytes)")


if __name__ == "__main__":
    main()
