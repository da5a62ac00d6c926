"""fp64 numpy model of the MI355X kernels' algebra (test infrastructure).

Mirrors, step for step, what Passes A, B and C compute (helix_params.h): the
super-chunk groups, the per-segment in-register walk of Pass A with its
in-segment prefix states R_c and segment aggregates D_s, the segment scan of
Pass B, and Pass C's S_init(c) = R_c + exp(ld_c) S_seg(s) assembly. Its only
job is to show that this two-level reassociation equals the sequential
recurrence before any device code runs, the role the reference's own
scan_chunked_ref.cpp plays for its three passes.
"""
from __future__ import annotations

import numpy as np

CS = 64


def softplus(v):
    v = np.asarray(v, np.float64)
    return np.where(v > 20.0, v, np.log1p(np.exp(np.minimum(v, 20.0))))


def two_level_scan(s0, x, dt, A, B, C, ids=None, seg_len=4, chunks_per_group=None,
                   dt_min=0.0, dt_max=np.inf):
    """x [S,L,H,P], dt [S,L,H], A [H], B/C [S,L,G,N], s0 [S,H,P,N] -> y, s1."""
    s0, x, dt, A, B, C = (np.asarray(a, np.float64) for a in (s0, x, dt, A, B, C))
    S, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    hpg = H // G
    n_chunks = (L + CS - 1) // CS
    cpg = chunks_per_group or n_chunks
    y = np.zeros((S, L, H, P))
    s1 = np.zeros((S, H, P, N))
    dtv_all = np.clip(softplus(dt), dt_min, dt_max)  # [S, L, H]

    for base in range(0, n_chunks, cpg):
        n_cg = min(cpg, n_chunks - base)
        n_seg = (n_cg + seg_len - 1) // seg_len
        for seq in range(S):
            src = ids[seq] if ids is not None else seq
            for h in range(H):
                g = h // hpg
                # ---- Pass A: walk each segment with the state "in registers"
                R_local = {}
                D = np.zeros((n_seg, P, N))
                ld = np.zeros(n_cg)
                segld = np.zeros(n_seg)
                chunk_info = {}
                for s in range(n_seg):
                    R = np.zeros((P, N))
                    lam = 0.0
                    for c in range(s * seg_len, min((s + 1) * seg_len, n_cg)):
                        t0 = (base + c) * CS
                        tl = min(CS, L - t0)
                        dtv = dtv_all[seq, t0:t0 + tl, h]
                        lcum = np.cumsum(A[h] * dtv)
                        lend = lcum[-1]
                        sdec = np.exp(lend - lcum)
                        Bc = B[seq, t0:t0 + tl, g, :]
                        Xc = x[seq, t0:t0 + tl, h, :]
                        R_local[c] = R.copy()
                        ld[c] = lam
                        dS = (Xc * (sdec * dtv)[:, None]).T @ Bc        # [P, N]
                        R = np.exp(lend) * R + dS
                        lam += lend
                        chunk_info[c] = (t0, tl, dtv, lcum)
                    D[s] = R
                    segld[s] = lam
                # ---- Pass B: scan over segments
                carry = s0[src, h] if base == 0 else s1[seq, h]
                S_seg = np.zeros_like(D)
                for s in range(n_seg):
                    S_seg[s] = carry
                    carry = np.exp(segld[s]) * carry + D[s]
                s1[seq, h] = carry
                # ---- Pass C: per chunk output
                for c in range(n_cg):
                    s = c // seg_len
                    t0, tl, dtv, lcum = chunk_info[c]
                    S_init = (R_local[c] if c % seg_len else 0.0) + np.exp(ld[c]) * S_seg[s]
                    Cc = C[seq, t0:t0 + tl, g, :]
                    Bc = B[seq, t0:t0 + tl, g, :]
                    CB = np.tril(Cc @ Bc.T)
                    M = CB * np.exp(np.tril(lcum[:, None] - lcum[None, :]))
                    M = np.tril(M)
                    dtX = x[seq, t0:t0 + tl, h, :] * dtv[:, None]
                    y[seq, t0:t0 + tl, h, :] = M @ dtX + np.exp(lcum)[:, None] * (Cc @ S_init.T)
    return y.astype(np.float32), s1.astype(np.float32)
