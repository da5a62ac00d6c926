"""Torch-facing SSD scan operator over the HELIX C ABI.

The host-side mirror of what the reference's ggml bridge does for llama.cpp
(integration/ggml/ggml-helix.cpp:157-361): map tensors (sizes and element
strides) onto a helix_scan_desc, keep a context and a scratch buffer, and
enqueue on the caller's stream. PyTorch provides device memory and the stream
only; all arithmetic runs in the HIP kernels of libhelix.so.
"""
from __future__ import annotations

import math
import threading

import torch

from .abi import Context, HelixError
from .desc import (HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA, HELIX_BF16, HELIX_F16,
                   HELIX_F32, HELIX_OK, HELIX_TENSOR_NULL, HelixScanDesc, HelixTensor)

BACKENDS = {"auto": HELIX_BACKEND_AUTO, "fp32": HELIX_BACKEND_SGMMA, "sgmma": HELIX_BACKEND_SGMMA,
            "bf16": HELIX_BACKEND_MPP, "mpp": HELIX_BACKEND_MPP}
# Storage type of x, B, C and y (helix_scan_desc.io_dtype).
IO_DTYPES = {torch.float32: HELIX_F32, torch.bfloat16: HELIX_BF16, torch.float16: HELIX_F16}

_ctx_lock = threading.Lock()
_contexts: dict[int, Context] = {}
# Scratch is per thread and device, grown monotonically, as the ggml bridge
# keeps it (ggml-helix.cpp:94-130): concurrent encoders must not share one.
_scratch = threading.local()


def context(device: int) -> Context:
    with _ctx_lock:
        ctx = _contexts.get(device)
        if ctx is None:
            ctx = Context(device)
            _contexts[device] = ctx
        return ctx


def tensor_arg(t: torch.Tensor | None) -> HelixTensor:
    if t is None:
        return HELIX_TENSOR_NULL
    return HelixTensor(t.data_ptr(), 0)


def _scratch_for(device: int, nbytes: int) -> torch.Tensor | None:
    if nbytes == 0:
        return None
    pool = getattr(_scratch, "pool", None)
    if pool is None:
        pool = _scratch.pool = {}
    buf = pool.get(device)
    if buf is None or buf.numel() < nbytes:
        buf = torch.empty(nbytes, dtype=torch.uint8, device=f"cuda:{device}")
        pool[device] = buf
    return buf


def make_desc(x: torch.Tensor, dt: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
              s: torch.Tensor, y: torch.Tensor, A: torch.Tensor, *, backend: str = "auto",
              multipass: bool = True, dt_min: float = 0.0, dt_max: float = math.inf) -> HelixScanDesc:
    """Descriptor from tensor shapes and element strides:
    x, y [S, L, H, P]; dt [S, L, H]; B, C [S, L, G, N]; s [S, H, P, N]; A [H]."""
    S, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    d = HelixScanDesc()
    d.n_tok, d.n_seq, d.n_head, d.head_dim, d.d_state, d.n_group = L, S, H, P, N, G
    sx, sy, sb, sc, sdt, ss = x.stride(), y.stride(), B.stride(), C.stride(), dt.stride(), s.stride()
    d.s_x[0], d.s_x[1], d.s_x[2], d.seq_x = sx[1], sx[2], sx[3], sx[0]
    d.s_y[0], d.s_y[1], d.s_y[2], d.seq_y = sy[1], sy[2], sy[3], sy[0]
    d.s_b[0], d.s_b[1], d.s_b[2], d.seq_b = sb[1], sb[2], sb[3], sb[0]
    d.s_c[0], d.s_c[1], d.s_c[2], d.seq_c = sc[1], sc[2], sc[3], sc[0]
    d.s_dt[0], d.s_dt[1], d.seq_dt = sdt[1], sdt[2], sdt[0]
    d.s_s[0], d.s_s[1], d.s_s[2], d.seq_s = ss[1], ss[2], ss[3], ss[0]
    d.s_a = A.stride(0)
    d.io_dtype = IO_DTYPES[x.dtype]
    d.chunk = 0
    d.backend = BACKENDS[backend]
    d.multipass = multipass
    d.dt_min = dt_min
    d.dt_max = dt_max
    return d


def ssd_scan(x: torch.Tensor, dt: torch.Tensor, A: torch.Tensor, B: torch.Tensor, C: torch.Tensor,
             s0: torch.Tensor | None = None, ids: torch.Tensor | None = None, *,
             backend: str = "auto", dt_min: float = 0.0, dt_max: float = math.inf,
             multipass: bool = True,
             y: torch.Tensor | None = None, s1: torch.Tensor | None = None,
             scratch: torch.Tensor | None = None, stream: torch.cuda.Stream | None = None):
    """Chunked SSD prefill scan on the MI355X kernels. Returns (y, s1).

    x [S,L,H,P], dt [S,L,H] (pre-softplus), A [H], B/C [S,L,G,N], s0 [S,H,P,N]
    (zeros when None), ids int32 [S] (source state row per sequence), on one
    gfx950 device. x, B, C and y are float32, bfloat16 or float16 (one type);
    dt, A and the states are float32. multipass=False runs the single-pass kernel (fp32,
    no scratch; backend "bf16" is then declined). Raises HelixError when the
    shape is declined.
    """
    dev = x.device
    if dev.type != "cuda":
        raise ValueError("ssd_scan runs on a HIP device; got " + str(dev))
    # x, B, C (and y) share one storage type: float32, bfloat16 or float16;
    # dt, A and the states are float32.
    if x.dtype not in IO_DTYPES:
        raise ValueError(f"x must be float32, bfloat16 or float16; got {x.dtype}")
    for name, t, want in (("x", x, x.dtype), ("dt", dt, torch.float32), ("A", A, torch.float32),
                          ("B", B, x.dtype), ("C", C, x.dtype)):
        if t.dtype != want or t.device != dev:
            raise ValueError(f"{name} must be {want} on {dev}")
    S, L, H, P = x.shape
    G, N = B.shape[2], B.shape[3]
    if s0 is None:
        s0 = torch.zeros((S, H, P, N), dtype=torch.float32, device=dev)
    if y is None:
        y = torch.empty((S, L, H, P), dtype=x.dtype, device=dev)
    elif y.dtype != x.dtype:
        raise ValueError(f"y must be {x.dtype}")
    if s1 is None:
        s1 = torch.empty((S, H, P, N), dtype=torch.float32, device=dev)
    if ids is not None and (ids.dtype != torch.int32 or not ids.is_contiguous()):
        raise ValueError("ids must be a contiguous int32 tensor")
    d = make_desc(x, dt, B, C, s0, y, A, backend=backend, multipass=multipass, dt_min=dt_min,
                  dt_max=dt_max)
    if tuple(s1.stride()) != tuple(s0.stride()):
        raise ValueError("s0 and s1 must share strides")
    ctx = context(dev.index if dev.index is not None else torch.cuda.current_device())
    if not ctx.supported(d):
        raise HelixError(1, f"shape declined: {ctx.backend_desc(d)}")
    need = ctx.scratch_size(d)
    if scratch is None:
        scratch = _scratch_for(dev.index, need)
    elif scratch.numel() * scratch.element_size() < need:
        raise ValueError(f"scratch needs {need} bytes")
    st = stream if stream is not None else torch.cuda.current_stream(dev)
    rc = ctx.encode(st.cuda_stream, d, tensor_arg(s0), tensor_arg(x), tensor_arg(dt),
                    tensor_arg(A), tensor_arg(B), tensor_arg(C), tensor_arg(ids), tensor_arg(y),
                    tensor_arg(s1), tensor_arg(scratch))
    if rc != HELIX_OK:
        raise HelixError(rc, ctx.last_error())
    return y, s1
