"""Host-side logic of libhelix.so, runnable without a GPU.

Covers what the reference keeps in caps.mm / dispatch.mm / desc.cpp:
descriptor defaults, the shape gate, backend selection, scratch planning and
argument validation, plus the ABI surface itself (every symbol the headers
declare is exported, struct layouts match the reference). A host-only context
(include/helix/helix_host.h) answers exactly as a gfx950 context would, and
its encode returns HELIX_ERR_NO_DEVICE without touching HIP.
"""
from __future__ import annotations

import ctypes
import math
import os
import re

import numpy as np
import pytest

from helix_amd import abi
from helix_amd.desc import (HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_REF,
                            HELIX_BACKEND_SGMMA, HELIX_BF16, HELIX_F16, HELIX_ERR_INVALID_ARG,
                            HELIX_ERR_NO_DEVICE, HELIX_ERR_SCRATCH_TOO_SMALL,
                            HELIX_ERR_UNSUPPORTED_SHAPE, HELIX_A_DIAG_PER_CHANNEL,
                            HELIX_TENSOR_NULL, HelixScanDesc, HelixTensor, algorithmic_bytes,
                            algorithmic_flops, desc_init)
from oracle import pyoracle as po
from algebra_model import two_level_scan
from gpu_harness import env

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CONFIG_SHAPES = {
    "cfg0": (256, 1, 8, 64, 64, 1), "cfg1": (2048, 1, 64, 64, 128, 8),
    "cfg2": (8192, 1, 64, 64, 128, 8), "cfg3": (1000, 4, 32, 128, 128, 1),
    "cfg4a": (4096, 8, 80, 64, 128, 1), "cfg4b": (4096, 8, 27, 192, 128, 1),
}


@pytest.fixture(scope="module")
def host():
    c = abi.Context(host_only=True)
    yield c
    c.close()


def mp(shape, backend=HELIX_BACKEND_AUTO):
    d = abi.desc_init_c(*shape)
    d.multipass = True
    d.backend = backend
    return d


# ---------------------------------------------------------------------------
# ABI surface
# ---------------------------------------------------------------------------

def _declared(header):
    text = open(os.path.join(ROOT, "include", "helix", header)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(helix_[a-z_]+)\s*\(", text)) - {"helix_tensor_is_null"}


def test_library_exports_every_declared_symbol():
    L = abi.lib()
    declared = _declared("helix.h") | _declared("helix_host.h")
    assert declared == set(abi.ABI_SYMBOLS) | set(abi.HOST_SYMBOLS)
    for name in declared:
        assert hasattr(L, name), f"{name} not exported by libhelix.so"


def test_abi_version_and_enums_match_header():
    text = open(os.path.join(ROOT, "include", "helix", "helix.h")).read()
    assert "#define HELIX_ABI_VERSION 1" in text
    for name, val in [("HELIX_OK", 0), ("HELIX_ERR_UNSUPPORTED_SHAPE", 1),
                      ("HELIX_ERR_NO_DEVICE", 2), ("HELIX_ERR_SCRATCH_TOO_SMALL", 3),
                      ("HELIX_ERR_INVALID_ARG", 4), ("HELIX_ERR_PIPELINE", 5),
                      ("HELIX_BACKEND_AUTO", 0), ("HELIX_BACKEND_SGMMA", 1),
                      ("HELIX_BACKEND_MPP", 2), ("HELIX_BACKEND_REF", 3),
                      ("HELIX_F32", 0), ("HELIX_F16", 1), ("HELIX_BF16", 2)]:
        assert re.search(rf"\b{name}\s*=\s*{val}\b", text), name


def test_desc_layout_matches_reference():
    assert ctypes.sizeof(HelixScanDesc) == 248
    assert ctypes.sizeof(HelixTensor) == 16
    R = po.ref_lib()
    if R is not None:
        assert R.ref_desc_size() == ctypes.sizeof(HelixScanDesc)


@pytest.mark.parametrize("shape", list(CONFIG_SHAPES.values()) + [(1, 1, 1, 8, 8, 1), (509, 3, 6, 72, 40, 2)])
def test_desc_init_c_python_and_reference_agree(shape):
    c = abi.desc_init_c(*shape)
    py = desc_init(*shape)
    assert bytes(c) == bytes(py)
    assert c.dt_max == math.inf and c.multipass is False and c.chunk == 0
    R = po.ref_lib()
    if R is not None:
        r = HelixScanDesc()
        R.ref_desc_init(ctypes.byref(r), *shape)
        assert bytes(r) == bytes(c)


# ---------------------------------------------------------------------------
# Shape gate (reference caps.mm:112-151, plus this build's own limits)
# ---------------------------------------------------------------------------

def test_all_baseline_configs_supported(host):
    for name, shape in CONFIG_SHAPES.items():
        for b in (HELIX_BACKEND_AUTO, HELIX_BACKEND_SGMMA, HELIX_BACKEND_MPP):
            assert host.supported(mp(shape, b)), name


def _declined(host, mutate):
    d = mp((256, 2, 4, 64, 128, 2))
    assert host.supported(d)
    mutate(d)
    return not host.supported(d)


@pytest.mark.parametrize("why,mutate", [
    ("zero tokens", lambda d: setattr(d, "n_tok", 0)),
    ("negative heads", lambda d: setattr(d, "n_head", -4)),
    ("heads not a multiple of groups", lambda d: setattr(d, "n_group", 3)),
    ("diagonal A with explicit MPP",
     lambda d: (setattr(d, "a_form", HELIX_A_DIAG_PER_CHANNEL), setattr(d, "backend", HELIX_BACKEND_MPP))),
    ("diagonal A at d_state 256",
     lambda d: (setattr(d, "a_form", HELIX_A_DIAG_PER_CHANNEL), setattr(d, "d_state", 256),
                d.s_s.__setitem__(1, 256))),
    ("unknown A form", lambda d: setattr(d, "a_form", 7)),
    ("bf16 storage with diagonal A",
     lambda d: (setattr(d, "io_dtype", HELIX_BF16), setattr(d, "a_form", HELIX_A_DIAG_PER_CHANNEL))),
    ("bf16 storage with an odd B row stride",
     lambda d: (setattr(d, "io_dtype", HELIX_BF16), d.s_b.__setitem__(0, 2 * 128 + 1))),
    ("unknown storage type", lambda d: setattr(d, "io_dtype", 5)),
    ("bf16 compute dtype", lambda d: setattr(d, "compute_dtype", HELIX_BF16)),
    ("d_state not a multiple of 8", lambda d: setattr(d, "d_state", 60)),
    ("head_dim not a multiple of 8", lambda d: setattr(d, "head_dim", 60)),
    ("d_state above 256 with explicit MPP",
     lambda d: (setattr(d, "d_state", 264), d.s_s.__setitem__(1, 264), setattr(d, "backend", HELIX_BACKEND_MPP))),
    ("d_state above 256 with bf16 storage",
     lambda d: (setattr(d, "d_state", 264), d.s_s.__setitem__(1, 264), setattr(d, "io_dtype", HELIX_BF16))),
    ("strided B state", lambda d: d.s_b.__setitem__(2, 2)),
    ("strided C state", lambda d: d.s_c.__setitem__(2, 2)),
    ("strided s state", lambda d: d.s_s.__setitem__(2, 2)),
    ("s rows not d_state apart", lambda d: d.s_s.__setitem__(1, 256)),
    ("chunk 32", lambda d: setattr(d, "chunk", 32)),
    ("single pass with explicit MPP",
     lambda d: (setattr(d, "multipass", False), setattr(d, "backend", HELIX_BACKEND_MPP))),
    ("REF backend", lambda d: setattr(d, "backend", HELIX_BACKEND_REF)),
    ("grid z overflow", lambda d: setattr(d, "n_seq", 70000)),
])
def test_gate_declines(host, why, mutate):
    assert _declined(host, mutate), why


def test_gate_accepts_ragged_strided_and_odd_shapes(host):
    for shape in [(1, 1, 1, 8, 8, 1), (1000, 3, 6, 72, 40, 2), (129, 2, 4, 192, 256, 4)]:
        assert host.supported(mp(shape))
    d = mp((300, 2, 4, 64, 128, 1))
    d.s_x[0] = 4 * 64 + 16          # padded token rows (a ggml view)
    d.s_x[2] = 1
    d.s_y[2] = 1
    d.chunk = 64
    assert host.supported(d)


@pytest.mark.parametrize("n,blocks,size", [(264, 3, 88), (384, 3, 128), (512, 4, 128), (520, 5, 104),
                                            (1000, 8, 128), (4104, 33, 128)])
@pytest.mark.parametrize("multipass", [True, False])
def test_state_blocks_above_256(host, n, blocks, size, multipass):
    """d_state above 256 (the reference gate takes any multiple of 8,
    caps.mm:129) runs as equal blocks of at most 128 state indices on the
    fp32 path; the plan is one block's, launched once per block."""
    d = abi.desc_init_c(300, 2, 4, 64, n, 2)
    d.multipass = multipass
    assert host.supported(d)
    assert host.select_backend(d) == HELIX_BACKEND_SGMMA
    k = host.plan_info(d)
    assert k.state_blocks == blocks
    b = abi.desc_init_c(300, 2, 4, 64, size, 2)
    b.multipass = multipass
    b.backend = HELIX_BACKEND_SGMMA
    kb = host.plan_info(b)
    assert kb.state_blocks == 1
    assert k.np == kb.np == 128
    assert host.scratch_size(d) == host.scratch_size(b)
    if multipass:
        assert k.kernel_a == kb.kernel_a and k.kernel_c == kb.kernel_c and k.seg_len == kb.seg_len
        assert k.launches == blocks * kb.launches
        assert host.scratch_size(d) > 0
    else:
        # The first block may keep its tiles in y (as one block of its size
        # would); the others run the one-launch kernel.
        assert k.kernel_1pass == kb.kernel_1pass == b"helix_scan_1pass_f32_n128"
        assert k.state_in_y == kb.state_in_y
        assert k.launches == (3 if k.state_in_y else 1) + blocks - 1
        assert host.scratch_size(d) == 0
    for mutate in (lambda x: setattr(x, "backend", HELIX_BACKEND_MPP),
                   lambda x: setattr(x, "io_dtype", HELIX_F16),
                   lambda x: setattr(x, "a_form", HELIX_A_DIAG_PER_CHANNEL),
                   lambda x: x.s_s.__setitem__(1, n + 8)):
        e = abi.desc_init_c(300, 2, 4, 64, n, 2)
        e.multipass = multipass
        mutate(e)
        assert not host.supported(e)


def test_state_blocks_from_129(host):
    # From d_state 129 to 256 blocks of at most 128 are the default with fp32
    # storage and scalar A (faster than the d_state 256 kernels);
    # HELIX_STATE_BLOCKS=0 keeps one launch sequence there.
    native = tuned(HELIX_STATE_BLOCKS="0")
    for n, blocks in ((8, 1), (128, 1), (136, 2), (192, 2), (256, 2)):
        for backend in (HELIX_BACKEND_AUTO, HELIX_BACKEND_MPP, HELIX_BACKEND_SGMMA):
            d = mp((300, 2, 4, 64, n, 2), backend)
            k = host.plan_info(d)
            assert k.state_blocks == blocks, (n, backend)
            assert k.np == (64 if n <= 64 else 128)
            assert native.plan_info(d).state_blocks == 1
            # The caller's backend is kept up to 256.
            assert host.select_backend(d) == (HELIX_BACKEND_SGMMA if backend == HELIX_BACKEND_SGMMA
                                              else HELIX_BACKEND_MPP)
    # Each block reads 128 of the 256 columns of B's and C's rows: Pass A
    # writes bf16 copies of its columns for the walks.
    d = mp((300, 2, 4, 64, 256, 2))
    assert host.plan_info(d).kernel_c == b"helix_scan_walk16_bf16_bc_n128"
    assert tuned(HELIX_WALK_BCCOPY="0").plan_info(d).kernel_c == b"helix_scan_walk16_bf16_n128"
    assert native.plan_info(d).kernel_c == b"helix_scan_walk16_bf16_n256"
    # 16-bit storage and diagonal A keep one launch sequence.
    e = mp((300, 2, 4, 64, 256, 2))
    e.io_dtype = HELIX_BF16
    assert host.plan_info(e).state_blocks == 1
    f = abi.desc_init_c(300, 2, 4, 64, 256, 2)
    f.multipass = False
    kf = host.plan_info(f)
    assert kf.state_blocks == 2 and kf.launches == (3 if kf.state_in_y else 1) + 1
    native.close()


def test_diagonal_a_runs_the_single_pass_walk(host):
    # Diagonal A: one launch of the diagonal single-pass kernel for either
    # value of multipass, AUTO or SGMMA, no scratch.
    for multipass in (True, False):
        for backend in (HELIX_BACKEND_AUTO, HELIX_BACKEND_SGMMA):
            for n, want in ((16, 64), (64, 64), (128, 128)):
                d = mp((300, 2, 4, 64, n, 2), backend)
                d.multipass = multipass
                d.a_form = HELIX_A_DIAG_PER_CHANNEL
                d.s_a = n
                assert host.supported(d)
                assert host.select_backend(d) == HELIX_BACKEND_SGMMA
                assert host.backend_desc(d) == f"mfma fp32, single pass, diagonal A (d_state<={want})"
                assert host.scratch_size(d) == 0
                k = host.plan_info(d)
                assert k.kernel_1pass == b"helix_scan_1pass_diag_f32_n%d" % want
                assert (k.launches, k.total_bytes, k.kernel_a) == (1, 0, None)


def tuned(**kv):
    """A host-only context created under these environment settings: the
    tuning knobs are read once, when a context is created."""
    with env(**kv):
        return abi.Context(host_only=True)


@pytest.mark.parametrize("io,name", [(HELIX_BF16, "bf16"), (HELIX_F16, "f16")])
def test_16bit_storage_selection(host, io, name):
    # 16-bit x/B/C/y: a bf16 multipass request walks segments (Pass A's
    # aggregate and the walking Pass C read 16-bit operands); everything else
    # runs the single pass with fp32 compute and no scratch.
    shape = CONFIG_SHAPES["cfg2"]
    d = mp(shape)
    d.io_dtype = io
    assert host.supported(d)
    assert host.backend_desc(d) == (f"mfma bf16 pass C, chunk walk, pass A fp16x3 (scaled planes), {name} storage "
                                    f"(d_state<=128)")
    k = host.plan_info(d)
    assert (k.kernel_a, k.kernel_b, k.kernel_c) == (
        f"helix_chunk_state_hb_h3agg_{name}io_n128".encode(), b"helix_state_scan_f32",
        f"helix_scan_walk16_bf16_{name}io_n128".encode())
    x6 = tuned(HELIX_PASSA_F16="0")         # six bf16 split products
    assert x6.plan_info(d).kernel_a == f"helix_chunk_state_hb_x6agg_{name}io_n128".encode()
    assert x6.backend_desc(d) == f"mfma bf16 pass C, chunk walk, pass A bf16x6, {name} storage (d_state<=128)"
    assert k.pass_b == abi.PASS_B_LAUNCHED
    x3 = tuned(HELIX_PASSA_SPLIT="3")       # Pass A on three split products: opt-in
    assert x3.plan_info(d).kernel_a == f"helix_chunk_state_hb_x3agg_{name}io_n128".encode()
    assert x3.backend_desc(d) == (f"mfma bf16 pass C, chunk walk, pass A bf16x3 (narrower state: opt-in), "
                                  f"{name} storage (d_state<=128)")
    assert k.total_bytes == host.scratch_size(d) > 0 and k.s_local_bytes == 0
    for backend, multipass in ((HELIX_BACKEND_SGMMA, True), (HELIX_BACKEND_AUTO, False),
                               (HELIX_BACKEND_SGMMA, False)):
        d = mp((300, 2, 4, 64, 256, 2), backend)
        d.multipass = multipass
        d.io_dtype = io
        assert host.supported(d)
        assert host.backend_desc(d) == f"mfma fp32, single pass, {name} storage (d_state<=256)"
        assert host.scratch_size(d) == 0
        assert host.plan_info(d).kernel_1pass == f"helix_scan_1pass_{name}io_n256".encode()
    d = mp(shape)
    d.io_dtype = io
    assert tuned(HELIX_FORCE_BACKEND="sgmma").plan_info(d).kernel_1pass == f"helix_scan_1pass_{name}io_n128".encode()


def test_null_context_and_desc():
    L = abi.lib()
    d = mp((64, 1, 1, 8, 8, 1))
    assert not L.helix_scan_supported(None, ctypes.byref(d))
    assert L.helix_ctx_select_backend(None, ctypes.byref(d)) == HELIX_BACKEND_REF
    assert L.helix_ctx_backend_desc(None, ctypes.byref(d)) == b"unavailable (null context)"
    assert L.helix_scan_scratch_size(None, None) == 0


def test_noalloc_host_checks(host):
    # helix_scan_encode_noalloc plans for its fixed array: a scan whose plan
    # needs more under the context's budget (config 4a with fourteen sequences
    # on the bf16 path, 168 MiB; config 2 at d_state 256 on the fp32 path, whose
    # Pass A stores every chunk's state, 520 MiB) is cut into more groups;
    # only one that does not fit at one chunk per group is refused, before
    # anything is enqueued. A host-only context has no device for one that
    # fits. Config 4a itself fits (76 MiB).
    # (d_state 256 cases with one launch sequence, HELIX_STATE_BLOCKS=0: in
    # blocks of 128 the same shapes need far less.)
    t = [HelixTensor(0x1000 * (i + 1), 0) for i in range(9)]
    native = tuned(HELIX_STATE_BLOCKS="0")
    assert 0 < host.scratch_size(mp(CONFIG_SHAPES["cfg4a"])) <= abi.NOALLOC_SCRATCH_BYTES
    for shape, backend, c in (((4096, 14, 80, 64, 128, 1), HELIX_BACKEND_MPP, host),
                              ((8192, 1, 64, 64, 256, 8), HELIX_BACKEND_SGMMA, native)):
        d = mp(shape, backend)
        assert c.scratch_size(d) > abi.NOALLOC_SCRATCH_BYTES
        with env(HELIX_SCRATCH_MB=str(abi.NOALLOC_SCRATCH_BYTES >> 20),
                 HELIX_STATE_BLOCKS="0" if c is native else None):
            capped = abi.Context(host_only=True).plan_info(d)
        assert capped.n_groups > 1 and capped.total_bytes <= abi.NOALLOC_SCRATCH_BYTES
        assert c.encode_noalloc(0, d, *t) == HELIX_ERR_NO_DEVICE
    assert 0 < host.scratch_size(mp((8192, 1, 64, 64, 256, 8), HELIX_BACKEND_SGMMA)) <= abi.NOALLOC_SCRATCH_BYTES
    huge = mp((64, 1, 4096, 64, 256, 1), HELIX_BACKEND_SGMMA)   # one chunk's state is 256 MiB
    assert native.encode_noalloc(0, huge, *t) == HELIX_ERR_SCRATCH_TOO_SMALL
    assert "HELIX_NOALLOC_SCRATCH_BYTES" in native.last_error()
    native.close()
    fits = mp(CONFIG_SHAPES["cfg2"])
    assert 0 < host.scratch_size(fits) <= abi.NOALLOC_SCRATCH_BYTES
    assert host.encode_noalloc(0, fits, *t) == HELIX_ERR_NO_DEVICE
    bad = mp((64, 1, 2, 64, 260, 1))
    assert host.encode_noalloc(0, bad, *t) == HELIX_ERR_UNSUPPORTED_SHAPE
    assert abi.lib().helix_scan_encode_noalloc(None, None, None, *t) == HELIX_ERR_INVALID_ARG
    header = open(os.path.join(ROOT, "include", "helix", "helix_host.h")).read()
    assert re.search(r"#define HELIX_NOALLOC_SCRATCH_BYTES \(128u << 20\)", header)
    assert abi.NOALLOC_SCRATCH_BYTES == 128 << 20


def test_tuning_read_once_per_context():
    # A context keeps the tuning it was created with: changing the environment
    # afterwards changes neither its kernels nor its scratch layout, so
    # helix_scan_scratch_size and helix_scan_encode always agree.
    shape = CONFIG_SHAPES["cfg2"]
    c = tuned()
    k0 = c.plan_info(mp(shape))
    with env(HELIX_PASSA_SPLIT="3", HELIX_SCRATCH_MB="1", HELIX_SEG_LEN="2", HELIX_WALK_BCCOPY="0",
             HELIX_FORCE_BACKEND="sgmma", HELIX_FUSE_B="1"):
        k1 = c.plan_info(mp(shape))
        assert c.select_backend(mp(shape)) == HELIX_BACKEND_MPP
        assert c.scratch_size(mp(shape)) == k0.total_bytes
    for f in ("kernel_a", "kernel_b", "kernel_c", "total_bytes", "seg_len", "n_groups", "launches"):
        assert getattr(k0, f) == getattr(k1, f), f
    c.close()


# ---------------------------------------------------------------------------
# Backend selection (reference caps.mm:79-110)
# ---------------------------------------------------------------------------

def test_backend_selection(host):
    shape = CONFIG_SHAPES["cfg2"]
    assert host.select_backend(mp(shape, HELIX_BACKEND_AUTO)) == HELIX_BACKEND_MPP
    assert host.select_backend(mp(shape, HELIX_BACKEND_MPP)) == HELIX_BACKEND_MPP
    assert host.select_backend(mp(shape, HELIX_BACKEND_SGMMA)) == HELIX_BACKEND_SGMMA
    # bf16x6 split products: Pass A on every path, and the fp32 path's Pass C
    # up to d_state 128, which walks each segment with the state in registers
    # (HELIX_F32_WALK=0: chunk-parallel on stored states).
    assert (host.backend_desc(mp(shape, HELIX_BACKEND_SGMMA))
            == "mfma fp32, passes A and C bf16x6, chunk walk (d_state<=128)")
    kw = host.plan_info(mp(shape, HELIX_BACKEND_SGMMA))
    assert (kw.kernel_a, kw.kernel_b, kw.kernel_c) == (
        b"helix_chunk_state_hb_x6agg_r64_n128", b"helix_state_scan_f32", b"helix_scan_walk_x6_n128")
    assert kw.pass_b == abi.PASS_B_LAUNCHED and kw.launches == 3
    assert kw.s_local_bytes == 0 and kw.bf16_state == 0 and (kw.seg_len, kw.walk_len) == (8, 16)
    f0 = tuned(HELIX_F32_WALK="0")
    assert (f0.backend_desc(mp(shape, HELIX_BACKEND_SGMMA))
            == "mfma fp32, passes A and C bf16x6 (d_state<=128)")
    assert f0.plan_info(mp(shape, HELIX_BACKEND_SGMMA)).kernel_c == b"helix_chunk_out_x6_n128"
    # The bf16 path walks segments in Pass C at every d_state. Its Pass A keeps
    # the carried state fp32-accurate (reference caps.mm:65-73): on two scaled
    # fp16 planes (three products) with fp32 storage up to d_state 128, on six
    # bf16 split products otherwise or with HELIX_PASSA_F16=0;
    # HELIX_PASSA_SPLIT=3 opts into three bf16 products.
    h3 = "mfma bf16 pass C, chunk walk, pass A fp16x3 (scaled planes) (d_state<=128)"
    assert host.backend_desc(mp(shape)) == h3
    assert host.backend_desc(mp((64, 1, 1, 64, 128, 1))) == h3
    x6 = tuned(HELIX_PASSA_F16="0")
    assert x6.backend_desc(mp(shape)) == "mfma bf16 pass C, chunk walk, pass A bf16x6 (d_state<=128)"
    assert x6.plan_info(mp(shape)).kernel_a == b"helix_chunk_state_hb_x6agg_n128"
    assert host.plan_info(mp(shape)).kernel_a == b"helix_chunk_state_hb_h3agg_n128"
    assert host.plan_info(mp((64, 1, 1, 64, 64, 1))).kernel_a == b"helix_chunk_state_hb_h3agg_n64"
    # d_state 256: blocks of 128 by default, one launch sequence on the d_state
    # 256 kernels with HELIX_STATE_BLOCKS=0.
    native = tuned(HELIX_STATE_BLOCKS="0")
    assert (host.backend_desc(mp((4096, 1, 32, 64, 256, 1)))
            == h3 + ", in blocks of at most 128 state indices")
    assert (native.backend_desc(mp((4096, 1, 32, 64, 256, 1)))
            == "mfma bf16 pass C, chunk walk, pass A bf16x6 (d_state<=256)")
    assert (native.backend_desc(mp((64, 1, 1, 64, 256, 1)))
            == "mfma bf16 pass C, chunk walk, pass A bf16x6 (d_state<=256)")
    x3 = tuned(HELIX_PASSA_SPLIT="3")
    assert x3.backend_desc(mp(shape)) == ("mfma bf16 pass C, chunk walk, pass A bf16x3 (narrower state: opt-in) "
                                          "(d_state<=128)")
    assert x3.plan_info(mp(shape)).kernel_a == b"helix_chunk_state_hb_x3agg_n128"
    assert (native.backend_desc(mp((64, 1, 1, 64, 256, 1), HELIX_BACKEND_SGMMA))
            == "mfma fp32, pass A bf16x6 (d_state<=256)")
    native.close()
    # d_state 64 walks too, where the plan walks more than one chunk; one
    # chunk (a single-chunk sequence, or config 0's four chunks over eight
    # heads) keeps the chunk-parallel Pass C unless HELIX_F32_WALK=1.
    n64 = (8192, 1, 64, 64, 64, 8)
    assert (host.backend_desc(mp(n64, HELIX_BACKEND_SGMMA))
            == "mfma fp32, passes A and C bf16x6, chunk walk (d_state<=64)")
    k64 = host.plan_info(mp(n64, HELIX_BACKEND_SGMMA))
    assert (k64.kernel_a, k64.kernel_c) == (b"helix_chunk_state_hb_x6agg_r64_n64", b"helix_scan_walk_x6_n64")
    assert k64.walk_len > 1
    assert tuned(HELIX_F32_WALK="0").plan_info(mp(n64, HELIX_BACKEND_SGMMA)).kernel_c == b"helix_chunk_out_x6_n64"
    for short in ((64, 1, 1, 64, 64, 1), CONFIG_SHAPES["cfg0"]):
        assert (host.backend_desc(mp(short, HELIX_BACKEND_SGMMA))
                == "mfma fp32, passes A and C bf16x6 (d_state<=64)")
        kw1 = tuned(HELIX_F32_WALK="1").plan_info(mp(short, HELIX_BACKEND_SGMMA))
        assert kw1.kernel_c == b"helix_scan_walk_x6_n64" and kw1.walk_len == 1
    # The plan names the kernels each pass launches.
    k = host.plan_info(mp(shape))
    # Eight heads per group: the walk reads the caller's fp32 B and C (no
    # bf16 copies). Pass B keeps its own launch: the walk's prologue scans
    # only walk segments that are Pass A's segments too (HELIX_FUSE_B=1 with
    # HELIX_SEG_LEN=16 runs it there).
    assert (k.kernel_a, k.kernel_b, k.kernel_c) == (
        b"helix_chunk_state_hb_h3agg_n128", b"helix_state_scan_f32", b"helix_scan_walk16_bf16_n128")
    assert k.bccopy_bytes == 0 and k.pass_b == abi.PASS_B_LAUNCHED
    # Pass A (head blocks of four heads) runs 8-chunk segments, 16 per
    # sequence; the walk runs 16-chunk ones, each starting at every other
    # Pass A segment.
    assert (k.seg_len, k.segs_per_group, k.walk_len, k.walks_per_group) == (8, 16, 16, 8)
    assert k.launches == 3
    assert tuned(HELIX_FUSE_B="1").plan_info(mp(shape)).kernel_b == b"helix_state_scan_f32"
    kf = tuned(HELIX_FUSE_B="1", HELIX_SEG_LEN="16").plan_info(mp(shape))
    assert kf.kernel_b is None and kf.launches == 2 and kf.seg_len == kf.walk_len == 16
    assert kf.pass_b == abi.PASS_B_IN_C
    # Configs 4a and 4b: one group, walks that are Pass A's segments, fused by
    # default. The dispatch model takes 43-chunk walks (43 + 21 per sequence)
    # at 4a and 22-chunk ones (22 + 22 + 20) at 4b, where a 16-chunk cap gave
    # four of each.
    k4 = host.plan_info(mp(CONFIG_SHAPES["cfg4a"]))
    assert k4.segs_per_group == 2 and k4.kernel_b is None and k4.launches == 2 and k4.pass_b == abi.PASS_B_IN_C
    assert k4.seg_len == k4.walk_len == 43 and k4.walks_per_group == 2
    k4b = host.plan_info(mp(CONFIG_SHAPES["cfg4b"]))
    assert (k4b.seg_len, k4b.walk_len, k4b.segs_per_group, k4b.pass_b) == (22, 22, 3, abi.PASS_B_IN_C)
    # HELIX_WALK_LEN and HELIX_SEG_LEN override it (the 16-chunk plan), and
    # HELIX_WALK_LEN alone sets both lengths where Pass A's segment is the walk.
    k16 = tuned(HELIX_WALK_LEN="16", HELIX_SEG_LEN="16").plan_info(mp(CONFIG_SHAPES["cfg4a"]))
    assert (k16.seg_len, k16.walk_len, k16.segs_per_group, k16.pass_b) == (16, 16, 4, abi.PASS_B_IN_C)
    kw = tuned(HELIX_WALK_LEN="32").plan_info(mp(CONFIG_SHAPES["cfg4a"]))
    assert (kw.seg_len, kw.walk_len, kw.segs_per_group) == (32, 32, 2)
    km = tuned(HELIX_SCRATCH_MB="1").plan_info(mp(shape))   # many groups, carried through s1
    assert km.n_groups > 1 and km.kernel_b == b"helix_state_scan_f32" and km.pass_b == abi.PASS_B_LAUNCHED
    assert km.launches == 3 * km.n_groups
    L, S, H, P, N, G = shape
    # HELIX_WALK_BCCOPY=1: Pass A writes bf16 copies of B and C that the walk reads.
    kc = tuned(HELIX_WALK_BCCOPY="1").plan_info(mp(shape))
    assert (kc.kernel_a, kc.kernel_c) == (b"helix_chunk_state_hb_h3agg_bc_n128", b"helix_scan_walk16_bf16_bc_n128")
    assert kc.bccopy_bytes == 2 * (S * L * G * N * 2)
    assert k4.bccopy_bytes > 0   # 80 heads per group: copies by default
    # Pass A writes one decay record per (seq, chunk, head, token) for the
    # walk and for the fp32 path's bf16x6 Pass C.
    # 8 bytes for the walk (dt, Lcum log2 e), 16 for the fp32 path (dt,
    # exp(Lcum), Lcum in fp64).
    recs = S * (-(-L // 64)) * H * 64
    assert k.rec_bytes == 8 * recs
    assert host.plan_info(mp(shape, HELIX_BACKEND_SGMMA)).rec_bytes == 16 * recs
    native = tuned(HELIX_STATE_BLOCKS="0")   # d_state 256 on its own kernels
    assert native.plan_info(mp((64, 1, 1, 64, 256, 1), HELIX_BACKEND_SGMMA)).rec_bytes == 0
    assert kc.total_bytes >= kc.s_seg_bytes + kc.bccopy_bytes and kc.total_bytes > k.total_bytes
    k0 = tuned(HELIX_WALK_BCCOPY="0").plan_info(mp(CONFIG_SHAPES["cfg4a"]))
    assert b"_bc_" not in k0.kernel_a and b"_bc_" not in k0.kernel_c and k0.bccopy_bytes == 0
    k = host.plan_info(mp(shape, HELIX_BACKEND_SGMMA))
    assert (k.kernel_a, k.kernel_c) == (b"helix_chunk_state_hb_x6agg_r64_n128", b"helix_scan_walk_x6_n128")
    k = tuned(HELIX_F32_WALK="0").plan_info(mp(shape, HELIX_BACKEND_SGMMA))
    assert (k.kernel_a, k.kernel_c) == (b"helix_chunk_state_hb_x6f32_n128", b"helix_chunk_out_x6_n128")
    k = native.plan_info(mp((64, 1, 1, 64, 256, 1), HELIX_BACKEND_SGMMA))
    assert (k.kernel_a, k.kernel_c) == (b"helix_chunk_state_x6f32_n256", b"helix_chunk_out_f32_n256")
    native.close()
    # multipass=false (the descriptor default) runs the fp32 single-pass
    # kernel under AUTO and SGMMA; an explicit MPP request is declined there
    # (reference caps.mm:66,145-147).
    d = mp(shape)
    d.multipass = False
    assert host.backend_desc(d) == "mfma fp32, single pass (d_state<=128)"
    assert host.select_backend(d) == HELIX_BACKEND_SGMMA
    d.backend = HELIX_BACKEND_SGMMA
    assert host.backend_desc(d) == "mfma fp32, single pass (d_state<=128)"
    d.backend = HELIX_BACKEND_MPP
    assert host.backend_desc(d) == "declined (shape unsupported)"
    # With fp32 storage, scalar A and d_state <= 128 the single pass runs as
    # the fp32 path's three passes with their state tiles in y (state_in_y),
    # where every segment has the rows of a tile: 65 rows at d_state 64 and a
    # 64-channel slab, 129 at 128. 100 tokens leave only d_state 64 there; the
    # one-launch kernel stays named as the encoder's fallback.
    # d_state 256 runs as two blocks of 128, each one launch.
    for n, want, in_y in ((64, 64, 1), (40, 64, 1), (96, 128, 0), (256, 128, 0)):
        d = mp((100, 1, 2, 64, n, 1))
        d.multipass = False
        k = host.plan_info(d)
        launches = 3 if in_y else 2 if n > 128 else 1
        assert (k.np, k.launches, k.total_bytes, k.n_groups, k.state_in_y) == (want, launches, 0, 1, in_y)
        assert k.kernel_1pass == b"helix_scan_1pass_f32_n%d" % want
        if in_y:
            assert (k.kernel_a, k.kernel_b, k.kernel_c) == (
                b"helix_chunk_state_hb_x6agg_n64", b"helix_state_scan_y_f32", b"helix_scan_walk_x6_y_n64")
            assert k.s_seg_bytes == k.rec_bytes == 0
        else:
            assert k.kernel_a is None and k.kernel_b is None and k.kernel_c is None
    # Config 2: Pass A's 8-chunk segments, 16-chunk walks, as the fp32 path;
    # HELIX_1PASS_Y=0 keeps the one-launch kernel.
    d = mp(CONFIG_SHAPES["cfg2"])
    d.multipass = False
    k = host.plan_info(d)
    assert (k.state_in_y, k.launches, k.seg_len, k.walk_len, k.total_bytes) == (1, 3, 8, 16, 0)
    k0 = tuned(HELIX_1PASS_Y="0").plan_info(d)
    assert (k0.state_in_y, k0.launches, k0.kernel_a) == (0, 1, None)
    # Config 1: the planner's 2-chunk segments are shorter than a tile's 129
    # rows, and 3-chunk ones leave a last segment of 128 tokens; the segments
    # grow to 4 chunks and the walks keep two of them.
    d = mp(CONFIG_SHAPES["cfg1"])
    d.multipass = False
    k = host.plan_info(d)
    assert (k.state_in_y, k.seg_len, k.walk_len) == (1, 4, 8)
    assert host.plan_info(mp(shape)).kernel_1pass is None
    assert tuned(HELIX_FORCE_BACKEND="sgmma").select_backend(mp(shape, HELIX_BACKEND_MPP)) == HELIX_BACKEND_SGMMA


# ---------------------------------------------------------------------------
# Scratch planning (reference caps.mm:153-241)
# ---------------------------------------------------------------------------

def test_bc_copy_condition(host):
    native = tuned(HELIX_STATE_BLOCKS="0")   # d_state 256 on its own kernels
    # Up to d_state 128 the head-block Pass A writes the copies when more than
    # eight (head, P slab) items share a group's rows (K = heads_per_group *
    # n_pslab > 8). At d_state 256 the per-item Pass A needs the K workgroups
    # of a chunk to cover its 64 rows with two quads of four state indices per
    # thread: ceil(64 / K) * d_state / 4 <= 512.
    for (H, P, N, G), copy in [((64, 64, 128, 8), False), ((72, 64, 128, 8), True), ((16, 64, 128, 1), True),
                               ((4, 64, 128, 1), False), ((2, 64, 128, 1), False), ((3, 192, 128, 1), True),
                               ((1, 192, 128, 1), False), ((9, 64, 64, 1), True), ((1, 64, 128, 1), False),
                               ((8, 64, 256, 1), True), ((4, 64, 256, 1), False), ((2, 128, 256, 1), False),
                               ((4, 128, 256, 1), True)]:
        d = mp((4096, 1, H, P, N, G))
        k = (native if N > 128 else host).plan_info(d)
        assert (k.bccopy_bytes > 0) == copy, (H, P, N, G)
        assert k.kernel_c.endswith(b"_n%d" % k.np)
        assert (b"_bc_" in k.kernel_a) == copy and (b"_bc_" in k.kernel_c) == copy
        assert (b"_hb_" in k.kernel_a) == (N <= 128)
    # A block of state indices reads d_state of each row's columns: copies at
    # any K. A caller's B and C inside wider rows are planned as usual.
    for G in (8, 1):
        H = 8 * G
        d = mp((4096, 1, H, 64, 256, G))
        k = host.plan_info(d)
        assert k.state_blocks == 2 and k.bccopy_bytes > 0 and b"_bc_" in k.kernel_c, G
        assert tuned(HELIX_WALK_BCCOPY="0").plan_info(d).bccopy_bytes == 0
        d = mp((4096, 1, H, 64, 128, G))
        for s in (d.s_b, d.s_c):
            s[0], s[1] = G * 256, 256
        d.seq_b = d.seq_c = 4096 * G * 256
        assert host.plan_info(d).bccopy_bytes == 0
    # Not with 16-bit storage (Pass C reads the caller's 16-bit B and C).
    d = mp((4096, 1, 64, 64, 128, 8))
    d.io_dtype = HELIX_BF16
    assert host.plan_info(d).bccopy_bytes == 0


@pytest.mark.parametrize("name", list(CONFIG_SHAPES))
@pytest.mark.parametrize("backend", [HELIX_BACKEND_SGMMA, HELIX_BACKEND_MPP])
def test_plan_invariants(host, name, backend):
    shape = CONFIG_SHAPES[name]
    L, S, H, P, N, G = shape
    d = mp(shape, backend)
    info = host.plan_info(d)
    assert info.total_bytes == host.scratch_size(d)
    assert info.n_chunks == (L + 63) // 64
    assert 1 <= info.chunks_per_group <= info.n_chunks
    assert info.n_groups * info.chunks_per_group >= info.n_chunks
    assert (info.n_groups - 1) * info.chunks_per_group < info.n_chunks
    assert 1 <= info.seg_len <= info.chunks_per_group
    assert info.segs_per_group == -(-info.chunks_per_group // info.seg_len)
    hpg = H // G
    assert info.hblk * info.n_hblk >= hpg and (info.n_hblk - 1) * info.hblk < hpg
    # State scratch is stored as padded 64 x np slab tiles (helix_params.h).
    state = S * H * (-(-P // 64)) * 64 * info.np
    assert info.np == (64 if N <= 64 else 128 if N <= 128 else 256)
    assert info.bf16_state == (backend == HELIX_BACKEND_MPP)
    # The walking Pass C keeps the chunk-local states in registers, so its
    # plan holds no s_local region; it is the bf16 path's Pass C, and the
    # fp32 path's at d_state <= 128 where its walks are longer than a chunk.
    walk = b"walk" in info.kernel_c
    assert walk == (backend == HELIX_BACKEND_MPP or (N <= 128 and info.walk_len > 1))
    want_sl = state * info.chunks_per_group * 4 if (info.seg_len > 1 and not walk) else 0
    assert info.s_local_bytes == want_sl
    assert info.s_seg_bytes == state * info.segs_per_group * 4
    # every region 256-byte aligned and the total covers them all
    assert info.total_bytes % 256 == 0
    assert info.total_bytes >= want_sl + info.s_seg_bytes
    # Pass A's segments nest in the walk's; off the walk they are the same.
    assert info.walk_len % info.seg_len == 0
    assert info.walks_per_group == -(-info.chunks_per_group // info.walk_len)
    assert walk or info.walk_len == info.seg_len
    # The walks (bf16, and the fp32 path's at d_state <= 128) run Pass B's
    # segment scan in their prologue when the plan has one group of at most
    # four segments that are also its walk segments: no Pass B launch.
    fused = walk and info.n_groups == 1 and info.segs_per_group <= 4 and info.seg_len == info.walk_len
    assert info.launches == (2 if fused else 3 * info.n_groups)
    assert (info.kernel_b is None) == fused
    assert info.pass_b == (abi.PASS_B_IN_C if fused else abi.PASS_B_LAUNCHED)


def test_plan_single_group_for_baseline_configs(host):
    # With the default budget every BASELINE config runs as one group.
    for name, shape in CONFIG_SHAPES.items():
        for b in (HELIX_BACKEND_SGMMA, HELIX_BACKEND_MPP):
            assert host.plan_info(mp(shape, b)).n_groups == 1, name


def test_tiny_budget_forces_many_groups(host):
    shape = (2048, 1, 8, 64, 128, 2)
    info = tuned(HELIX_SCRATCH_MB=1).plan_info(mp(shape))
    assert info.n_groups > 1
    # 1 MiB admits at least one chunk; never more than the budget unless
    # a single chunk alone exceeds it.
    one_chunk = 8 * 64 * 128 * 2
    assert info.total_bytes <= max(1 << 20, 2 * one_chunk + 4096) or info.chunks_per_group == 1
    assert tuned(HELIX_SCRATCH_MB=None).plan_info(mp(shape)).n_groups == 1


def test_scratch_zero_for_single_pass(host):
    d = mp(CONFIG_SHAPES["cfg1"])
    d.multipass = False
    assert host.scratch_size(d) == 0


def test_seg_len_and_hblk_overrides(host):
    shape = CONFIG_SHAPES["cfg2"]
    info = tuned(HELIX_SEG_LEN=4, HELIX_HBLK=8).plan_info(mp(shape))
    assert info.seg_len == 4 and info.hblk == 8 and info.n_hblk == 1


# ---------------------------------------------------------------------------
# Encode argument validation (reference dispatch.mm:55-153): no GPU needed,
# every error is detected before anything is enqueued.
# ---------------------------------------------------------------------------

def _tensors(n=10, ptr=0x1000):
    return [HelixTensor(ptr + 0x100 * i, 0) for i in range(n)]


def test_encode_errors(host):
    d = mp((128, 1, 2, 64, 128, 1))
    s0, x, dt, A, B, C, ids, y, s1, sc = _tensors()
    L = abi.lib()
    # null context / descriptor
    assert L.helix_scan_encode(None, None, ctypes.byref(d), s0, x, dt, A, B, C, ids, y, s1, sc) == HELIX_ERR_INVALID_ARG
    assert L.helix_scan_encode(host.handle, None, None, s0, x, dt, A, B, C, ids, y, s1, sc) == HELIX_ERR_INVALID_ARG
    # null required tensor
    assert host.encode(0, d, s0, x, HELIX_TENSOR_NULL, A, B, C, ids, y, s1, sc) == HELIX_ERR_INVALID_ARG
    assert "null tensor" in host.last_error()
    # unsupported shape
    bad = d.copy()
    bad.chunk = 32
    assert host.encode(0, bad, s0, x, dt, A, B, C, ids, y, s1, sc) == HELIX_ERR_UNSUPPORTED_SHAPE
    # host-only context: refuses before touching HIP
    assert host.encode(0, d, s0, x, dt, A, B, C, ids, y, s1, sc) == HELIX_ERR_NO_DEVICE
    assert host.encode(0, d, s0, x, dt, A, B, C, ids, y, s1, sc, into=True) == HELIX_ERR_NO_DEVICE
    assert "host-only" in host.last_error()


def test_last_error_is_per_thread(host):
    import threading
    d = mp((128, 1, 2, 64, 128, 1))
    d.chunk = 32
    t = _tensors()
    host.encode(0, d, *t)
    mine = host.last_error()
    seen = []
    th = threading.Thread(target=lambda: seen.append(host.last_error()))
    th.start()
    th.join()
    assert mine and seen == [""]


def test_ctx_create_reports_missing_device():
    # No GPU in this container: creation must fail cleanly with a message.
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is present")
    with pytest.raises(abi.HelixError) as e:
        abi.Context(0)
    assert e.value.status == HELIX_ERR_NO_DEVICE


# ---------------------------------------------------------------------------
# Kernel algebra on the CPU: the two-level scheme equals the recurrence
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("seg_len,cpg", [(1, None), (3, None), (4, 5), (2, 1), (16, None)])
@pytest.mark.parametrize("memory", ["short", "long"])
def test_two_level_algebra(seg_len, cpg, memory):
    p = po.problem_harness(700, 2, 4, 24, 16, 2, 4242, memory)
    p.ids = np.array([1, 0], np.int32)
    y, s1 = po.scan(p)
    ym, sm = two_level_scan(p.s0, p.x, p.dt, p.A, p.B, p.C, ids=p.ids, seg_len=seg_len,
                            chunks_per_group=cpg)
    assert po.allclose_ratio(ym, y, 1e-6, 1e-9) <= 1.0
    assert po.allclose_ratio(sm, s1, 1e-6, 1e-9) <= 1.0


def test_flop_and_byte_counts_match_baseline():
    # The reference's own FLOP and byte counts (bench_scan.mm:205-209).
    assert abs(algorithmic_flops(2048, 1, 64, 64, 128) / 1e9 - 5.931) < 1e-3
    assert abs(algorithmic_flops(8192, 1, 64, 64, 128) / 1e9 - 23.723) < 1e-3
    assert abs(algorithmic_bytes(8192, 1, 64, 64, 128, 8) / 1e6 - 341.8) < 0.1
    assert abs(algorithmic_flops(4096, 8, 80, 64, 128) / 1e9 - 118.615) < 1e-2
