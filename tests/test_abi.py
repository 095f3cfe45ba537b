"""CPU: the C-ABI library loads, exports every entry point include/mi355moe.h declares, and rejects bad arguments on
the host before any launch (no GPU needed: every call here returns before touching a device)."""
import ctypes
import os
import re
import subprocess
import sys

import numpy as np
import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(REPO, "include", "mi355moe.h")


@pytest.fixture(scope="module")
def L(pkg):
    if not os.path.exists(pkg._lib.LIB_PATH):
        subprocess.run([sys.executable, os.path.join(REPO, "kaggle-llm-endpoint_amd", "build.py")], check=True)
    return pkg._lib.lib()


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_binding(pkg):
    assert declared() == sorted(pkg._lib.EXPORTS)


def test_library_exports_every_declared_symbol(L):
    for name in declared():
        assert hasattr(L, name), name
    out = subprocess.run(["nm", "-D", "--defined-only", L._name], capture_output=True, text=True).stdout
    syms = set(re.findall(r"\bT (mi_[a-z0-9_]+)$", out, flags=re.M))
    assert set(declared()) <= syms


def test_status_strings_and_version(L, pkg):
    assert L.mi_version() >= 1
    for code in range(0, 9):
        assert L.mi_strerror(code)
    assert b"unknown" in L.mi_strerror(99)


def _table(pkg, qtype=1, rows=256, cols=1280, E=4, planes=2):
    t = pkg._lib.MiTable()
    t.qtype, t.rows, t.cols, t.n_experts = qtype, rows, cols, E
    for i in range(planes):
        t.plane[i] = 0x1000 * (i + 1)            # never dereferenced: validation fails before any launch
    return t


def test_host_validation_codes(L, pkg):
    lib = pkg._lib
    P = ctypes.c_void_p
    x, idx, w, out, ws = P(0x10000), P(0x20000), P(0x30000), P(0x40000), P(0x50000)
    g, u, d = _table(pkg, rows=256, cols=1280), _table(pkg, rows=256, cols=1280), _table(pkg, rows=1280, cols=256)
    call = lambda gg, uu, dd, N=1, k=2, shared=-1, limit=10.0, o=out: L.mi_moe_decode(
        ctypes.byref(gg), ctypes.byref(uu), ctypes.byref(dd), x, N, k, idx, w, shared, ctypes.c_float(limit),
        o, None, ws, 1 << 30, None)
    assert call(_table(pkg, qtype=9), u, d) == 2                                   # MI_ERR_QTYPE
    assert call(_table(pkg, rows=100), u, d) == 3                                  # MI_ERR_SHAPE (rows % 64)
    assert call(_table(pkg, cols=1000), u, d) == 3                                 # MI_ERR_SHAPE (cols % 128)
    assert call(_table(pkg, planes=1), u, d) == 1                                  # MI_ERR_NULL (codebook plane)
    assert call(g, _table(pkg, rows=512, cols=1280), d) == 6                       # MI_ERR_MISMATCH (up shape)
    assert call(g, u, _table(pkg, rows=1280, cols=512)) == 6                       # MI_ERR_MISMATCH (down.cols)
    assert call(g, u, d, N=0) == 4 and call(g, u, d, N=17) == 4                    # MI_ERR_TOKENS
    assert call(g, u, d, N=16, k=9) == 4                                           # N*k > MI_MAX_SLOTS
    assert call(g, u, d, shared=4) == 8 and call(g, u, d, limit=0.0) == 8          # MI_ERR_ARG
    assert call(g, u, d, o=None) == 1                                              # MI_ERR_NULL (no output)
    assert L.mi_matvec(ctypes.byref(g), idx, 0, x, lib.MI_X_BF16, 1280, out, ws, 1 << 30, None) == 4
    assert L.mi_matvec(ctypes.byref(g), idx, 4, x, 7, 1280, out, ws, 1 << 30, None) == 8
    assert L.mi_matvec(ctypes.byref(g), idx, 4, x, lib.MI_X_BF16, 1000, out, ws, 1 << 30, None) == 8
    assert L.mi_dequant(ctypes.byref(g), 4, out, None) == 8                        # expert out of range
    assert L.mi_int8_project(x, 0, P(1), P(2), 1, 256, 64, out, None, ws, 1 << 20, None) == 4
    assert L.mi_int8_project(x, 8, P(1), P(2), 1, 300, 64, out, None, ws, 1 << 20, None) == 3
    assert L.mi_int8_project(x, 8, P(1), P(2), 1, 256, 40, out, None, ws, 1 << 20, None) == 3
    assert L.mi_int8_project(x, 8, P(1), P(2), 1, 256, 64, None, None, ws, 1 << 20, None) == 1
    assert L.mi_int8_project_workspace(8, 6144, 6144, 1) > 0
    assert L.mi_int8_project_workspace(8, 300, 64, 1) == 0
    assert L.mi_int8_project(x, 8, P(1), P(2), 3, 256, 64, out, None, ws, 1 << 20, None) == 8   # int8 forms only
    assert L.mi_bf16_project(x, 0, P(0x1000), 256, 64, out, None, ws, 1 << 20, None) == 4
    assert L.mi_bf16_project(x, 8, P(0x1000), 300, 64, out, None, ws, 1 << 20, None) == 3
    assert L.mi_bf16_project(x, 8, P(0x1000), 256, 40, out, None, ws, 1 << 20, None) == 3
    assert L.mi_bf16_project(x, 8, P(0x1002), 256, 64, out, None, ws, 1 << 20, None) == 8     # 16-byte aligned
    assert L.mi_bf16_project(x, 8, None, 256, 64, out, None, ws, 1 << 20, None) == 1
    assert L.mi_bf16_project(x, 8, P(0x1000), 256, 64, None, None, ws, 1 << 20, None) == 1
    assert L.mi_bf16_project(x, 8, P(0x1000), 6144, 2048, out, None, ws, 16, None) == 5         # workspace
    assert L.mi_bf16_project_workspace(8, 6144, 2048) > 0 and L.mi_bf16_project_workspace(33, 6144, 2048) == 0
    mlp = lambda B=4, D=512, I=256, limit=7.0, g=P(0x1000), wsb=1 << 30: L.mi_bf16_mlp(
        x, B, D, I, g, P(0x2000), P(0x3000), ctypes.c_float(limit), out, None, P(0x100000), wsb, None)
    assert mlp(B=0) == 4 and mlp(B=33) == 4                                        # MI_ERR_TOKENS
    assert mlp(D=640) == 3 and mlp(I=300) == 3                                     # MI_ERR_SHAPE
    assert mlp(limit=0.0) == 8 and mlp(g=P(0x1008)) == 8                           # MI_ERR_ARG
    assert mlp(g=None) == 1 and mlp(wsb=16) == 5
    assert L.mi_bf16_mlp_workspace(8, 6144, 2048) > 0 and L.mi_bf16_mlp_workspace(8, 6144, 2000) == 0


def test_prefill_host_validation(L, pkg):
    P = ctypes.c_void_p
    x, idx, w, out, ws = P(0x10000), P(0x20000), P(0x30000), P(0x40000), P(0x50000)
    g, u, d = _table(pkg, rows=256, cols=1280), _table(pkg, rows=256, cols=1280), _table(pkg, rows=1280, cols=256)
    call = lambda gg, uu, dd, T=4, k=2, shared=-1, limit=10.0, comb=0, o=out, wsb=1 << 30: L.mi_moe_prefill(
        ctypes.byref(gg), ctypes.byref(uu), ctypes.byref(dd), x, T, k, idx, w, shared, ctypes.c_float(limit), comb,
        o, None, ws, wsb, None)
    assert call(_table(pkg, qtype=9), u, d) == 2                                 # MI_ERR_QTYPE
    assert call(_table(pkg, qtype=2, planes=5), u, d) == 6                       # one format for all three tables
    iq = lambda rows, cols, planes=5: _table(pkg, qtype=2, rows=rows, cols=cols, planes=planes)
    gi, ui, di = iq(256, 1280), iq(256, 1280), iq(1280, 256)
    assert call(gi, ui, di, wsb=16) == 5                                         # IQ3_S tables pass validation
    assert call(iq(256, 640), iq(256, 640), iq(1280, 256)) == 3                  # IQ3_S: whole 256-weight blocks
    assert call(gi, ui, iq(1280, 256, planes=4)) == 1                            # IQ3_S: five planes
    assert call(_table(pkg, rows=192), _table(pkg, rows=192), d) == 3             # gate rows % 128
    assert call(g, u, _table(pkg, rows=1152, cols=256)) == 3                     # down rows % 256
    assert call(g, u, _table(pkg, rows=1280, cols=512)) == 6                     # down.cols != gate.rows
    assert call(g, u, d, T=0) == 4 and call(g, u, d, k=0) == 4                   # MI_ERR_TOKENS
    assert call(g, u, d, T=1 << 22, k=8) == 4                                    # past the slot / byte limits
    assert call(g, u, d, shared=4) == 8 and call(g, u, d, comb=2) == 8           # MI_ERR_ARG
    assert call(g, u, d, limit=-1.0) == 8
    assert call(g, u, d, o=None) == 1                                            # no output
    assert call(g, u, d, wsb=16) == 5                                            # MI_ERR_WORKSPACE
    assert L.mi_moe_prefill_workspace(ctypes.byref(g), ctypes.byref(d), 512, 8, 3) > 0
    assert L.mi_moe_prefill_workspace(ctypes.byref(g), ctypes.byref(d), 0, 8, -1) == 0
    form = lambda comb, chunk=8, wsb=1 << 30: L.mi_moe_prefill_form(
        ctypes.byref(g), ctypes.byref(u), ctypes.byref(d), x, 4, 2, idx, w, -1, ctypes.c_float(10.0), comb, chunk,
        out, None, ws, wsb, None)
    assert form(5) == 8 and form(-1) == 8 and form(4, chunk=0) == 8            # unknown form; XLA sweep chunk > 0
    assert form(2, wsb=16) == 5 and form(4, chunk=3, wsb=16) == 5              # the sweeps pass validation
    fws = lambda comb: L.mi_moe_prefill_form_workspace(ctypes.byref(g), ctypes.byref(d), 512, 8, 3, comb)
    assert fws(0) == fws(1) == fws(3) == L.mi_moe_prefill_workspace(ctypes.byref(g), ctypes.byref(d), 512, 8, 3)
    assert fws(2) == fws(4) > fws(0) and fws(5) == 0                             # the sweeps' y is f32
    outs =[P(0x60000 + 0x1000 * i) for i in range(5)]
    plan = lambda T=4, k=2, E=8, tm=32, i=idx: L.mi_ragged_plan(i, w, T, k, E, tm, *outs, None)
    assert plan(E=0) == 8 and plan(E=1025) == 8 and plan(tm=0) == 8              # MI_ERR_ARG
    assert plan(T=0) == 4 and plan(T=1 << 21, k=4) == 4                          # MI_ERR_TOKENS
    assert plan(i=None) == 1                                                     # MI_ERR_NULL


def test_route_host_validation(L):
    """mi_moe_route rejects bad shapes and arguments before any launch (fake, aligned device pointers)."""
    P = ctypes.c_void_p
    x, rw, idx, w, ws = P(0x1000), P(0x2000), P(0x3000), P(0x4000), P(0x5000)
    need = L.mi_moe_route_workspace(4, 6144, 64)
    assert need == 24 * 4 * 64 * 4                              # 256-column chunks x N x E floats

    def call(N=4, D=6144, E=64, k=8, norm=1, x_=x, ws_bytes=need, idx_=idx):
        return L.mi_moe_route(x_, rw, None, N, D, E, k, norm, 2.5, idx_, w, ws, ws_bytes, None)

    assert call(x_=None) == 1                                    # MI_ERR_NULL
    assert call(idx_=None) == 1
    assert call(N=0) == 4                                        # MI_ERR_TOKENS
    assert call(D=6143) == 3                                     # MI_ERR_SHAPE: odd D
    assert call(E=1025) == 3
    assert call(k=0) == 8 and call(k=65, E=64) == 8 and call(k=33, E=256) == 8   # MI_ERR_ARG
    assert call(norm=2) == 8
    assert call(x_=P(0x1002)) == 8                               # rows read as bf16 pairs: 4-byte alignment
    assert call(ws_bytes=need - 1) == 5                          # MI_ERR_WORKSPACE
    assert L.mi_moe_route_workspace(0, 6144, 64) == 0


def test_expert_table_rejects_partial_blocks(pkg):
    import torch
    with pytest.raises(ValueError, match="whole 256-weight blocks"):
        pkg.ExpertTable("Q2_K", {k: torch.zeros(4, 64, dtype=torch.int32) for k in ("qs", "sc", "d")}, 64, 128)


def test_python_wrappers_reject_bad_arguments(pkg):
    """The host side of the new entry points raises before any device work."""
    import torch
    with pytest.raises(ValueError):
        pkg.pack_planes_device(torch.zeros(10, dtype=torch.uint8), "Q2_K", 1, 64, 256)      # K-quants: host packer
    with pytest.raises(ValueError, match="bytes are not"):
        pkg.pack_planes_device(torch.zeros(10, dtype=torch.uint8), "IQ2_S", 1, 64, 256)
    with pytest.raises(ValueError, match="router_w must be"):
        pkg.route(torch.zeros(2, 64, dtype=torch.bfloat16), torch.zeros(32, 8), None, 2)
    with pytest.raises(ValueError):
        pkg.formats.kq_pack_planes(np.zeros((1, 4, 1, 83), np.uint8), "Q2_K")


def test_noalloc_rejects_a_layer_beyond_the_scratch(L, pkg):
    """mi_moe_decode_noalloc returns MI_ERR_WORKSPACE, before any launch, for a layer whose data region exceeds
    MI_NOALLOC_SCRATCH_BYTES (D = 262144: the down partials alone do).  Run here, on the CPU, the fabricated
    pointers can never be dereferenced by a kernel whatever the order of the entry point's checks."""
    lib = pkg._lib
    tabs = []
    for R, K in ((256, 262144), (256, 262144), (262144, 256)):
        t = lib.MiTable()
        t.qtype, t.rows, t.cols, t.n_experts = lib.MI_QT_CB3, R, K, 4
        t.plane[0], t.plane[1] = 0x1000, 0x2000
        tabs.append(t)
    P = ctypes.c_void_p
    assert L.mi_moe_decode_workspace(ctypes.byref(tabs[0]), ctypes.byref(tabs[2]), 16, 4, -1) > \
        lib.NOALLOC_SCRATCH_BYTES
    st = L.mi_moe_decode_noalloc(ctypes.byref(tabs[0]), ctypes.byref(tabs[1]), ctypes.byref(tabs[2]), P(0x10000),
                                 16, 4, P(0x20000), P(0x30000), -1, 10.0, P(0x40000), None, None)
    assert st == 5                                      # MI_ERR_WORKSPACE
