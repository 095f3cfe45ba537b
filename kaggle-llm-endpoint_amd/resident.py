"""The drop-in operator: a ``ResidentFetch`` with the reference's constructor and ``apply`` signature
(resident.py:68-108), backed by the HIP kernels of libmi355moe.so.

``moe_dense`` duck-types its ``fetch`` argument (model.py:847-848):
    y = fetch.apply(p, xf, idx, w, layer, cfg.swiglu_limit)
with ``p = {"gate_q" | "up_q" | "down_q": {plane: u32 [1 or none, E*rows_p, R]}, ...}`` and ``self.qtypes[layer]``
naming each table's format.  The same call works here with the planes held as torch int32 tensors on the GPU.

Everything runs on the current torch (HIP) stream; there is no CPU path.
"""
import ctypes
from typing import NamedTuple

import numpy as np
import torch

from . import _lib, formats
from ._lib import MiTable, check, lib

QK = 256


def _plane_rows(qtype, K):
    """IQ2_S / IQ3_S / IQ4_XS / Q2_K / Q3_K: rows_p per expert of each plane [E*rows_p, R] (planes.py:56-70)."""
    nblk = K // QK
    if qtype == "IQ2_S":
        W = 8 * nblk
        return {"qs": W, "sg": W, "qh": W // 4, "sc": W // 4, "d": (nblk + 1) // 2}
    if qtype == "IQ3_S":
        W = 16 * nblk
        return {"qs": W, "sg": W // 2, "qh": W // 8, "sc": W // 16, "d": (nblk + 1) // 2}
    if qtype == "IQ4_XS":
        return {"qs": 32 * nblk, "sl": nblk, "sh": nblk, "d": (nblk + 1) // 2}
    if qtype == "Q2_K":
        return {"qs": 16 * nblk, "sc": 4 * nblk, "d": nblk}
    if qtype == "Q3_K":
        return {"qs": 16 * nblk, "hm": 8 * nblk, "sc": 4 * nblk, "d": nblk}
    raise ValueError(qtype)                     # the reference raises ValueError on an unknown qtype (planes.py:70)


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _ptr(t):
    return ctypes.c_void_p(t.data_ptr()) if t is not None else None


def to_device_planes(planes, device="cuda"):
    """{plane: numpy u32 array} -> {plane: torch int32 tensor} on the device (bit-identical)."""
    return {k: torch.from_numpy(np.ascontiguousarray(v).view(np.int32)).to(device) for k, v in planes.items()}


class ExpertTable:
    """One matrix kind (gate, up or down) of E experts, R rows x K inputs each, as device planes."""

    def __init__(self, qtype, planes, rows, cols):
        if qtype not in _lib.QTYPES:
            raise ValueError("unsupported qtype %r" % (qtype,))
        self.qtype, self.rows, self.cols = qtype, int(rows), int(cols)
        keys = _lib.PLANE_KEYS[qtype]
        if qtype != "CB3" and (self.cols <= 0 or self.cols % QK):
            raise ValueError("%s tables need whole %d-weight blocks per row, got %d columns" % (qtype, QK, self.cols))
        self.planes = {}
        for k in keys:
            a = planes[k]
            if a.dtype not in (torch.int32, torch.uint32) or not a.is_cuda:
                raise ValueError("plane %r must be a 32-bit integer tensor on the GPU" % k)
        if qtype == "CB3":
            # tile planes (formats.cb3_pack_planes): [E, words] or flat, whole experts
            pw = formats.cb3_plane_words(self.rows, self.cols)
            if self.rows % 64:
                raise ValueError("CB3 tables need rows in multiples of 64, got %d" % self.rows)
            for k in keys:
                a = planes[k].contiguous().reshape(-1)
                if a.numel() % pw[k]:
                    raise ValueError("plane %r has %d words, not whole experts of %d" % (k, a.numel(), pw[k]))
                self.planes[k] = a
            self.n_experts = self.planes["qs"].numel() // pw["qs"]
            per = {k: pw[k] for k in keys}
        else:
            rp = _plane_rows(qtype, cols)
            for k in keys:
                a = planes[k]
                if a.dim() == 3:                       # the reference's leading chip axis [1, E*rows_p, R]
                    if a.shape[0] != 1:
                        raise ValueError("one device holds the full expert set: leading axis must be 1")
                    a = a[0]
                if a.shape[-1] != self.rows or a.shape[0] % rp[k]:
                    raise ValueError("plane %r has shape %s, expected [E*%d, %d]" % (k, tuple(a.shape), rp[k],
                                                                                     self.rows))
                self.planes[k] = a.contiguous()
            self.n_experts = self.planes["qs"].shape[0] // rp["qs"]
            per = {k: rp[k] * self.rows for k in keys}
        for k in keys:
            if self.planes[k].numel() != self.n_experts * per[k]:
                raise ValueError("plane %r does not hold %d experts" % (k, self.n_experts))
        self._c = MiTable()
        self._c.qtype = _lib.QTYPES[qtype]
        self._c.rows, self._c.cols, self._c.n_experts = self.rows, self.cols, self.n_experts
        for i, k in enumerate(keys):
            self._c.plane[i] = self.planes[k].data_ptr()

    @property
    def c(self):
        return ctypes.byref(self._c)

    def hbm_bytes_per_expert(self):
        return sum(int(a.numel()) * 4 for a in self.planes.values()) // self.n_experts


def random_cb3_table(E, R, K, generator, scale=0.02):
    """An ExpertTable of E random CB3 experts generated on the GPU in the kernel layout: uniform random code tiles
    (every bit pattern of a tile word is a valid set of codes; the zero-activation padding columns of the last tile
    multiply whatever codes they hold) and, per (group, row), 8 sorted N(0, scale) bf16 centroids.  For benchmarks
    and size-independent tests at full shape, where generating canonical codes on the host is too slow."""
    CT, G = (K + 159) // 160, K // 128
    qs = torch.randint(-2 ** 31, 2 ** 31 - 1, (E, CT * (R // 16) * 256), dtype=torch.int32, device="cuda",
                       generator=generator)
    sh = torch.tensor([0, 8, 16, 24], device="cuda", dtype=torch.int32)
    pack = lambda a: (a << sh).sum(-1).to(torch.int32)
    cbs = []
    for _ in range(E):
        c = torch.randn((G, R, 8), device="cuda", generator=generator) * scale
        c = torch.sort(c, dim=-1).values.to(torch.bfloat16).view(torch.int16).to(torch.int32) & 0xFFFF
        lo, hi = c & 0xFF, c >> 8
        cbs.append(torch.stack([pack(lo[..., 0:4]), pack(lo[..., 4:8]), pack(hi[..., 0:4]), pack(hi[..., 4:8])],
                               -1).reshape(1, G * R * 4))
    return ExpertTable("CB3", {"qs": qs, "cb": torch.cat(cbs, 0).contiguous()}, R, K)


def random_iq3s_table(E, R, K, generator, scale=0.02):
    """An ExpertTable of E random IQ3_S experts in the reference's planes, generated on the GPU: uniform random qs,
    sg, qh and sc words (every bit pattern is a valid set of grid indices, signs and scales) and per-block f16 d
    uniform in [scale / 2, scale] (as oracle.iq3s.random_blocks draws them).  For benchmarks at full shape."""
    rp = _plane_rows("IQ3_S", K)
    planes = {}
    for k in ("qs", "sg", "qh", "sc"):
        planes[k] = torch.randint(-2 ** 31, 2 ** 31 - 1, (E * rp[k], R), dtype=torch.int32, device="cuda",
                                  generator=generator)
    d = torch.rand((E * rp["d"], R, 2), device="cuda", generator=generator) * (0.5 * scale) + 0.5 * scale
    bits = d.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    planes["d"] = (bits[..., 0] | (bits[..., 1] << 16)).contiguous()
    return ExpertTable("IQ3_S", planes, R, K)


def random_iq2s_table(E, R, K, generator, scale=0.02):
    """An ExpertTable of E random IQ2_S experts in the reference's planes, generated on the GPU: uniform random qs,
    sg, qh and sc words (every bit pattern is a valid set of grid indices, signs and scales) and per-block f16 d
    uniform in [scale / 2, scale].  For benchmarks at full shape."""
    rp = _plane_rows("IQ2_S", K)
    planes = {}
    for k in ("qs", "sg", "qh", "sc"):
        planes[k] = torch.randint(-2 ** 31, 2 ** 31 - 1, (E * rp[k], R), dtype=torch.int32, device="cuda",
                                  generator=generator)
    d = torch.rand((E * rp["d"], R, 2), device="cuda", generator=generator) * (0.5 * scale) + 0.5 * scale
    bits = d.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    planes["d"] = (bits[..., 0] | (bits[..., 1] << 16)).contiguous()
    return ExpertTable("IQ2_S", planes, R, K)


def random_kq_table(qtype, E, R, K, generator, scale=0.02):
    """An ExpertTable of E random Q2_K or Q3_K experts in the reference's planes, generated on the GPU: uniform random
    qs (and hm) words, random scale bytes (Q3_K: six-bit), f16 d (and dmin) uniform in [scale / 2, scale]."""
    rp = _plane_rows(qtype, K)
    planes = {}
    for k in ("qs", "hm", "sc"):
        if k in rp:
            planes[k] = torch.randint(-2 ** 31, 2 ** 31 - 1, (E * rp[k], R), dtype=torch.int32, device="cuda",
                                      generator=generator)
    if qtype == "Q3_K":
        planes["sc"] &= 0x3F3F3F3F
    d = torch.rand((E * rp["d"], R, 2), device="cuda", generator=generator) * (0.5 * scale) + 0.5 * scale
    bits = d.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    planes["d"] = (bits[..., 0] | ((bits[..., 1] << 16) if qtype == "Q2_K" else 0)).contiguous()
    return ExpertTable(qtype, planes, R, K)


def random_iq4xs_table(E, R, K, generator, scale=0.02):
    """An ExpertTable of E random IQ4_XS experts in the reference's planes, generated on the GPU: uniform random qs, sl
    and sh words (every bit pattern is a valid set of indices and scales) and per-block f16 d uniform in
    [scale / 2, scale].  For benchmarks at full shape."""
    rp = _plane_rows("IQ4_XS", K)
    planes = {}
    for k in ("qs", "sl", "sh"):
        planes[k] = torch.randint(-2 ** 31, 2 ** 31 - 1, (E * rp[k], R), dtype=torch.int32, device="cuda",
                                  generator=generator)
    planes["sh"] &= 0xFFFF                     # 16 bits of high scale pairs per block (zero-extended)
    d = torch.rand((E * rp["d"], R, 2), device="cuda", generator=generator) * (0.5 * scale) + 0.5 * scale
    bits = d.to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    planes["d"] = (bits[..., 0] | (bits[..., 1] << 16)).contiguous()
    return ExpertTable("IQ4_XS", planes, R, K)


class _Workspaces:
    """Device workspaces, one per (device, stream, purpose); grown on demand.  They are zero-filled when allocated:
    the decode workspace's counter block must start at zero (each mi_moe_decode call leaves it zero again)."""

    def __init__(self):
        self._ws = {}

    def get(self, purpose, nbytes):
        dev = torch.cuda.current_device()
        key = (dev, torch.cuda.current_stream().cuda_stream, purpose)
        buf = self._ws.get(key)
        if buf is None or buf.numel() < nbytes:
            buf = torch.zeros(max(int(nbytes), 256), dtype=torch.uint8, device="cuda")
            self._ws[key] = buf
        return buf


WORKSPACES = _Workspaces()


class tuning:
    """Launch-plan overrides for tests and measurement runs (mi_tuning_set): ``with tuning(S1=3, CUMULTI=0): ...``
    sets them for the block and clears every override on exit (mi_tuning_reset).  The library reads no environment
    variables; calls outside such a block use the built-in plans.  Overrides change launch shapes (and with them
    workspace sizes and f32 summation orders), so workspaces are sized inside the block."""

    def __init__(self, **overrides):
        self.overrides = overrides

    def __enter__(self):
        lib().mi_tuning_reset()
        for name, value in self.overrides.items():
            check("mi_tuning_set(%s)" % name, lib().mi_tuning_set(name.encode(), int(value)))
        return self

    def __exit__(self, *exc):
        lib().mi_tuning_reset()
        return False


# ------------------------------------------------------------------------------------------------ kernel-level ops
def matvec(table, idx, X):
    """moe_matvec (pallas_moe.py:238-307): out[i, r] = sum_n W_{idx[i]}[r, n] X_i[n].
    idx int32 [n_slots]; X [n_slots, K] bf16 or f32 (natural input order) -> f32 [n_slots, R]."""
    n = int(idx.numel())
    out = torch.zeros((n, table.rows), dtype=torch.float32, device=X.device)      # rows of invalid ids stay 0
    return matvec_into(table, idx, X, out, None)


def pm_to_natural(qtype, X):
    """The reference's per-word activation matrix X [..., W, C] (X[w, c] = x[input(w, c)], planes.py:73-112) back in
    natural input order [..., W*C]: the inverse of pm_x's reshapes and transposes (a view for IQ2_S / IQ3_S, one
    transposing copy for IQ4_XS and the K-quants).  CB3, which has no reference layout, is in natural order."""
    lead = tuple(X.shape[:-2])
    n = X.shape[-2] * X.shape[-1]
    if qtype in ("IQ2_S", "IQ3_S", "CB3"):
        return X.reshape(lead + (n,))
    if qtype == "IQ4_XS":                       # [sub, wq, pos, j] -> [sub, pos, wq, j]
        return X.reshape(lead + (n // 32, 4, 2, 4)).transpose(-3, -2).reshape(lead + (n,))
    if qtype in ("Q2_K", "Q3_K"):               # [b, n, q, s, j] -> [b, n, s, q, j]
        return X.reshape(lead + (n // 256, 2, 8, 4, 4)).transpose(-3, -2).reshape(lead + (n,))
    raise ValueError(qtype)


def moe_matvec(planes, qtype, nblk, idx, X, *, interpret=False, lane_block=None):
    """moe_matvec (pallas_moe.py:238-307) with the reference's arguments: planes {plane: int32 [1 or none,
    E*rows_p, R]} in ``qtype``'s planar layout, nblk = K / 256, idx int32 [Nk], X [Nk, W, C] in the planar order
    (planes.py:96-112) -> f32 [Nk, R], out[i, r] = sum_n W_idx[i][r, n] x_i[n].  ``interpret`` and ``lane_block``
    are the Pallas call's own options and change nothing here.  Rows of ids outside [0, E) are zero."""
    R = int(planes["qs"].shape[-1])
    table = ExpertTable(qtype, planes, R, QK * int(nblk))
    if X.shape[0] != idx.numel():
        raise ValueError("X must hold one [W, C] matrix per slot")
    return matvec(table, idx, pm_to_natural(qtype, X))


def matvec_into(table, idx, X, out, workspace):
    """``matvec`` writing into ``out`` f32 [n_slots, R]; a preallocated ``workspace`` (uint8 device tensor of at
    least mi_matvec_workspace bytes) makes the call allocation-free."""
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    idx = idx.contiguous()
    n = int(idx.numel())
    if X.dim() != 2 or X.shape[0] != n or X.shape[1] != table.cols:
        raise ValueError("X must be [n_slots, K]")
    if X.dtype == torch.bfloat16:
        xd = _lib.MI_X_BF16
    elif X.dtype == torch.float32:
        xd = _lib.MI_X_F32
    else:
        raise ValueError("X must be bf16 or f32")
    X = X.contiguous()
    ws = workspace
    if ws is None:
        ws = WORKSPACES.get("matvec", lib().mi_matvec_workspace(table.c, n))
    check("mi_matvec", lib().mi_matvec(table.c, _ptr(idx), n, _ptr(X), xd, X.shape[1], _ptr(out), _ptr(ws),
                                       ws.numel(), _stream()))
    return out


def dequant(table, expert):
    """Exact f32 weights [R, K] of one expert (natural input order)."""
    out = torch.empty((table.rows, table.cols), dtype=torch.float32, device="cuda")
    check("mi_dequant", lib().mi_dequant(table.c, int(expert), _ptr(out), _stream()))
    return out


def decode_workspace_bytes(gate, down, N, k, shared_expert=-1):
    n = lib().mi_moe_decode_workspace(gate.c, down.c, int(N), int(k), int(shared_expert))
    if n == 0:
        raise ValueError("mi_moe_decode: invalid tables or token counts (N=%d, k=%d)" % (N, k))
    return n


def decode_plan(gate, down, N, k, shared_expert=-1):
    """The launch plan of mi_moe_decode (dict), without launching anything."""
    info = (ctypes.c_int32 * 27)()
    check("mi_moe_decode_plan", lib().mi_moe_decode_plan(gate.c, down.c, int(N), int(k), int(shared_expert), info, 27))
    keys = ("fused", "workgroups", "lists", "S1", "align1", "rtw1", "rbg1", "S2", "align2", "rtw2", "rbg2", "lds",
            "groups", "token_class", "err_word", "ctr_bytes", "sep_S1", "sep_rtw1", "sep_P1", "sep_S2", "sep_rtw2",
            "sep_P2", "sep_lds1", "sep_lds2", "sep_kind", "cu_combine", "reserved")
    return {key: int(info[i]) for i, key in enumerate(keys)}


def fused_error(workspace, gate, down):
    """The error word of mi_moe_decode_fused in ``workspace`` (synchronises the current stream): nonzero when a
    bounded wait of the last call on that workspace gave up, i.e. its results are invalid."""
    err = decode_plan(gate, down, 1, 1)["err_word"]
    torch.cuda.current_stream().synchronize()
    return int(workspace[4 * err:4 * err + 4].view(torch.int32).item())


def moe_decode(gate, up, down, x, idx, w, limit, shared_expert=-1, want_f32=True, want_bf16=False, out_f32=None,
               out_bf16=None, workspace=None, phases=3, fused=False, check_error=False):
    """Fused decode MoE (resident.py:110-120 composition), tokens grouped by expert on the device.
    x bf16 or f32 [N, D] (the layer dtype; f32 through mi_moe_decode_x); idx int32 [N, k]; w f32 [N, k] ->
    (out_f32 [N, D] or None, out_bf16 [N, D] or None).
    Preallocated ``out_f32`` / ``out_bf16`` / ``workspace`` (a uint8 device tensor of decode_workspace_bytes, kept
    for later calls) make the call allocation-free (graph capture).  ``fused=True`` runs the layer as one persistent
    launch (mi_moe_decode_fused: CB3, N <= 8); with ``check_error=True`` the call then synchronises and raises if a bounded
    wait of that launch gave up (results invalid; ``fused_error``).  ``phases`` 1 / 2 run part of the separate
    launches (mi_moe_decode_phases): 1 = the gate/up launch only, 2 = SwiGLU + down + combine only (after a phase-1
    call on the same workspace), 3 = all (mi_moe_decode)."""
    if x.dtype not in (torch.bfloat16, torch.float32):
        raise ValueError("decode activations are bf16 or f32")
    if x.dtype == torch.float32 and (fused or phases != 3):
        raise ValueError("f32 activations take the separate launches (phases=3, fused=False)")
    N, k = idx.shape
    x = x.contiguous()
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    if w.dtype != torch.float32:
        w = w.to(torch.float32)
    idx, w = idx.contiguous(), w.contiguous()
    D = down.rows
    of, ob = out_f32, out_bf16
    if phases & 2:
        if of is None and want_f32:
            of = torch.empty((N, D), dtype=torch.float32, device=x.device)
        if ob is None and want_bf16:
            ob = torch.empty((N, D), dtype=torch.bfloat16, device=x.device)
    ws = workspace
    if ws is None:
        ws = WORKSPACES.get("decode", decode_workspace_bytes(gate, down, N, k, shared_expert))
    if fused:
        check("mi_moe_decode_fused", lib().mi_moe_decode_fused(gate.c, up.c, down.c, _ptr(x), N, k, _ptr(idx),
                                                               _ptr(w), int(shared_expert), float(limit), _ptr(of),
                                                               _ptr(ob), _ptr(ws), ws.numel(), _stream()))
        if check_error and fused_error(ws, gate, down):
            raise RuntimeError("mi_moe_decode_fused: a bounded wait gave up (workgroups of the launch were not "
                               "resident together); the results of this call are invalid")
    elif x.dtype == torch.float32:
        check("mi_moe_decode_x", lib().mi_moe_decode_x(gate.c, up.c, down.c, _ptr(x), _lib.MI_X_F32, N, k, _ptr(idx),
                                                       _ptr(w), int(shared_expert), float(limit), _ptr(of), _ptr(ob),
                                                       _ptr(ws), ws.numel(), _stream()))
    elif phases == 3:
        check("mi_moe_decode", lib().mi_moe_decode(gate.c, up.c, down.c, _ptr(x), N, k, _ptr(idx), _ptr(w),
                                                   int(shared_expert), float(limit), _ptr(of), _ptr(ob), _ptr(ws),
                                                   ws.numel(), _stream()))
    else:
        check("mi_moe_decode_phases", lib().mi_moe_decode_phases(gate.c, up.c, down.c, _ptr(x), N, k, _ptr(idx),
                                                                 _ptr(w), int(shared_expert), float(limit), _ptr(of),
                                                                 _ptr(ob), _ptr(ws), ws.numel(), int(phases),
                                                                 _stream()))
    return of, ob


def ragged_plan(idx, w, E, tm):
    """ragged_plan (pallas_moe.py:564-592) on the device: idx int32 [T, k], w f32 [T, k] -> dict of device tensors
    blk_expert int32 [G], n_blocks int32 [1], tok_row int32 [Rp], w_row f32 [Rp], row_slot int32 [T, k] with
    G = ceil(T*k / tm) + E, Rp = G * tm (slots sorted stably by expert, every expert padded to whole blocks)."""
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    if w.dtype != torch.float32:
        w = w.to(torch.float32)
    idx, w = idx.contiguous(), w.contiguous()
    T, k = idx.shape
    G = -(-(T * k) // tm) + E
    dev = idx.device
    out = {"blk_expert": torch.empty(G, dtype=torch.int32, device=dev),
           "n_blocks": torch.empty(1, dtype=torch.int32, device=dev),
           "tok_row": torch.empty(G * tm, dtype=torch.int32, device=dev),
           "w_row": torch.empty(G * tm, dtype=torch.float32, device=dev),
           "row_slot": torch.empty((T, k), dtype=torch.int32, device=dev)}
    check("mi_ragged_plan", lib().mi_ragged_plan(_ptr(idx), _ptr(w), T, k, int(E), int(tm),
                                                 _ptr(out["blk_expert"]), _ptr(out["n_blocks"]),
                                                 _ptr(out["tok_row"]), _ptr(out["w_row"]), _ptr(out["row_slot"]),
                                                 _stream()))
    return out


def pack_planes_device(blocks, qtype, E, R, K):
    """GGUF blocks on the device (u8 tensor holding [E][R][K/256][block bytes], the expert tensor as stored) -> the
    reference's planes {plane: int32 [E * rows_p, R]} (planes.py:136-170), split on the device by mi_pack_planes."""
    if qtype not in ("IQ2_S", "IQ3_S", "IQ4_XS"):
        raise ValueError(qtype)
    bb = {"IQ2_S": 82, "IQ3_S": 110, "IQ4_XS": 136}[qtype]
    if blocks.dtype != torch.uint8 or blocks.numel() != E * R * (K // QK) * bb or K % QK:
        raise ValueError("pack_planes_device: %d bytes are not %d x %d %s weights" % (blocks.numel(), R, K, qtype))
    blocks = blocks.contiguous()
    rp = _plane_rows(qtype, K)
    keys = _lib.PLANE_KEYS[qtype]
    planes = {k: torch.empty((E * rp[k], R), dtype=torch.int32, device=blocks.device) for k in keys}
    arr = (ctypes.c_void_p * len(keys))(*[planes[k].data_ptr() for k in keys])
    check("mi_pack_planes", lib().mi_pack_planes(_lib.QTYPES[qtype], _ptr(blocks), int(E), int(R), int(K), arr,
                                                 _stream()))
    return planes


def route(x, router_w, bias, k, norm_topk=True, scaling=1.0, workspace=None):
    """The router (moe_route, model.py:798-808) on the device: x bf16 [N, D], router_w f32 [D, E], bias f32 [E] or
    None -> (idx int32 [N, k], w f32 [N, k]).  sigmoid scores, top-k of scores + bias (lower id first on equal
    values), weights = scores (renormalised over the k with ``norm_topk``) times ``scaling``."""
    if x.dtype != torch.bfloat16:
        x = x.to(torch.bfloat16)
    x = x.contiguous()
    router_w = router_w.to(torch.float32).contiguous()
    if bias is not None:
        bias = bias.to(torch.float32).contiguous()
    N, D = x.shape
    E = router_w.shape[1]
    if router_w.shape[0] != D or (bias is not None and tuple(bias.shape) != (E,)):
        raise ValueError("route: router_w must be [D, E] = [%d, E] and bias [E]" % D)
    need = lib().mi_moe_route_workspace(N, D, E)
    if workspace is None:
        workspace = torch.empty(max(need, 1), dtype=torch.uint8, device=x.device)
    idx = torch.empty((N, k), dtype=torch.int32, device=x.device)
    w = torch.empty((N, k), dtype=torch.float32, device=x.device)
    check("mi_moe_route", lib().mi_moe_route(_ptr(x), _ptr(router_w), _ptr(bias), N, D, E, int(k),
                                             1 if norm_topk else 0, float(scaling), _ptr(idx), _ptr(w),
                                             _ptr(workspace), workspace.numel(), _stream()))
    return idx, w


def moe_route(p, x, cfg):
    """The reference's moe_route(p, x, cfg) (model.py:798-808): p["router_w"] [D, E], p["router_bias"] [E];
    cfg.topk, cfg.norm_topk, cfg.scaling -> (idx int32 [N, k], w f32 [N, k])."""
    return route(x, p["router_w"], p.get("router_bias"), cfg.topk, cfg.norm_topk, cfg.scaling)


def prefill_workspace_bytes(gate, down, T, k, shared_expert=-1, combine="matmul"):
    n = lib().mi_moe_prefill_form_workspace(gate.c, down.c, int(T), int(k), int(shared_expert),
                                            _lib.PREFILL_FORMS[combine])
    if n == 0:
        raise ValueError("mi_moe_prefill: invalid tables or token counts (T=%d, k=%d)" % (T, k))
    return n


def moe_prefill(gate, up, down, x, idx, w, limit, shared_expert=-1, combine="matmul", want_f32=True,
                want_bf16=False, out_f32=None, out_bf16=None, workspace=None, chunk=8):
    """Grouped prefill MoE on the matrix cores, slots sorted by expert (ragged_plan), with the rounding points of
    one of the reference's bf16 branches:
      "matmul" / "gather": _apply_ragged_kernel (resident.py:144-165): h = bf16(swiglu(x Wg^T, x Wu^T)),
          y = bf16(h Wd^T), out = sum_j wt * y with wt = bf16(w) ("matmul") or w ("gather");
      "sweep": _apply_sweep_kernel (resident.py:169-187): hk = bf16(h * rw) with rw the token's summed weight of
          the expert, y = hk Wd^T in f32, out = f32 sum over the token's experts;
      "xla_gather": _apply_gather (resident.py:122-135): g, u rounded to bf16, then as "gather";
      "xla_sweep": _apply_sweep_xla (resident.py:189-210): g, u rounded to bf16, then as "sweep" except that the
          experts' y are summed per group of ``chunk`` expert ids, each group rounded to bf16 once.
    f32 accumulation throughout.  x bf16 [T, D]; idx int32 [T, k]; w f32 [T, k] -> (out_f32 [T, D] or None,
    out_bf16 [T, D] or None).  Preallocated outputs and ``workspace`` (uint8, prefill_workspace_bytes with the same
    ``combine``) make the call allocation-free."""
    if x.dtype != torch.bfloat16:
        raise ValueError("prefill activations are bf16")
    if combine not in _lib.PREFILL_FORMS:
        raise ValueError("combine must be one of %s" % ", ".join(sorted(_lib.PREFILL_FORMS)))
    if combine == "xla_sweep" and int(chunk) <= 0:
        raise ValueError("chunk must be positive")
    T, k = idx.shape
    x = x.contiguous()
    if idx.dtype != torch.int32:
        idx = idx.to(torch.int32)
    if w.dtype != torch.float32:
        w = w.to(torch.float32)
    idx, w = idx.contiguous(), w.contiguous()
    D = down.rows
    of, ob = out_f32, out_bf16
    if of is None and want_f32:
        of = torch.empty((T, D), dtype=torch.float32, device=x.device)
    if ob is None and want_bf16:
        ob = torch.empty((T, D), dtype=torch.bfloat16, device=x.device)
    ws = workspace
    if ws is None:
        ws = WORKSPACES.get("prefill", prefill_workspace_bytes(gate, down, T, k, shared_expert, combine))
    check("mi_moe_prefill_form", lib().mi_moe_prefill_form(gate.c, up.c, down.c, _ptr(x), T, k, _ptr(idx), _ptr(w),
                                                           int(shared_expert), float(limit),
                                                           _lib.PREFILL_FORMS[combine], int(chunk), _ptr(of),
                                                           _ptr(ob), _ptr(ws), ws.numel(), _stream()))
    return of, ob


def _scale_len(scale_axis, n_in, n_out):
    if scale_axis not in (_lib.MI_I8_ROW_SCALES, _lib.MI_I8_COL_SCALES, _lib.MI_I8_COL_AFTER):
        raise ValueError("scale_axis must be MI_I8_ROW_SCALES, MI_I8_COL_SCALES or MI_I8_COL_AFTER")
    return n_in if scale_axis == _lib.MI_I8_ROW_SCALES else n_out


def int8_tile(qT):
    """qT int8 [n_out, n_in] (device) -> the same weights in the tiled layout of mi_int8_tile, int8
    [n_in / 128, n_out / 16, 2048]: per 128-column block and 16-row tile the 2 KB the projection kernels load, 1 KB
    of contiguous memory per wavefront load.  The int8 entry points take either form (a 3-d weight is a tiled one)."""
    n_out, n_in = qT.shape
    if n_out % 16 or n_in % 256:
        raise ValueError("int8_tile: n_out must be a multiple of 16 and n_in of 256 (got %d x %d)" % (n_out, n_in))
    qT = qT.contiguous()
    out = torch.empty((n_in // 128, n_out // 16, 2048), dtype=torch.int8, device=qT.device)
    check("mi_int8_tile", lib().mi_int8_tile(_ptr(qT), n_out, n_in, _ptr(out), _stream()))
    return out


def _i8_dims(qT):
    """(n_out, n_in, layout bit) of a weight in either layout (3-d: tiled)."""
    if qT.dim() == 3:
        return qT.shape[1] * 16, qT.shape[0] * 128, _lib.MI_I8_TILED
    return qT.shape[0], qT.shape[1], 0


def int8_project(x, qT, s, want_f32=False, y_bf16=None, y_f32=None, workspace=None, scale_axis=_lib.MI_I8_COL_SCALES):
    """y = x @ bf16(f32(q) * s) (quant8.py:91-99): x bf16 [B, n_in], qT int8 [n_out, n_in], s f32 [n_out]
    (``scale_axis`` MI_I8_COL_SCALES, the reference's [1, out]) or [n_in] (MI_I8_ROW_SCALES, its [in, 1]);
    MI_I8_COL_AFTER: y = (x @ f32(q)) * s[o], the int8 lm_head (engine.py:345-351).
    Preallocated outputs / workspace make the call allocation-free.
    The workspace's first 256 KB are completion counters that must be zero before its first int8 call (a
    zero-filled allocation; every call leaves them zero again): a workspace left nonzero gives wrong sums, silently."""
    B, n_in = x.shape
    n_out, w_in, tiled = _i8_dims(qT)
    if w_in != n_in:
        raise ValueError("int8_project: x has %d columns, the weight %d" % (n_in, w_in))
    if s.numel() != _scale_len(scale_axis, n_in, n_out):
        raise ValueError("int8_project: %d scales for scale_axis %d" % (s.numel(), scale_axis))
    x = x.contiguous()
    yb = y_bf16 if y_bf16 is not None else torch.empty((B, n_out), dtype=torch.bfloat16, device=x.device)
    yf = y_f32 if y_f32 is not None else (
        torch.empty((B, n_out), dtype=torch.float32, device=x.device) if want_f32 else None)
    nbytes = lib().mi_int8_project_workspace(B, n_in, n_out, int(scale_axis))
    if nbytes == 0:
        raise ValueError("mi_int8_project: unsupported shape B=%d n_in=%d n_out=%d" % (B, n_in, n_out))
    ws = workspace if workspace is not None else WORKSPACES.get("int8", nbytes)
    check("mi_int8_project", lib().mi_int8_project(_ptr(x), B, _ptr(qT), _ptr(s), int(scale_axis) | tiled, n_in,
                                                   n_out, _ptr(yb), _ptr(yf), _ptr(ws), ws.numel(), _stream()))
    return (yb, yf) if want_f32 else yb


def int8_leaf(leaf, device="cuda"):
    """A reference int8 leaf {"q": int8 [in, out], "s": f32 [1, out] or [in, 1]} (quant8.py:17-18,26-32) -> the
    device operands (qT int8 [out, in], s f32 flat, scale_axis) of int8_project."""
    qT, s, axis = formats.int8_pack(leaf["q"], leaf["s"])
    return (torch.from_numpy(qT).to(device), torch.from_numpy(s).to(device),
            _lib.MI_I8_ROW_SCALES if axis == 0 else _lib.MI_I8_COL_SCALES)


def int8_logits(h, leaf, **kw):
    """The int8 lm_head (Engine._logits_local, engine.py:345-351): (h @ f32(q)) * s, then h's dtype (bf16)."""
    qT, s, axis = int8_leaf(leaf, h.device) if isinstance(leaf, dict) else leaf
    if axis != _lib.MI_I8_COL_SCALES:
        raise ValueError("the lm_head's scales are per output column [1, out]")
    return int8_project(h, qT, s, scale_axis=_lib.MI_I8_COL_AFTER, **kw)


def int8_project_many(x, projections, want_f32=False, outputs=None, workspace=None,
                      scale_axis=_lib.MI_I8_COL_SCALES):
    """Several projections of the same activations in one launch (Q, K, V of x; the shared expert's gate and up):
    projections = [(qT int8 [n_out_j, n_in], s f32), ...] (at most 8, one ``scale_axis`` for all) -> a list with,
    per projection, what ``int8_project`` returns.  ``outputs`` = [(y_bf16, y_f32 or None), ...] preallocated makes
    the call allocation-free.
    The workspace's first 256 KB are completion counters that must be zero before its first int8 call (a
    zero-filled allocation; every call leaves them zero again): a workspace left nonzero gives wrong sums, silently."""
    B, n_in = x.shape
    x = x.contiguous()
    n = len(projections)
    dims = [_i8_dims(qT) for qT, _ in projections]
    if len({d[2] for d in dims}) != 1:
        raise ValueError("int8_project_many: the projections of one launch share one weight layout")
    for (qT, s), (n_out, w_in, _) in zip(projections, dims):
        if w_in != n_in:
            raise ValueError("int8_project_many: x has %d columns, a weight %d" % (n_in, w_in))
        if s.numel() != _scale_len(scale_axis, n_in, n_out):
            raise ValueError("int8_project_many: %d scales for scale_axis %d" % (s.numel(), scale_axis))
    arr = (_lib.MiI8Proj * n)()
    outs = []
    for j, (qT, s) in enumerate(projections):
        n_out = dims[j][0]
        if outputs is not None:
            yb, yf = outputs[j]
        else:
            yb = torch.empty((B, n_out), dtype=torch.bfloat16, device=x.device)
            yf = torch.empty((B, n_out), dtype=torch.float32, device=x.device) if want_f32 else None
        arr[j] = _lib.MiI8Proj(qT.data_ptr(), s.data_ptr(), n_out, _ptr(yb), _ptr(yf))
        outs.append((yb, yf) if want_f32 else yb)
    n_outs = (ctypes.c_int32 * n)(*[int(d[0]) for d in dims])
    nbytes = lib().mi_int8_project_many_workspace(B, n_in, n_outs, n, int(scale_axis))
    if nbytes == 0:
        raise ValueError("mi_int8_project_many: unsupported shapes (B=%d, n_in=%d, n_proj=%d)" % (B, n_in, n))
    ws = workspace if workspace is not None else WORKSPACES.get("int8", nbytes)
    check("mi_int8_project_many", lib().mi_int8_project_many(_ptr(x), B, n_in, arr, n, int(scale_axis) | dims[0][2],
                                                             _ptr(ws), ws.numel(), _stream()))
    return outs


def int8_mlp(x, gate, up, down, limit, want_f32=False, y_bf16=None, y_f32=None, workspace=None):
    """mlp_partial over int8 leaves (model.py:125-127 with quant8.py:91-99): y = bf16(h @ Wd) with
    h = bf16(swiglu_clamped(bf16(x @ Wg), bf16(x @ Wu))), W = bf16(f32(q) * s).  x bf16 [B, D]; gate, up, down:
    reference leaves {"q", "s"} or int8_leaf triples (qT, s, scale_axis); gate and up share one scale form.
    -> y bf16 [B, D] (and y f32, the down projection before its rounding, with want_f32).  Tokens go 32 per call
    (mi_int8_mlp's limit); preallocated outputs / workspace make each call allocation-free.
    The workspace's first 256 KB are completion counters that must be zero before its first int8 call (a
    zero-filled allocation; every call leaves them zero again): a workspace left nonzero gives wrong sums, silently."""
    g, u, d = [int8_leaf(l, x.device) if isinstance(l, dict) else l for l in (gate, up, down)]
    if g[2] != u[2]:
        raise ValueError("int8_mlp: gate and up take one scale form")
    (I, gd, gt), (_, _, ut), (_, _, dt) = _i8_dims(g[0]), _i8_dims(u[0]), _i8_dims(d[0])
    if gt != ut:
        raise ValueError("int8_mlp: gate and up take one weight layout")
    B, D = x.shape
    x = x.contiguous()
    yb = y_bf16 if y_bf16 is not None else torch.empty((B, D), dtype=torch.bfloat16, device=x.device)
    yf = y_f32 if y_f32 is not None else (
        torch.empty((B, D), dtype=torch.float32, device=x.device) if want_f32 else None)
    for b0 in range(0, B, 32):
        n = min(32, B - b0)
        nbytes = lib().mi_int8_mlp_workspace(n, D, I, int(g[2]), int(d[2]))
        if nbytes == 0:
            raise ValueError("mi_int8_mlp: unsupported shape B=%d D=%d I=%d" % (n, D, I))
        ws = workspace if workspace is not None else WORKSPACES.get("int8", nbytes)
        check("mi_int8_mlp", lib().mi_int8_mlp(_ptr(x[b0:b0 + n]), n, D, I, _ptr(g[0]), _ptr(g[1]), _ptr(u[0]),
                                               _ptr(u[1]), int(g[2]) | gt, _ptr(d[0]), _ptr(d[1]), int(d[2]) | dt,
                                               float(limit), _ptr(yb[b0:b0 + n]),
                                               _ptr(yf[b0:b0 + n]) if yf is not None else None, _ptr(ws),
                                               ws.numel(), _stream()))
    return (yb, yf) if want_f32 else yb


class Bf16Leaf(NamedTuple):
    """A bf16 weight prepared for bf16_project / bf16_mlp: wT bf16 [n_out, n_in] on the device (the reference's
    W [in, out] transposed once)."""
    wT: torch.Tensor


def bf16_leaf(w, device="cuda"):
    """A reference bf16 leaf W [in, out] (x @ W, model.py:125-127; int8_nonexpert=False keeps the non-expert weights
    so, engine.py:281,305) -> Bf16Leaf.  Only torch.bfloat16 tensors: any other dtype would be a rounding the
    reference does not make."""
    if isinstance(w, Bf16Leaf):
        return w
    if not isinstance(w, torch.Tensor) or w.dtype != torch.bfloat16 or w.dim() != 2:
        raise TypeError("bf16_leaf expects a 2-d torch.bfloat16 tensor W [in, out]")
    return Bf16Leaf(w.to(device).t().contiguous())


def bf16_project(x, w, want_f32=False, y_bf16=None, y_f32=None, workspace=None):
    """y = x @ W (the reference's bf16 matmul: f32 accumulation, bf16 out): x bf16 [B, n_in]; w the reference's W
    bf16 [n_in, n_out] or a Bf16Leaf.  Returns y bf16 [B, n_out] (and y f32 with want_f32); 32 tokens per launch.
    The workspace's first 256 KB are completion counters that must be zero before its first call (a zero-filled
    allocation; every call leaves them zero again)."""
    wT = bf16_leaf(w, x.device).wT
    B, n_in = x.shape
    n_out, w_in = wT.shape
    if w_in != n_in:
        raise ValueError("bf16_project: x has %d columns, the weight %d rows" % (n_in, w_in))
    x = x.contiguous()
    yb = y_bf16 if y_bf16 is not None else torch.empty((B, n_out), dtype=torch.bfloat16, device=x.device)
    yf = y_f32 if y_f32 is not None else (
        torch.empty((B, n_out), dtype=torch.float32, device=x.device) if want_f32 else None)
    for b0 in range(0, B, 32):
        n = min(32, B - b0)
        nbytes = lib().mi_bf16_project_workspace(n, n_in, n_out)
        if nbytes == 0:
            raise ValueError("mi_bf16_project: unsupported shape B=%d n_in=%d n_out=%d" % (n, n_in, n_out))
        ws = workspace if workspace is not None else WORKSPACES.get("int8", nbytes)
        check("mi_bf16_project", lib().mi_bf16_project(_ptr(x[b0:b0 + n]), n, _ptr(wT), n_in, n_out,
                                                       _ptr(yb[b0:b0 + n]),
                                                       _ptr(yf[b0:b0 + n]) if yf is not None else None, _ptr(ws),
                                                       ws.numel(), _stream()))
    return (yb, yf) if want_f32 else yb


def bf16_mlp(x, gate, up, down, limit, want_f32=False, y_bf16=None, y_f32=None, workspace=None):
    """mlp_partial over bf16 leaves (model.py:125-127): y = bf16(h @ Wd) with h = bf16(swiglu_clamped(bf16(x @ Wg),
    bf16(x @ Wu))).  x bf16 [B, D]; gate, up: W bf16 [D, I], down: W bf16 [I, D] (reference leaves) or Bf16Leaf.
    -> y bf16 [B, D] (and y f32, the down projection before its rounding, with want_f32).  Tokens go 32 per call
    (mi_bf16_mlp's limit); preallocated outputs / workspace make each call allocation-free.
    The workspace's first 256 KB are completion counters that must be zero before its first call (a zero-filled
    allocation; every call leaves them zero again)."""
    g, u, d = [bf16_leaf(l, x.device).wT for l in (gate, up, down)]
    B, D = x.shape
    I = g.shape[0]
    if g.shape != (I, D) or u.shape != (I, D) or d.shape != (D, I):
        raise ValueError("bf16_mlp: gate/up must be [D, I] and down [I, D] with D = %d (got %s, %s, %s)"
                         % (D, tuple(g.shape[::-1]), tuple(u.shape[::-1]), tuple(d.shape[::-1])))
    x = x.contiguous()
    yb = y_bf16 if y_bf16 is not None else torch.empty((B, D), dtype=torch.bfloat16, device=x.device)
    yf = y_f32 if y_f32 is not None else (
        torch.empty((B, D), dtype=torch.float32, device=x.device) if want_f32 else None)
    for b0 in range(0, B, 32):
        n = min(32, B - b0)
        nbytes = lib().mi_bf16_mlp_workspace(n, D, I)
        if nbytes == 0:
            raise ValueError("mi_bf16_mlp: unsupported shape B=%d D=%d I=%d" % (n, D, I))
        ws = workspace if workspace is not None else WORKSPACES.get("int8", nbytes)
        check("mi_bf16_mlp", lib().mi_bf16_mlp(_ptr(x[b0:b0 + n]), n, D, I, _ptr(g), _ptr(u), _ptr(d), float(limit),
                                               _ptr(yb[b0:b0 + n]), _ptr(yf[b0:b0 + n]) if yf is not None else None,
                                               _ptr(ws), ws.numel(), _stream()))
    return (yb, yf) if want_f32 else yb


def mlp_partial(p, x, limit):
    """The reference's mlp_partial(p, x, cfg) (model.py:125-127) for p = {"gate", "up", "down"}: int8 leaves
    {"q", "s"} (quant8.py:17-18, int8_nonexpert on) or int8_leaf triples go to int8_mlp; bf16 leaves (W [in, out]
    torch.bfloat16, the engine's default, engine.py:281) or Bf16Leaf to bf16_mlp.  x bf16 [B, D] -> bf16 [B, D]
    (cfg.swiglu_limit passed as ``limit``)."""
    kinds = {"int8" if isinstance(p[k], (dict, tuple)) and not isinstance(p[k], Bf16Leaf) else "bf16"
             for k in ("gate", "up", "down")}
    if len(kinds) != 1:
        raise ValueError("mlp_partial: gate, up and down must be all int8 or all bf16 leaves")
    if kinds == {"int8"}:
        return int8_mlp(x, p["gate"], p["up"], p["down"], limit)
    return bf16_mlp(x, p["gate"], p["up"], p["down"], limit)


# ------------------------------------------------------------------------------------------------ the operator
def _is_f32(dtype):
    """out_dtype given as a torch dtype, a numpy/JAX dtype or its name: True for float32."""
    return dtype in (torch.float32, "float32", "f32") or str(dtype).endswith("float32")


def decode_chunked(gate, up, down, x, idx, w, limit, shared_expert=-1, out=None):
    """The decode composition (resident.py:110-120, f32 end to end) for any number of tokens: mi_moe_decode /
    mi_moe_decode_x over consecutive chunks of at most 16 tokens and 128 slots (tokens are independent, so the
    chunking does not change any result).  x bf16 or f32 [N, D] -> f32 [N, D]."""
    N, k = idx.shape
    if k > _lib.MI_MAX_SLOTS:
        raise NotImplementedError("top-%d routing exceeds the decode kernels' %d slots per call" % (k, _lib.MI_MAX_SLOTS))
    step = min(_lib.MAX_DECODE_TOKENS, _lib.MI_MAX_SLOTS // k)
    if out is None:
        out = torch.empty((N, down.rows), dtype=torch.float32, device=x.device)
    for c0 in range(0, N, step):
        c1 = min(N, c0 + step)
        moe_decode(gate, up, down, x[c0:c1], idx[c0:c1], w[c0:c1], limit, shared_expert=shared_expert,
                   out_f32=out[c0:c1])
    return out


class ResidentFetch:
    """Drop-in for glm53.resident.ResidentFetch (resident.py:68-108): same constructor, ``qtypes`` and ``apply``.

    apply(p, x, idx, w, layer, limit): x [N, D] (bf16 or f32); idx [N, k] int32 into E; w [N, k] f32 -> f32 [N, D]
    (routed experts only; the caller adds the shared expert, model.py:847-855).  The branches of the reference's
    apply (resident.py:100-108,137-143), each with that branch's rounding points:
      * N*k <= gather_max_rows, use_pallas: _apply_kernel -- the fused decode kernels, f32 end to end
        (resident.py:110-120), in chunks of <= 16 tokens / 128 slots;
      * N*k > gather_max_rows, use_pallas, sweep_mode "ragged": _apply_ragged_kernel -- the grouped prefill GEMMs with
        the bf16 rounding points and ``combine`` (resident.py:144-165);
      * N*k > gather_max_rows, use_pallas, sweep_mode "dense": _apply_sweep_kernel -- the grouped GEMMs with the
        dense sweep's rounding points (hk = bf16(h * rw), y f32; resident.py:169-187);
      * use_pallas=False: _apply_gather (N*k <= gather_max_rows, resident.py:122-135) and _apply_sweep_xla
        (resident.py:189-210, experts summed in groups of ``chunk``) -- the grouped GEMMs with those paths' bf16
        rounding points (g and u rounded to bf16);
      * out_dtype float32, any branch: every value stays f32 (test_resident_cpu.py:81,124), i.e. the decode
        composition in f32, taken by the decode kernels in chunks.
    Every prefill form decodes gate and up with one format (mixed formats raise NotImplementedError).
    ``interpret`` is accepted and has no effect."""

    def __init__(self, qtypes, D, ml, out_dtype=torch.bfloat16, gather_max_rows=64, chunk=8, use_pallas=True,
                 interpret=False, sweep_mode="ragged", tm=32, combine="matmul"):
        if sweep_mode not in ("ragged", "dense"):
            raise ValueError("sweep_mode must be 'ragged' or 'dense'")
        if combine not in _lib.COMBINES:
            raise ValueError("combine must be 'matmul' or 'gather'")
        self.qtypes = qtypes
        self.rows = {"gate_q": ml, "up_q": ml, "down_q": D}
        self.cols = {"gate_q": D, "up_q": D, "down_q": ml}
        self.nblk = {"gate_q": D // QK, "up_q": D // QK, "down_q": ml // QK}
        self.out_dtype = out_dtype
        self.gather_max_rows = gather_max_rows
        self.chunk = chunk
        self.use_pallas = use_pallas
        self.interpret = interpret
        self.sweep_mode = sweep_mode
        self.tm = tm
        self.combine = combine
        self._tables = {}

    def tables(self, p, layer):
        """ExpertTable views of p's planes (cached per layer and storage)."""
        key = (layer,) + tuple(p[k]["qs"].data_ptr() for k in ("gate_q", "up_q", "down_q"))
        t = self._tables.get(key)
        if t is None:
            t = tuple(ExpertTable(self.qtypes[layer][k], p[k], self.rows[k], self.cols[k])
                      for k in ("gate_q", "up_q", "down_q"))
            self._tables = {key: t}
        return t

    def branch(self, N, k):
        """The reference's branch for an [N, k] routing: "kernel", "gather", "ragged", "sweep" or "sweep_xla"."""
        if N * k <= self.gather_max_rows:
            return "kernel" if self.use_pallas else "gather"
        if not self.use_pallas:
            return "sweep_xla"
        return "ragged" if self.sweep_mode == "ragged" else "sweep"

    def apply(self, p, x, idx, w, layer, limit):
        gate, up, down = self.tables(p, layer)
        N, k = idx.shape
        br = self.branch(N, k)
        if x.dtype not in (torch.bfloat16, torch.float32):
            x = x.to(torch.float32)
        if br == "kernel" or _is_f32(self.out_dtype):
            return decode_chunked(gate, up, down, x, idx, w, limit)
        if gate.qtype != up.qtype:
            raise NotImplementedError("ResidentFetch.apply: the grouped GEMMs take one format for gate and up "
                                      "(moe_ragged_gateup / moe_sweep_gateup decode both with one qtype)")
        if br == "sweep_xla" and gate.n_experts % self.chunk:
            raise ValueError("ResidentFetch: %d experts are not whole chunks of %d (resident.py:192)" %
                             (gate.n_experts, self.chunk))
        form = {"ragged": self.combine, "sweep": "sweep", "gather": "xla_gather", "sweep_xla": "xla_sweep"}[br]
        out, _ = moe_prefill(gate, up, down, x.to(torch.bfloat16), idx, w, limit, combine=form, chunk=self.chunk)
        return out
