"""ctypes binding of the C ABI in include/mi355moe.h (the in-tree libmi355moe.so built by build.py).

Loading fails loudly when the library is missing: there is no CPU fallback anywhere in the package.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libmi355moe.so")

MI_OK = 0
MI_QT_CB3 = 1
MI_QT_IQ3_S = 2
MI_QT_IQ4_XS = 3
MI_QT_IQ2_S = 4
MI_QT_Q2_K = 5
MI_QT_Q3_K = 6
MI_X_BF16 = 0
MI_X_F32 = 1
MI_MAX_SLOTS = 128
MAX_DECODE_TOKENS = 16
MI_I8_ROW_SCALES = 0         # s [n_in]: the reference's per-row scales [in, 1]
MI_I8_COL_SCALES = 1         # s [n_out]: per-column scales [1, out]
MI_I8_COL_AFTER = 2          # s [n_out] applied after the dot (the int8 lm_head)
MI_I8_TILED = 0x100          # OR'ed into scale_axis: qT in the tiled layout of mi_int8_tile
MI_COMBINE_MATMUL = 0
MI_COMBINE_GATHER = 1
MI_COMBINE_SWEEP = 2         # the dense sweep's rounding points (sweep_mode="dense")
MI_COMBINE_XLA_GATHER = 3    # the XLA decode path's (use_pallas=False, N*k <= gather_max_rows)
MI_COMBINE_XLA_SWEEP = 4     # the XLA prefill path's (use_pallas=False), experts summed in chunks
COMBINES = {"matmul": MI_COMBINE_MATMUL, "gather": MI_COMBINE_GATHER}
PREFILL_FORMS = {"matmul": MI_COMBINE_MATMUL, "gather": MI_COMBINE_GATHER, "sweep": MI_COMBINE_SWEEP,
                 "xla_gather": MI_COMBINE_XLA_GATHER, "xla_sweep": MI_COMBINE_XLA_SWEEP}
PREFILL_TM = 80              # rows per block of mi_moe_prefill's own plan
NOALLOC_SCRATCH_BYTES = 64 << 20     # MI_NOALLOC_SCRATCH_BYTES: the static data region of mi_moe_decode_noalloc

QTYPES = {"CB3": MI_QT_CB3, "IQ3_S": MI_QT_IQ3_S, "IQ4_XS": MI_QT_IQ4_XS, "IQ2_S": MI_QT_IQ2_S, "Q2_K": MI_QT_Q2_K,
          "Q3_K": MI_QT_Q3_K}
PLANE_KEYS = {"CB3": ("qs", "cb"), "IQ3_S": ("qs", "sg", "qh", "sc", "d"), "IQ4_XS": ("qs", "sl", "sh", "d"),
              "IQ2_S": ("qs", "sg", "qh", "sc", "d"), "Q2_K": ("qs", "sc", "d"), "Q3_K": ("qs", "hm", "sc", "d")}

# every symbol the header declares (tests check the library exports them)
EXPORTS = ("mi_matvec", "mi_matvec_workspace", "mi_moe_decode", "mi_moe_decode_fused", "mi_moe_decode_phases",
           "mi_moe_decode_workspace", "mi_moe_decode_plan", "mi_moe_decode_noalloc", "mi_moe_decode_x",
           "mi_ragged_plan", "mi_moe_prefill", "mi_moe_prefill_workspace", "mi_moe_prefill_form",
           "mi_moe_prefill_form_workspace", "mi_dequant", "mi_int8_project", "mi_int8_project_workspace", "mi_int8_project_many",
           "mi_int8_project_many_workspace", "mi_int8_mlp", "mi_int8_mlp_workspace", "mi_moe_route", "mi_moe_route_workspace", "mi_pack_planes", "mi_int8_tile", "mi_bf16_project", "mi_bf16_project_workspace",
           "mi_bf16_mlp", "mi_bf16_mlp_workspace", "mi_tuning_set", "mi_tuning_reset",
           "mi_strerror",
           "mi_version")


class MiTable(ctypes.Structure):
    _fields_ = [("qtype", ctypes.c_int32), ("rows", ctypes.c_int32), ("cols", ctypes.c_int32),
                ("n_experts", ctypes.c_int32), ("plane", ctypes.c_void_p * 5)]


class MiI8Proj(ctypes.Structure):
    _fields_ = [("qT", ctypes.c_void_p), ("s", ctypes.c_void_p), ("n_out", ctypes.c_int32),
                ("y_bf16", ctypes.c_void_p), ("y_f32", ctypes.c_void_p)]


class MiError(RuntimeError):
    def __init__(self, fn, status, msg):
        super().__init__("%s failed: status %d (%s)" % (fn, status, msg))
        self.status = status


_LIB = None


def lib():
    """The loaded library (raises if it has not been built)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(LIB_PATH):
        raise RuntimeError("libmi355moe.so is not built: run `python kaggle-llm-endpoint_amd/build.py` "
                           "(or __graft_entry__.build()) first")
    L = ctypes.CDLL(LIB_PATH)
    P, I, Z, F = ctypes.c_void_p, ctypes.c_int32, ctypes.c_size_t, ctypes.c_float
    T = ctypes.POINTER(MiTable)
    sig = {
        "mi_matvec": (I, [T, P, I, P, I, I, P, P, Z, P]),
        "mi_matvec_workspace": (Z, [T, I]),
        "mi_moe_decode": (I, [T, T, T, P, I, I, P, P, I, F, P, P, P, Z, P]),
        "mi_moe_decode_fused": (I, [T, T, T, P, I, I, P, P, I, F, P, P, P, Z, P]),
        "mi_moe_decode_phases": (I, [T, T, T, P, I, I, P, P, I, F, P, P, P, Z, I, P]),
        "mi_moe_decode_workspace": (Z, [T, T, I, I, I]),
        "mi_moe_decode_noalloc": (I, [T, T, T, P, I, I, P, P, I, F, P, P, P]),
        "mi_moe_decode_x": (I, [T, T, T, P, I, I, I, P, P, I, F, P, P, P, Z, P]),
        "mi_moe_decode_plan": (I, [T, T, I, I, I, ctypes.POINTER(ctypes.c_int32), I]),
        "mi_ragged_plan": (I, [P, P, I, I, I, I, P, P, P, P, P, P]),
        "mi_moe_prefill": (I, [T, T, T, P, I, I, P, P, I, F, I, P, P, P, Z, P]),
        "mi_moe_prefill_workspace": (Z, [T, T, I, I, I]),
        "mi_moe_prefill_form": (I, [T, T, T, P, I, I, P, P, I, F, I, I, P, P, P, Z, P]),
        "mi_moe_prefill_form_workspace": (Z, [T, T, I, I, I, I]),
        "mi_int8_tile": (I, [P, I, I, P, P]),
        "mi_int8_mlp": (I, [P, I, I, I, P, P, P, P, I, P, P, I, F, P, P, P, Z, P]),
        "mi_int8_mlp_workspace": (Z, [I, I, I, I, I]),
        "mi_dequant": (I, [T, I, P, P]),
        "mi_int8_project": (I, [P, I, P, P, I, I, I, P, P, P, Z, P]),
        "mi_int8_project_workspace": (Z, [I, I, I, I]),
        "mi_int8_project_many": (I, [P, I, I, ctypes.POINTER(MiI8Proj), I, I, P, Z, P]),
        "mi_int8_project_many_workspace": (Z, [I, I, ctypes.POINTER(ctypes.c_int32), I, I]),
        "mi_bf16_project": (I, [P, I, P, I, I, P, P, P, Z, P]),
        "mi_bf16_project_workspace": (Z, [I, I, I]),
        "mi_bf16_mlp": (I, [P, I, I, I, P, P, P, F, P, P, P, Z, P]),
        "mi_bf16_mlp_workspace": (Z, [I, I, I]),
        "mi_moe_route": (I, [P, P, P, I, I, I, I, I, F, P, P, P, Z, P]),
        "mi_moe_route_workspace": (Z, [I, I, I]),
        "mi_pack_planes": (I, [I, P, I, I, I, ctypes.POINTER(ctypes.c_void_p), P]),
        "mi_tuning_set": (I, [ctypes.c_char_p, I]),
        "mi_tuning_reset": (None, []),
        "mi_strerror": (ctypes.c_char_p, [I]),
        "mi_version": (I, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = L
    return L


PROBE_PATH = os.path.join(HERE, "libmi355probe.so")
_PROBE = None


def probe_lib():
    """The streaming-read probe (libmi355probe.so: measurement only, not part of the operator's C ABI):
    mi_read_probe(src, bytes, sink, workgroups, stream) reads `bytes` (a multiple of 16) from src with 16-byte loads
    in a grid-stride loop of `workgroups` 256-thread workgroups and writes one XOR word per wavefront to sink
    (workgroups * 4 u32)."""
    global _PROBE
    if _PROBE is None:
        if not os.path.exists(PROBE_PATH):
            raise RuntimeError("libmi355probe.so is not built: run `python kaggle-llm-endpoint_amd/build.py`")
        L = ctypes.CDLL(PROBE_PATH)
        L.mi_read_probe.restype = ctypes.c_int32
        L.mi_read_probe.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p, ctypes.c_int32,
                                    ctypes.c_void_p]
        _PROBE = L
    return _PROBE


def check(fn, status):
    if status != MI_OK:
        raise MiError(fn, status, lib().mi_strerror(status).decode())
