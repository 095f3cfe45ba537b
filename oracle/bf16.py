"""bf16 / f16 bit-level helpers for the oracle (test infrastructure only).

The reference rounds with XLA ``astype(bfloat16)`` (round to nearest, ties to even) at fixed points:
prefill tiles (pallas_moe.py:350), prefill h/y (pallas_moe.py:682,747), the prefill combine weights
(resident.py:162-163) and the int8 dequant (quant8.py:94).  These helpers restate that rounding on raw bits so
the oracle does not depend on a bf16-capable numpy.
"""
import numpy as np


def f32_to_bf16_bits(a):
    """f32 array -> uint16 bf16 bits, round to nearest even (NaN kept quiet)."""
    a = np.ascontiguousarray(np.asarray(a, dtype=np.float32))
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    r = ((u + 0x7FFF + lsb) >> 16).astype(np.uint32)
    nan = np.isnan(a)
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint32), r)
    return r.astype(np.uint16)


def bf16_bits_to_f32(b):
    """uint16 bf16 bits -> f32 (exact)."""
    b = np.asarray(b, dtype=np.uint16)
    return (b.astype(np.uint32) << 16).view(np.float32)


def round_bf16(a):
    """f32/f64 array -> f32 array holding the bf16-rounded values (input first rounded to f32)."""
    return bf16_bits_to_f32(f32_to_bf16_bits(np.asarray(a, dtype=np.float32)))


def f16_bits_to_f32(h):
    """uint16/uint32 (low 16 bits) f16 bit patterns -> f32 (exact, IEEE incl. subnormals/inf/nan)."""
    h = (np.asarray(h).astype(np.uint32) & 0xFFFF).astype(np.uint16)
    return h.view(np.float16).astype(np.float32)


def rel_l2(a, b):
    """||a - b|| / ||b|| in f64."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))
