"""int8 per-channel projection oracle (test infrastructure only).

Reference: a quantized leaf is {"q": int8 [in, out], "s": f32 [1, out]} (quant8.py:17-18,26-32); every layer program
replaces it by W = bf16(f32(q) * s) (quant8.py:91-99) and the projection is x @ W with f32 accumulation, bf16 out.
A non-int8 leaf (the engine's default, int8_nonexpert=False, engine.py:281) is W itself, bf16 [in, out]; mlp_partial
takes either kind.
"""
import numpy as np

from .bf16 import round_bf16


def quantize_array(w, axis):
    """w [in, out] -> (q int8, s f32); axis 0 = per-row scales [in,1], 1 = per-column [1,out] (quant8.py:26-32)."""
    w32 = np.asarray(w, dtype=np.float32)
    amax = np.max(np.abs(w32), axis=1 - axis, keepdims=True)
    s = (np.maximum(amax, np.float32(1e-12)) / np.float32(127.0)).astype(np.float32)
    q = np.clip(np.round(w32 / s), -127, 127).astype(np.int8)
    return q, s


def generate(rng, n_in, n_out):
    """Benchmark inputs: q uniform in [-127, 127], s ~ U(0.5e-3, 2e-3) per output channel."""
    q = rng.integers(-127, 128, (n_in, n_out), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (1, n_out)).astype(np.float32)
    return q, s


def dequant_bf16(q, s):
    """bf16(f32(q) * s) as f32 values (quant8.py:94)."""
    return round_bf16(np.asarray(q, dtype=np.float32) * np.asarray(s, dtype=np.float32))


def project_f32(x, q, s):
    """x [B, in] (bf16 values) @ bf16(q*s) with f64 accumulation -> f32 [B, out] (before the bf16 output rounding)."""
    W = dequant_bf16(q, s).astype(np.float64)
    return (np.asarray(x, dtype=np.float64) @ W).astype(np.float32)


def project_bf16(x, q, s):
    """The projection's bf16 output, as f32 values."""
    return round_bf16(project_f32(x, q, s))


def project_after_f32(x, q, s):
    """The int8 lm_head (Engine._logits_local, engine.py:345-351): dot(x, f32(q)) with f64 accumulation rounded to
    f32, times s [1, out] in f32 -> f32 [B, out] (before the cast to x's dtype)."""
    z = (np.asarray(x, dtype=np.float64) @ np.asarray(q, dtype=np.float64)).astype(np.float32)
    return (z * np.asarray(s, dtype=np.float32)).astype(np.float32)


def project_w_f32(x, W):
    """x [B, in] (bf16 values) @ W [in, out] (bf16 values: the reference's non-int8 leaf, model.py:125-127) with f64
    accumulation -> f32 [B, out] (before the bf16 output rounding)."""
    return (np.asarray(x, dtype=np.float64) @ np.asarray(W, dtype=np.float64)).astype(np.float32)


def _project_leaf(x, leaf):
    return project_f32(x, *leaf) if isinstance(leaf, tuple) else project_w_f32(x, leaf)


def mlp_partial_f32(x, gate, up, down, limit, _drop=()):
    """mlp_partial (model.py:125-127) over int8 leaves gate, up, down = (q [in, out], s [1, out] or [in, 1]), as
    every layer program sees them after dequant_tree (quant8.py:91-99), or over bf16 leaves W [in, out] (arrays of
    bf16 values; int8_nonexpert off, engine.py:281): g = bf16(x @ Wg), u = bf16(x @ Wu) (bf16 matmuls with f32
    accumulation; f64 here), h = bf16(swiglu_clamped(g, u)) (one rounding of the SwiGLU evaluated in f64),
    y = h @ Wd -> f32 [B, D] before the output's bf16 rounding.  ``_drop`` ("g", "u", "h") skips a rounding:
    planted-mistake tests only."""
    from .moe import swiglu_clamped
    rnd = lambda name, a: np.asarray(a, dtype=np.float32) if name in _drop else round_bf16(a)
    g = rnd("g", _project_leaf(x, gate))
    u = rnd("u", _project_leaf(x, up))
    h = rnd("h", swiglu_clamped(g, u, limit).astype(np.float32))
    return _project_leaf(h, down)
