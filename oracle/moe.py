"""MoE operator oracle: decode and prefill compositions of the reference (test infrastructure only).

Weights are supplied lazily: ``deq(name, e) -> f32 [R, K]`` returns the exactly dequantized matrix ``name`` in
{"gate", "up", "down"} of expert ``e`` (natural input order), so full-size layers dequantize only what is routed.
"""
import numpy as np

from .bf16 import round_bf16


def silu(z):
    """z * sigmoid(z) (model.py:114-115), evaluated in f64 (exp(-z) overflowing to inf for very negative z gives the
    correct limit -0)."""
    z = np.asarray(z, dtype=np.float64)
    with np.errstate(over="ignore"):
        return z / (1.0 + np.exp(-z))


def swiglu_clamped(g, u, limit):
    """silu(min(g, L)) * clip(u, -L, L) (model.py:119-122)."""
    g = np.minimum(np.asarray(g, dtype=np.float64), limit)
    u = np.clip(np.asarray(u, dtype=np.float64), -limit, limit)
    return silu(g) * u


def matvec_f64(W, x):
    """W [R, K] (f32 values), x [n, K] -> f64 [n, R]."""
    return np.asarray(x, dtype=np.float64) @ np.asarray(W, dtype=np.float64).T


def decode_apply(deq, x, idx, w, limit):
    """The fused decode composition ResidentFetch._apply_kernel (resident.py:110-120) in f64:
    per slot i = (n, j): g = Wg[e] x_n, u = Wu[e] x_n (pallas_moe.py:238-307 == moe_matvec_ref :310-323),
    h = swiglu_clamped(g, u, L) (resident.py:118), y = Wd[e] h (resident.py:119), out[n] = sum_j w[n,j] y
    (resident.py:120).  x is upcast to f32 first (resident.py:114).  Returns f64 [N, D] (routed experts only).
    Experts are visited once each (grouped) -- the result is the same as the per-slot reference."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    idx = np.asarray(idx)
    w = np.asarray(w, dtype=np.float64)
    N, k = idx.shape
    out = None
    for e in np.unique(idx):
        rows = np.argwhere(idx == e)                           # [(n, j)]
        xs = x[rows[:, 0]]
        g = matvec_f64(deq("gate", int(e)), xs)
        u = matvec_f64(deq("up", int(e)), xs)
        h = swiglu_clamped(g, u, limit)
        y = matvec_f64(deq("down", int(e)), h)                 # [n_rows, D]
        if out is None:
            out = np.zeros((N, y.shape[1]), np.float64)
        for r, (n, j) in enumerate(rows):
            out[n] += w[n, j] * y[r]
    return out


def shared_apply(deq_shared, x, limit):
    """A 3-bit shared expert applied to every token (the benchmark layer adds it to the routed sum): f64 [N, D]."""
    x = np.asarray(x, dtype=np.float32).astype(np.float64)
    g = matvec_f64(deq_shared("gate"), x)
    u = matvec_f64(deq_shared("up"), x)
    return matvec_f64(deq_shared("down"), swiglu_clamped(g, u, limit))


# ------------------------------------------------------------------------------------------------ prefill
def route(x, router_w, bias, k, norm_topk=True, scaling=1.0):
    """Restates moe_route (model.py:798-808) in f64: logits = x @ router_w ([N, D] @ [D, E]), scores = sigmoid,
    idx = top_k(scores + bias, k) with lax.top_k's order (larger first, equal values: lower index first, here a
    stable sort), w = scores[idx], renormalised over the k (+1e-20) with norm_topk, times scaling.
    -> (idx int32 [N, k], w f64 [N, k], choice f64 [N, E])."""
    logits = np.asarray(x, np.float64) @ np.asarray(router_w, np.float64)
    scores = 1.0 / (1.0 + np.exp(-logits))
    choice = scores + (0.0 if bias is None else np.asarray(bias, np.float64))
    order = np.argsort(-choice, axis=-1, kind="stable")[:, :k]
    w = np.take_along_axis(scores, order, -1)
    if norm_topk:
        w = w / (w.sum(-1, keepdims=True) + 1e-20)
    return order.astype(np.int32), w * scaling, choice


def ragged_plan(idx, w, E, tm):
    """Restates pallas_moe.ragged_plan (pallas_moe.py:564-592) in numpy.  idx int [T, k], w f32 [T, k] ->
    dict(blk_expert int32 [G], n_blocks int32 [1], tok_row int32 [Rp] (-1 pad), w_row f32 [Rp],
    row_slot int32 [T, k]); G = ceil(T*k / tm) + E, Rp = G * tm."""
    idx = np.asarray(idx)
    T, k = idx.shape
    S = T * k
    G = -(-S // tm) + E
    Rp = G * tm
    flat = idx.reshape(-1).astype(np.int64)
    order = np.argsort(flat, kind="stable")
    se = flat[order]
    counts = np.bincount(flat, minlength=E)[:E]
    padded = -(-counts // tm) * tm
    pstart = np.cumsum(padded) - padded
    ustart = np.cumsum(counts) - counts
    row_sorted = pstart[se] + (np.arange(S) - ustart[se])
    tok_row = np.full((Rp,), -1, np.int32)
    tok_row[row_sorted] = (order // k).astype(np.int32)
    w_row = np.zeros((Rp,), np.float32)
    w_row[row_sorted] = np.asarray(w, dtype=np.float32).reshape(-1)[order]
    row_slot = np.zeros((S,), np.int32)
    row_slot[order] = row_sorted
    nb = padded // tm
    bstart = np.cumsum(nb) - nb
    n_blocks = int(nb.sum())
    g = np.arange(G)
    be = (g[:, None] >= (bstart + nb)[None, :]).sum(1)
    be = np.minimum(be, E - 1)
    last = be[max(n_blocks - 1, 0)]
    be = np.where(g < n_blocks, be, last).astype(np.int32)
    return {"blk_expert": be, "n_blocks": np.array([n_blocks], np.int32), "tok_row": tok_row, "w_row": w_row,
            "row_slot": row_slot.reshape(T, k)}


def prefill_apply(deq, x, idx, w, limit, E, tm=32, combine="matmul", deq_is_bf16=False):
    """The grouped prefill composition ResidentFetch._apply_ragged_kernel (resident.py:144-165) with the reference's
    bf16 rounding points: x rows -> bf16 (resident.py:153), dequantized tiles -> bf16 (pallas_moe.py:350),
    h = bf16(swiglu(f32 dots)) (pallas_moe.py:682), y = bf16(h @ Wd^T) (pallas_moe.py:747, out_dtype = bf16),
    combine "matmul": bf16(w_row) @ y with f32 accumulation (resident.py:161-163); "gather": f32 sum of
    y[row_slot] * w (resident.py:164-165).  Returns f64 [T, D].  ``deq`` returns exact weights; they are rounded
    to bf16 here (a no-op for CB3, whose weights are bf16 already)."""
    plan = ragged_plan(idx, w, E, tm)
    T, k = np.asarray(idx).shape
    xb = round_bf16(np.asarray(x, dtype=np.float32)).astype(np.float64)
    tok = plan["tok_row"]
    be = plan["blk_expert"]
    nb = int(plan["n_blocks"][0])
    D = None
    ys = {}
    for g0 in range(nb):
        e = int(be[g0])
        rows = np.arange(g0 * tm, (g0 + 1) * tm)
        t = tok[rows]
        xs = np.where((t >= 0)[:, None], xb[np.maximum(t, 0)], 0.0)
        Wg = round_bf16(deq("gate", e)).astype(np.float64)
        Wu = round_bf16(deq("up", e)).astype(np.float64)
        Wd = round_bf16(deq("down", e)).astype(np.float64)
        gg = (xs @ Wg.T).astype(np.float32)
        uu = (xs @ Wu.T).astype(np.float32)
        h = round_bf16(swiglu_clamped(gg, uu, limit)).astype(np.float64)
        y = round_bf16((h @ Wd.T).astype(np.float32)).astype(np.float64)
        D = y.shape[1]
        for i, r in enumerate(rows):
            ys[int(r)] = y[i]
    out = np.zeros((T, D), np.float64)
    if combine == "matmul":
        wr = round_bf16(plan["w_row"]).astype(np.float64)
        for r, t in enumerate(tok):
            if t >= 0 and r in ys:
                out[t] += wr[r] * ys[r]
    else:
        wf = np.asarray(w, dtype=np.float32).astype(np.float64)
        for t in range(T):
            for j in range(k):
                out[t] += wf[t, j] * ys[int(plan["row_slot"][t, j])]
    return out
