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


def prefill_apply(deq, x, idx, w, limit, E, tm=32, combine="matmul", out_dtype="bf16", _drop=()):
    """The grouped prefill composition ResidentFetch._apply_ragged_kernel (resident.py:144-165) with the reference's
    rounding points for ``out_dtype`` "bf16": x rows -> bf16 (resident.py:153), dequantized tiles -> bf16
    (pallas_moe.py:350), h = bf16(swiglu(f32 dots)) (pallas_moe.py:682), y = bf16(h @ Wd^T) (pallas_moe.py:747,
    out_dtype = the input's), combine "matmul": bf16(w_row) @ y with f32 accumulation (resident.py:161-163);
    "gather": f32 sum of y[row_slot] * w (resident.py:164-165).  ``out_dtype`` "f32" (the reference's CPU tests,
    test_resident_cpu.py:81,124): every one of those values stays f32 (f32 tiles, HIGHEST-precision dots,
    pallas_moe.py:353-355).  Returns f64 [T, D].  ``deq`` returns exact weights (rounded here for bf16; a no-op for
    CB3, whose weights are bf16 already).  ``_drop`` names bf16 rounding points to skip ("x", "w", "h", "y", "wc"):
    for the planted-mistake tests only."""
    rb = round_bf16 if out_dtype == "bf16" else (lambda a: np.asarray(a, dtype=np.float32))
    rnd = lambda name, a: np.asarray(a, dtype=np.float32) if name in _drop else rb(a)
    plan = ragged_plan(idx, w, E, tm)
    T, k = np.asarray(idx).shape
    xb = rnd("x", np.asarray(x, dtype=np.float32)).astype(np.float64)
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
        Wg = rnd("w", deq("gate", e)).astype(np.float64)
        Wu = rnd("w", deq("up", e)).astype(np.float64)
        Wd = rnd("w", deq("down", e)).astype(np.float64)
        gg = (xs @ Wg.T).astype(np.float32)
        uu = (xs @ Wu.T).astype(np.float32)
        h = rnd("h", swiglu_clamped(gg, uu, limit)).astype(np.float64)
        y = rnd("y", (h @ Wd.T).astype(np.float32)).astype(np.float64)
        D = y.shape[1]
        for i, r in enumerate(rows):
            ys[int(r)] = y[i]
    out = np.zeros((T, D), np.float64)
    if combine == "matmul":
        wr = rnd("wc", plan["w_row"]).astype(np.float64)
        for r, t in enumerate(tok):
            if t >= 0 and r in ys:
                out[t] += wr[r] * ys[r]
    else:
        wf = np.asarray(w, dtype=np.float32).astype(np.float64)
        for t in range(T):
            for j in range(k):
                out[t] += wf[t, j] * ys[int(plan["row_slot"][t, j])]
    return out


def routing_weights(idx, w, E):
    """rw [T, E] = sum_j w[t, j] [idx[t, j] == e] in f32 (the sweeps' one-hot einsum, resident.py:176-177,195-196)."""
    idx = np.asarray(idx)
    rw = np.zeros((idx.shape[0], E), np.float32)
    wf = np.asarray(w, dtype=np.float32)
    for t in range(idx.shape[0]):
        for j in range(idx.shape[1]):
            rw[t, idx[t, j]] += wf[t, j]
    return rw


def sweep_apply(deq, x, idx, w, limit, E, out_dtype="bf16", _drop=()):
    """The dense-sweep prefill ResidentFetch._apply_sweep_kernel (resident.py:169-187) with moe_sweep_gateup /
    moe_sweep_down (pallas_moe.py:382-555): for every active expert e (ascending id) and every token t,
    h = bf16(swiglu(f32 dots of bf16(x) and bf16 tiles)) (pallas_moe.py:467), hk = bf16(f32(h) * rw[t, e])
    (resident.py:183-184), y[t] = sum_e hk @ bf16(Wd_e)^T with f32 accumulation and f32 output (pallas_moe.py:540,
    no rounding of y).  rw is the summed routing weight of (t, e); a token not routed to e has rw = 0 and adds
    exactly zero, so only routed pairs are evaluated.  ``out_dtype`` "f32": no rounding anywhere.  Returns f64
    [T, D].  ``_drop`` ("x", "w", "h", "hk"): planted-mistake tests only."""
    rb = round_bf16 if out_dtype == "bf16" else (lambda a: np.asarray(a, dtype=np.float32))
    rnd = lambda name, a: np.asarray(a, dtype=np.float32) if name in _drop else rb(a)
    idx = np.asarray(idx)
    T = idx.shape[0]
    rw = routing_weights(idx, w, E)
    xb = rnd("x", np.asarray(x, dtype=np.float32)).astype(np.float64)
    out = None
    for e in np.unique(idx):
        e = int(e)
        toks = np.flatnonzero(rw[:, e] != 0)
        if toks.size == 0:
            continue
        Wg = rnd("w", deq("gate", e)).astype(np.float64)
        Wu = rnd("w", deq("up", e)).astype(np.float64)
        Wd = rnd("w", deq("down", e)).astype(np.float64)
        xs = xb[toks]
        gg = (xs @ Wg.T).astype(np.float32)
        uu = (xs @ Wu.T).astype(np.float32)
        h = rnd("h", swiglu_clamped(gg, uu, limit))
        hk = rnd("hk", h.astype(np.float32) * rw[toks, e][:, None]).astype(np.float64)
        y = hk @ Wd.T
        if out is None:
            out = np.zeros((T, y.shape[1]), np.float64)
        out[toks] += y
    return out


def gather_apply(deq, x, idx, w, limit, out_dtype="bf16"):
    """The XLA decode path ResidentFetch._apply_gather (resident.py:122-135, use_pallas=False): weights dequantized
    to out_dtype (resident.py:91), xs = x in out_dtype, g = einsum(xs, Wg) and u likewise in out_dtype (bf16: one
    rounding of the f32-accumulated dot), h = swiglu_clamped(g, u) rounded to out_dtype, y = einsum(h, Wd) in
    out_dtype, then f32, out = sum_j w y in f32 (resident.py:133-135).  bf16's h is modelled as one rounding of the
    f32 SwiGLU of the rounded g and u (XLA's per-op rounding inside silu is not reproducible without XLA).
    ``out_dtype`` "f32" is the decode composition in f32.  Returns f64 [N, D]."""
    rb = round_bf16 if out_dtype == "bf16" else (lambda a: np.asarray(a, dtype=np.float32))
    idx = np.asarray(idx)
    N, k = idx.shape
    xb = rb(np.asarray(x, dtype=np.float32)).astype(np.float64)
    wf = np.asarray(w, dtype=np.float32).astype(np.float64)
    out = None
    for n in range(N):
        for j in range(k):
            e = int(idx[n, j])
            Wg = rb(deq("gate", e)).astype(np.float64)
            Wu = rb(deq("up", e)).astype(np.float64)
            Wd = rb(deq("down", e)).astype(np.float64)
            g = rb((Wg @ xb[n]).astype(np.float32))
            u = rb((Wu @ xb[n]).astype(np.float32))
            h = rb(swiglu_clamped(g, u, limit)).astype(np.float64)
            y = rb((Wd @ h).astype(np.float32)).astype(np.float64)
            if out is None:
                out = np.zeros((N, y.shape[0]), np.float64)
            out[n] += wf[n, j] * y
    return out


def sweep_xla_apply(deq, x, idx, w, limit, E, chunk=8, out_dtype="bf16"):
    """The XLA prefill path ResidentFetch._apply_sweep_xla (resident.py:189-210, use_pallas=False): experts in
    chunks of ``chunk``; per chunk g = einsum(xg, Wg) and u in out_dtype, h = swiglu (rounded as in
    ``gather_apply``), h2 = out_dtype(f32(h) * rw) (resident.py:206), and the chunk's contribution
    einsum("nem,emd->nd", h2, Wd) -- summed over the chunk's experts and the intermediate dimension with one
    rounding to out_dtype -- is added to an f32 accumulator (resident.py:207).  Experts no token routes to add
    exactly zero.  Returns f64 [T, D]."""
    rb = round_bf16 if out_dtype == "bf16" else (lambda a: np.asarray(a, dtype=np.float32))
    idx = np.asarray(idx)
    T = idx.shape[0]
    rw = routing_weights(idx, w, E)
    xb = rb(np.asarray(x, dtype=np.float32)).astype(np.float64)
    acc = None
    for c0 in range(0, E, chunk):
        part = None
        for e in range(c0, min(E, c0 + chunk)):
            toks = np.flatnonzero(rw[:, e] != 0)
            if toks.size == 0:
                continue
            Wg = rb(deq("gate", e)).astype(np.float64)
            Wu = rb(deq("up", e)).astype(np.float64)
            Wd = rb(deq("down", e)).astype(np.float64)
            g = rb((xb[toks] @ Wg.T).astype(np.float32))
            u = rb((xb[toks] @ Wu.T).astype(np.float32))
            h = rb(swiglu_clamped(g, u, limit))
            h2 = rb(h.astype(np.float32) * rw[toks, e][:, None]).astype(np.float64)
            if part is None:
                part = np.zeros((T, Wd.shape[0]), np.float64)
            part[toks] += h2 @ Wd.T
        if part is None:
            continue
        if acc is None:
            acc = np.zeros_like(part)
        acc += rb(part.astype(np.float32)).astype(np.float64)
    return acc
