"""CPU: pins the oracle's prefill and fallback compositions (oracle.moe.prefill_apply, sweep_apply, gather_apply,
sweep_xla_apply, shared_apply) against independent restatements written here with torch: per-slot evaluation (no
ragged plan, no blocks, no padding), torch's own bf16 conversion and silu, and the reference's one-hot combine
matrix built directly.  Each pin runs on CB3 weights (exact in bf16) and on IQ3_S / IQ2_S weights (not exact in
bf16, so the tile rounding matters), f32 activations that are not bf16 values (so the x rounding matters),
duplicate experts within a token and several block sizes tm.

A planted mistake in the oracle -- one bf16 rounding point dropped (h, y, the tiles, x, the combine weights, the
sweep's h * rw) -- must move its result well beyond the agreement bound: each such variant is run and must fail.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import moe
from oracle.bf16 import rel_l2
from tests.util import Layer

AGREE = 1e-6          # torch restatement vs oracle: the same rounding points, f64 sums in a different order
PLANTED = 1e-4        # one dropped bf16 rounding point moves the result by ~1e-3 (one bf16 ulp per element)


def _bf(out_dtype):
    if out_dtype == "bf16":
        return lambda t: torch.as_tensor(t).to(torch.float32).to(torch.bfloat16).to(torch.float64)
    return lambda t: torch.as_tensor(t).to(torch.float32).to(torch.float64)


def _swiglu(g, u, limit):
    g = torch.as_tensor(g).to(torch.float64).clamp(max=limit)
    u = torch.as_tensor(u).to(torch.float64).clamp(-limit, limit)
    return F.silu(g) * u


def _weights(layer, bf, e):
    return tuple(bf(torch.from_numpy(layer.deq(m, e))) for m in ("gate", "up", "down"))


def torch_ragged(layer, x, idx, w, limit, combine, out_dtype):
    """_apply_ragged_kernel (resident.py:144-165) slot by slot: rows of bf16(x), bf16 tiles, h = bf16(f32 swiglu),
    y = bf16(f32 h Wd^T); matmul combine = one-hot [T, S] matrix times bf16(w), gather = f32 w."""
    bf = _bf(out_dtype)
    T, k = idx.shape
    X = bf(torch.from_numpy(x))
    Y = []
    for t in range(T):
        for j in range(k):
            Wg, Wu, Wd = _weights(layer, bf, int(idx[t, j]))
            g, u = (Wg @ X[t]).to(torch.float32), (Wu @ X[t]).to(torch.float32)
            h = bf(_swiglu(g, u, limit).to(torch.float32))
            Y.append(bf((Wd @ h).to(torch.float32)))
    Y = torch.stack(Y)                                                   # [S, D], slot order
    onehot = (torch.arange(T)[:, None] == torch.arange(T * k)[None, :] // k).to(torch.float64)
    wt = torch.from_numpy(w).reshape(-1)
    wc = bf(wt) if combine == "matmul" else wt.to(torch.float64)
    return (onehot * wc[None, :] @ Y).numpy()


def torch_sweep(layer, x, idx, w, limit, E, out_dtype):
    """_apply_sweep_kernel (resident.py:169-187): per (token, distinct routed expert): h = bf16(f32 swiglu),
    hk = bf16(f32(h) * rw) with rw the summed weight of that pair, y = sum of hk Wd^T unrounded."""
    bf = _bf(out_dtype)
    T, _ = idx.shape
    X = bf(torch.from_numpy(x))
    out = None
    for t in range(T):
        for e in sorted(set(idx[t].tolist())):
            rw = torch.tensor(w[t][idx[t] == e].astype(np.float32).sum(dtype=np.float32))
            Wg, Wu, Wd = _weights(layer, bf, e)
            g, u = (Wg @ X[t]).to(torch.float32), (Wu @ X[t]).to(torch.float32)
            h = bf(_swiglu(g, u, limit).to(torch.float32))
            hk = bf((h.to(torch.float32) * rw).to(torch.float32))
            y = Wd @ hk
            if out is None:
                out = torch.zeros((T, y.shape[0]), dtype=torch.float64)
            out[t] += y
    return out.numpy()


def torch_gather(layer, x, idx, w, limit, out_dtype):
    """_apply_gather (resident.py:122-135): every einsum's result in out_dtype, f32 combine."""
    bf = _bf(out_dtype)
    N, k = idx.shape
    X = bf(torch.from_numpy(x))
    out = None
    for n in range(N):
        for j in range(k):
            Wg, Wu, Wd = _weights(layer, bf, int(idx[n, j]))
            g, u = bf((Wg @ X[n]).to(torch.float32)), bf((Wu @ X[n]).to(torch.float32))
            h = bf(_swiglu(g, u, limit).to(torch.float32))
            y = bf((Wd @ h).to(torch.float32))
            if out is None:
                out = torch.zeros((N, y.shape[0]), dtype=torch.float64)
            out[n] += float(np.float32(w[n, j])) * y
    return out.numpy()


def torch_sweep_xla(layer, x, idx, w, limit, E, chunk, out_dtype):
    """_apply_sweep_xla (resident.py:189-210): per chunk of experts, one out_dtype rounding of the chunk's summed
    contribution, added in f32 order of chunks."""
    bf = _bf(out_dtype)
    T, _ = idx.shape
    X = bf(torch.from_numpy(x))
    acc = None
    for c0 in range(0, E, chunk):
        part = None
        for t in range(T):
            for e in sorted(set(idx[t].tolist())):
                if not c0 <= e < c0 + chunk:
                    continue
                rw = torch.tensor(w[t][idx[t] == e].astype(np.float32).sum(dtype=np.float32))
                Wg, Wu, Wd = _weights(layer, bf, e)
                g, u = bf((Wg @ X[t]).to(torch.float32)), bf((Wu @ X[t]).to(torch.float32))
                h = bf(_swiglu(g, u, limit).to(torch.float32))
                h2 = bf((h.to(torch.float32) * rw).to(torch.float32))
                if part is None:
                    part = torch.zeros((T, Wd.shape[0]), dtype=torch.float64)
                part[t] += Wd @ h2
        if part is not None:
            acc = bf(part.to(torch.float32)) if acc is None else acc + bf(part.to(torch.float32))
    return acc.numpy()


def _case(qtype, seed, T=7, k=3, E=5, dup=True):
    rng = np.random.default_rng(seed)
    D, I = (256, 256) if qtype != "CB3" else (128, 128)
    layer = Layer(rng, qtype, E, D, I, down_qtype=("IQ2_S" if qtype == "IQ3_S" else None))
    x = rng.standard_normal((T, D)).astype(np.float32)              # not bf16 values: the x rounding matters
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    if dup:
        idx[1, 1] = idx[1, 0]                                       # a token routed twice to one expert
    w = rng.random((T, k)).astype(np.float32)
    return layer, x, idx, w, E


QTYPES = ["CB3", "IQ3_S"]


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("combine", ["matmul", "gather"])
@pytest.mark.parametrize("out_dtype", ["bf16", "f32"])
def test_prefill_apply_equals_torch_restatement(qtype, combine, out_dtype):
    layer, x, idx, w, E = _case(qtype, 11)
    want = torch_ragged(layer, x, idx, w, 8.0, combine, out_dtype)
    for tm in (1, 3, 16):
        got = moe.prefill_apply(layer.deq, x, idx, w, 8.0, E, tm=tm, combine=combine, out_dtype=out_dtype)
        assert rel_l2(got, want) < AGREE, (tm, rel_l2(got, want))


@pytest.mark.parametrize("drop,qtype,combine", [("h", "CB3", "gather"), ("y", "CB3", "gather"),
                                                ("x", "CB3", "gather"), ("wc", "CB3", "matmul"),
                                                ("w", "IQ3_S", "gather"), ("h", "IQ3_S", "matmul")])
def test_prefill_planted_rounding_mistakes_fail(drop, qtype, combine):
    layer, x, idx, w, E = _case(qtype, 12)
    want = torch_ragged(layer, x, idx, w, 8.0, combine, "bf16")
    assert rel_l2(moe.prefill_apply(layer.deq, x, idx, w, 8.0, E, tm=4, combine=combine), want) < AGREE
    bad = moe.prefill_apply(layer.deq, x, idx, w, 8.0, E, tm=4, combine=combine, _drop=(drop,))
    assert rel_l2(bad, want) > PLANTED, drop


def test_prefill_clamps_engage():
    """A small limit makes the SwiGLU clamps bind on most elements: still equal to the restatement."""
    layer, x, idx, w, E = _case("CB3", 13)
    x = x * 40.0
    want = torch_ragged(layer, x, idx, w, 0.05, "matmul", "bf16")
    got = moe.prefill_apply(layer.deq, x, idx, w, 0.05, E, tm=2)
    assert rel_l2(got, want) < AGREE


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("out_dtype", ["bf16", "f32"])
def test_sweep_apply_equals_torch_restatement(qtype, out_dtype):
    layer, x, idx, w, E = _case(qtype, 21)
    want = torch_sweep(layer, x, idx, w, 8.0, E, out_dtype)
    assert rel_l2(moe.sweep_apply(layer.deq, x, idx, w, 8.0, E, out_dtype=out_dtype), want) < AGREE


@pytest.mark.parametrize("drop", ["h", "hk", "x"])
def test_sweep_planted_rounding_mistakes_fail(drop):
    layer, x, idx, w, E = _case("CB3", 22)
    want = torch_sweep(layer, x, idx, w, 8.0, E, "bf16")
    assert rel_l2(moe.sweep_apply(layer.deq, x, idx, w, 8.0, E, _drop=(drop,)), want) > PLANTED


@pytest.mark.parametrize("qtype", QTYPES)
@pytest.mark.parametrize("out_dtype", ["bf16", "f32"])
def test_gather_apply_equals_torch_restatement(qtype, out_dtype):
    layer, x, idx, w, E = _case(qtype, 31)
    want = torch_gather(layer, x, idx, w, 8.0, out_dtype)
    assert rel_l2(moe.gather_apply(layer.deq, x, idx, w, 8.0, out_dtype=out_dtype), want) < AGREE


@pytest.mark.parametrize("chunk", [1, 2, 8])
@pytest.mark.parametrize("out_dtype", ["bf16", "f32"])
def test_sweep_xla_apply_equals_torch_restatement(chunk, out_dtype):
    layer, x, idx, w, E = _case("IQ3_S", 41)
    want = torch_sweep_xla(layer, x, idx, w, 8.0, E, chunk, out_dtype)
    assert rel_l2(moe.sweep_xla_apply(layer.deq, x, idx, w, 8.0, E, chunk=chunk, out_dtype=out_dtype), want) < AGREE


def test_f32_compositions_agree_with_the_f64_decode():
    """out_dtype f32: the ragged, sweep, gather and XLA-sweep compositions are the decode composition in f32
    (resident.py:110-120) up to f32 rounding of the dots."""
    layer, x, idx, w, E = _case("IQ3_S", 51)
    ref = moe.decode_apply(layer.deq, x, idx, w, 8.0)
    for got in (moe.prefill_apply(layer.deq, x, idx, w, 8.0, E, tm=3, out_dtype="f32"),
                moe.prefill_apply(layer.deq, x, idx, w, 8.0, E, tm=3, combine="gather", out_dtype="f32"),
                moe.sweep_apply(layer.deq, x, idx, w, 8.0, E, out_dtype="f32"),
                moe.gather_apply(layer.deq, x, idx, w, 8.0, out_dtype="f32"),
                moe.sweep_xla_apply(layer.deq, x, idx, w, 8.0, E, chunk=2, out_dtype="f32")):
        assert rel_l2(got, ref) < 1e-6


def test_shared_apply_is_a_weight_one_decode_slot():
    layer, x, idx, w, E = _case("CB3", 61)
    s = 3
    got = moe.shared_apply(lambda m: layer.deq(m, s), x, 8.0)
    want = moe.decode_apply(layer.deq, x, np.full((x.shape[0], 1), s, np.int32), np.ones((x.shape[0], 1),
                                                                                         np.float32), 8.0)
    assert rel_l2(got, want) < 1e-14
