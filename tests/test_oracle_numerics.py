"""CPU: pins the oracle's rounding, int8, SwiGLU and MoE compositions against torch (an independent library) and
brute force on tiny inputs."""
import numpy as np
import pytest
import torch

from oracle import bf16 as ob, cb3, int8 as oi8, moe


# ------------------------------------------------------------------------------------------------ bf16 / f16
def test_bf16_rounding_matches_torch():
    rng = np.random.default_rng(0)
    a = np.concatenate([rng.standard_normal(20000).astype(np.float32) * 10.0 ** rng.integers(-30, 30, 20000),
                        np.array([0.0, -0.0, np.inf, -np.inf, 1.0 + 2 ** -8, 1.0 + 3 * 2 ** -8, 1e-40, -3e-39,
                                  3.4e38], np.float32)]).astype(np.float32)
    want = torch.from_numpy(a).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ob.f32_to_bf16_bits(a), want)
    nan = ob.f32_to_bf16_bits(np.array([np.nan], np.float32))
    assert np.isnan(ob.bf16_bits_to_f32(nan)).all()


def test_f16_bits_match_numpy():
    h = np.arange(0, 65536, 7, dtype=np.uint32)
    want = h.astype(np.uint16).view(np.float16).astype(np.float32)
    got = ob.f16_bits_to_f32(h)
    fin = np.isfinite(want)
    assert np.array_equal(got[fin].view(np.uint32), want[fin].view(np.uint32))


# ------------------------------------------------------------------------------------------------ int8
def test_int8_dequant_matches_torch():
    rng = np.random.default_rng(1)
    q, s = oi8.generate(rng, 256, 128)
    want = (torch.from_numpy(q).float() * torch.from_numpy(s)).to(torch.bfloat16).float().numpy()
    assert np.array_equal(oi8.dequant_bf16(q, s).view(np.uint32), want.view(np.uint32))


def test_int8_row_scales_match_torch():
    """Per-row scales [in, 1] (quant8.py:26-32, axis 0): bf16(f32(q) * s[i]), checked with torch's rounding."""
    rng = np.random.default_rng(11)
    q = rng.integers(-127, 128, (256, 64), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (256, 1)).astype(np.float32)
    want = (torch.from_numpy(q).float() * torch.from_numpy(s)).to(torch.bfloat16).float().numpy()
    got = oi8.dequant_bf16(q, s)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    assert not np.array_equal(got, oi8.dequant_bf16(q, s.reshape(1, -1)[:, :64]))    # not the per-column form
    qq, ss = oi8.quantize_array(rng.standard_normal((256, 64)).astype(np.float32), 0)
    assert ss.shape == (256, 1) and np.abs(qq).max() == 127


def test_int8_lm_head_form_matches_torch():
    """engine.py:345-351: dot(h, q as h's dtype) in f32, times s after the dot."""
    rng = np.random.default_rng(12)
    q = rng.integers(-127, 128, (512, 96), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (1, 96)).astype(np.float32)
    x = ob.round_bf16(rng.standard_normal((3, 512)).astype(np.float32))
    xt = torch.from_numpy(x).double()
    want = ((xt @ torch.from_numpy(q).double()).float() * torch.from_numpy(s)).numpy()
    assert np.array_equal(oi8.project_after_f32(x, q, s), want)
    assert ob.rel_l2(oi8.project_after_f32(x, q, s), oi8.project_f32(x, q, s)) > 1e-4    # differs from bf16(q*s)


def test_int8_projection_matches_torch():
    rng = np.random.default_rng(2)
    q, s = oi8.generate(rng, 512, 64)
    x = cb3.bf16_normal(rng, (4, 512))
    W = (torch.from_numpy(q).double() * torch.from_numpy(s).double()).float().to(torch.bfloat16).double()
    want = (torch.from_numpy(x).double() @ W).float().numpy()
    assert np.array_equal(oi8.project_f32(x, q, s), want)


def test_int8_quantize_array():
    rng = np.random.default_rng(3)
    w = rng.standard_normal((64, 32)).astype(np.float32)
    q, s = oi8.quantize_array(w, axis=1)                      # per column [1, out]
    assert s.shape == (1, 32) and np.abs(q).max() <= 127
    assert (np.abs(q).max(0) == 127).all()                    # every column's amax maps to 127
    assert (np.abs(q * s - w) <= s / 2 + 1e-6).all()
    q0, s0 = oi8.quantize_array(w, axis=0)
    assert s0.shape == (64, 1) and (np.abs(q0).max(1) == 127).all()


# ------------------------------------------------------------------------------------------------ SwiGLU / MoE
def test_swiglu_matches_torch():
    rng = np.random.default_rng(4)
    g = rng.standard_normal(1000) * 8
    u = rng.standard_normal(1000) * 8
    L = 7.0
    tg, tu = torch.from_numpy(g), torch.from_numpy(u)
    want = (torch.nn.functional.silu(torch.clamp(tg, max=L)) * torch.clamp(tu, -L, L)).numpy()
    np.testing.assert_allclose(moe.swiglu_clamped(g, u, L), want, rtol=1e-12, atol=1e-12)


def _tiny_layer(rng, E, D, I):
    W = {(m, e): rng.standard_normal(shape).astype(np.float32) * 0.1
         for e in range(E) for m, shape in (("gate", (I, D)), ("up", (I, D)), ("down", (D, I)))}
    return lambda m, e: W[(m, e)]


def test_decode_apply_equals_per_slot_brute_force():
    rng = np.random.default_rng(5)
    E, D, I, N, k, L = 5, 12, 8, 3, 2, 3.0
    deq = _tiny_layer(rng, E, D, I)
    x = rng.standard_normal((N, D)).astype(np.float32)
    idx = np.array([[0, 3], [3, 1], [4, 0]], np.int32)
    w = rng.random((N, k)).astype(np.float32)
    got = moe.decode_apply(deq, x, idx, w, L)
    want = np.zeros((N, D))
    for n in range(N):
        for j in range(k):
            e = idx[n, j]
            x64 = x[n].astype(np.float64)
            gg = deq("gate", e).astype(np.float64) @ x64
            uu = deq("up", e).astype(np.float64) @ x64
            h = np.array([(min(a, L) / (1 + np.exp(-min(a, L)))) * min(max(b, -L), L) for a, b in zip(gg, uu)])
            want[n] += float(w[n, j]) * (deq("down", e).astype(np.float64) @ h)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("T,k,E,tm", [(5, 2, 4, 4), (16, 3, 6, 8), (1, 1, 3, 2), (9, 4, 4, 4)])
def test_ragged_plan_invariants_and_brute_force(T, k, E, tm):
    rng = np.random.default_rng(T * 100 + k)
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    p = moe.ragged_plan(idx, w, E, tm)
    S = T * k
    G = -(-S // tm) + E
    assert p["blk_expert"].shape == (G,) and p["tok_row"].shape == (G * tm,)
    counts = np.bincount(idx.reshape(-1), minlength=E)
    nb = int(p["n_blocks"][0])
    assert nb == int((-(-counts // tm)).sum())
    # every (t, j) owns one row inside a block of its expert, rows of one expert in slot order
    rows = p["row_slot"].reshape(-1)
    assert len(set(rows.tolist())) == S
    for t in range(T):
        for j in range(k):
            r = p["row_slot"][t, j]
            assert p["tok_row"][r] == t and p["w_row"][r] == w[t, j] and p["blk_expert"][r // tm] == idx[t, j]
    # within an expert, rows follow the slot order t * k + j (the reference's stable argsort)
    for e in range(E):
        slots = np.flatnonzero(idx.reshape(-1) == e)
        assert (np.diff(rows[slots]) > 0).all()
    # padding rows: token -1, weight 0; blocks past n_blocks repeat the last real block's expert
    pad = np.setdiff1d(np.arange(G * tm), rows)
    assert (p["tok_row"][pad] == -1).all() and (p["w_row"][pad] == 0).all()
    assert (p["blk_expert"][nb:] == p["blk_expert"][nb - 1]).all()
    # brute force: experts in ascending order, each padded to whole blocks
    want = []
    for e in range(E):
        want += [e] * (-(-counts[e] // tm))
    assert p["blk_expert"][:nb].tolist() == want


def test_prefill_flow_agrees_with_decode_at_bf16_tolerance():
    """The grouped prefill composition (bf16 rounding points) against the f64 decode composition: the reference's
    own tolerance pattern for the bf16 path (rtol 2e-2, test_planes.py:134) -- and the two combine modes agree."""
    rng = np.random.default_rng(6)
    E, D, I, T, k, L = 4, 64, 32, 6, 2, 10.0
    deq = _tiny_layer(rng, E, D, I)
    x = cb3.bf16_normal(rng, (T, D))
    idx = np.stack([rng.choice(E, k, replace=False) for _ in range(T)]).astype(np.int32)
    w = rng.random((T, k)).astype(np.float32)
    ref = moe.decode_apply(deq, x, idx, w, L)
    for combine in ("matmul", "gather"):
        got = moe.prefill_apply(deq, x, idx, w, L, E, tm=4, combine=combine)
        assert ob.rel_l2(got, ref) < 2e-2
    a = moe.prefill_apply(deq, x, idx, w, L, E, tm=4, combine="matmul")
    b = moe.prefill_apply(deq, x, idx, w, L, E, tm=4, combine="gather")
    assert ob.rel_l2(a, b) < 1e-2


def _route_brute(x, rw, bias, k, norm, scaling):
    """moe_route by k rounds of an explicit argmax (first maximum = lowest id), with torch's sigmoid."""
    logits = torch.from_numpy(np.asarray(x, np.float64)) @ torch.from_numpy(np.asarray(rw, np.float64))
    scores = torch.sigmoid(logits).numpy()
    choice = scores + (0.0 if bias is None else np.asarray(bias, np.float64))
    idx, w = [], []
    for n in range(choice.shape[0]):
        c = list(choice[n])
        row_i = []
        for _ in range(k):
            best = max(range(len(c)), key=lambda e: (c[e], -e))
            row_i.append(best)
            c[best] = -np.inf
        ws = [scores[n, e] for e in row_i]
        if norm:
            tot = sum(ws)
            ws = [v / (tot + 1e-20) for v in ws]
        idx.append(row_i)
        w.append([v * scaling for v in ws])
    return np.array(idx, np.int32), np.array(w)


@pytest.mark.parametrize("norm", [True, False])
def test_route_equals_argmax_rounds(norm):
    rng = np.random.default_rng(8)
    N, D, E, k = 6, 40, 12, 4
    x = ob.round_bf16(rng.standard_normal((N, D)).astype(np.float32))
    rw = rng.standard_normal((D, E)).astype(np.float32) * 0.2
    bias = rng.standard_normal(E).astype(np.float32) * 0.1
    i1, w1, _ = moe.route(x, rw, bias, k, norm, 2.5)
    i2, w2 = _route_brute(x, rw, bias, k, norm, 2.5)
    assert np.array_equal(i1, i2)
    np.testing.assert_allclose(w1, w2, rtol=1e-13)
    if norm:
        np.testing.assert_allclose(w1.sum(-1), 2.5, rtol=1e-12)


def test_route_ties_bias_and_weights():
    """Equal choices: lower id first (lax.top_k).  The bias moves the selection, the weights stay the scores."""
    E, k = 10, 3
    x = np.zeros((2, 8), np.float32)
    rw = np.zeros((8, E), np.float32)
    idx, w, _ = moe.route(x, rw, None, k, True, 1.0)              # every score 0.5, every choice equal
    assert idx.tolist() == [[0, 1, 2]] * 2 and np.allclose(w, 1.0 / 3)
    bias = np.zeros(E, np.float32)
    bias[[7, 4, 9]] = [3.0, 2.0, 1.0]
    idx, w, _ = moe.route(x, rw, bias, k, False, 2.0)
    assert idx.tolist() == [[7, 4, 9]] * 2 and np.allclose(w, 0.5 * 2.0)
