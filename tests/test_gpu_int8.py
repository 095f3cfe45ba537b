"""GPU parity of the int8 projection (quant8.py:91-99 + x @ W) against the oracle: bf16(f32(q)*s) weights, exact
bf16 products, f32 accumulation, bf16 out."""
import os

import numpy as np
import pytest
import torch

from oracle import int8 as oi8
from oracle.bf16 import rel_l2, round_bf16

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("B,n_in,n_out", [(8, 512, 256), (1, 256, 16), (8, 2048, 6144), (16, 1024, 2048),
                                          (32, 512, 512), (3, 6144, 2048),
                                          (8, 6144, 6144), (8, 6144, 2048)])      # config 3: Q/K/V/O, shared gate/up
def test_int8_project(pkg, gpu, B, n_in, n_out):
    rng = np.random.default_rng(B * 1000 + n_out)
    q, s = oi8.generate(rng, n_in, n_out)
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    qT, sv, _ = pkg.formats.int8_pack(q, s)
    yb, yf = pkg.int8_project(torch.from_numpy(x).cuda().to(torch.bfloat16), torch.from_numpy(qT).cuda(),
                              torch.from_numpy(sv).cuda(), want_f32=True)
    want = oi8.project_f32(x, q, s)
    assert rel_l2(yf.cpu().numpy(), want) < 1e-5
    assert rel_l2(yb.float().cpu().numpy(), oi8.project_bf16(x, q, s)) < 1e-3


def test_int8_golden(pkg, gpu):
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "int8.npz"))
    qT, sv, _ = pkg.formats.int8_pack(z["q"], z["s"])
    yb = pkg.int8_project(torch.from_numpy(z["x"]).cuda().to(torch.bfloat16), torch.from_numpy(qT).cuda(),
                          torch.from_numpy(sv).cuda())
    assert rel_l2(yb.float().cpu().numpy(), z["y"]) < 1e-3


def test_int8_project_many_equals_single(pkg, gpu):
    """One launch over Q, K, V-like projections (and a narrower one) gives exactly what separate calls give."""
    rng = np.random.default_rng(9)
    B, n_in = 8, 1024
    shapes = [512, 512, 256, 768]
    qs = [oi8.generate(rng, n_in, n) for n in shapes]
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    projs = []
    for q, s in qs:
        qT, sv, _ = pkg.formats.int8_pack(q, s)
        projs.append((torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda()))
    many = pkg.int8_project_many(xt, projs, want_f32=True)
    for (q, s), (qT, sv), (yb, yf) in zip(qs, projs, many):
        yb1, yf1 = pkg.int8_project(xt, qT, sv, want_f32=True)
        assert rel_l2(yf.cpu().numpy(), yf1.cpu().numpy()) < 1e-6
        assert rel_l2(yf.cpu().numpy(), oi8.project_f32(x, q, s)) < 1e-5


@pytest.mark.parametrize("B,n_in,n_out", [(8, 6144, 6144), (8, 2048, 6144), (1, 512, 256), (20, 1024, 512)])
def test_int8_row_scales(pkg, gpu, B, n_in, n_out):
    """Per-row scales [in, 1], the reference's layout for row-sharded leaves (O and down projections;
    quant8.py:26-32,59-60): W = bf16(f32(q[i, o]) * s[i])."""
    rng = np.random.default_rng(B + n_in + n_out)
    q = rng.integers(-127, 128, (n_in, n_out), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (n_in, 1)).astype(np.float32)
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    qT, sv, axis = pkg.resident.int8_leaf({"q": q, "s": s})
    assert axis == pkg._lib.MI_I8_ROW_SCALES
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    yb, yf = pkg.int8_project(xt, qT, sv, want_f32=True, scale_axis=axis)
    assert rel_l2(yf.cpu().numpy(), oi8.project_f32(x, q, s)) < 1e-5
    assert rel_l2(yb.float().cpu().numpy(), oi8.project_bf16(x, q, s)) < 1e-3
    (yb2, yf2), = pkg.int8_project_many(xt, [(qT, sv)], want_f32=True, scale_axis=axis)
    assert torch.equal(yf2, yf)


@pytest.mark.parametrize("B,n_in,n_out", [(1, 6144, 2048), (8, 4096, 1024), (32, 512, 128)])
def test_int8_lm_head_form(pkg, gpu, B, n_in, n_out):
    """The int8 lm_head (engine.py:345-351): (h @ f32(q)) * s[o] with f32 accumulation, then bf16."""
    rng = np.random.default_rng(B * 7 + n_out)
    q = rng.integers(-127, 128, (n_in, n_out), dtype=np.int8)
    s = rng.uniform(0.5e-3, 2e-3, (1, n_out)).astype(np.float32)
    x = round_bf16(rng.standard_normal((B, n_in)).astype(np.float32))
    xt = torch.from_numpy(x).cuda().to(torch.bfloat16)
    yb, yf = pkg.resident.int8_logits(xt, {"q": q, "s": s}, want_f32=True)
    want = oi8.project_after_f32(x, q, s)
    assert rel_l2(yf.cpu().numpy(), want) < 1e-5
    assert rel_l2(yb.float().cpu().numpy(), round_bf16(want)) < 1e-3
