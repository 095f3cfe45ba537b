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
    qT, sv = pkg.formats.int8_pack(q, s)
    yb, yf = pkg.int8_project(torch.from_numpy(x).cuda().to(torch.bfloat16), torch.from_numpy(qT).cuda(),
                              torch.from_numpy(sv).cuda(), want_f32=True)
    want = oi8.project_f32(x, q, s)
    assert rel_l2(yf.cpu().numpy(), want) < 1e-5
    assert rel_l2(yb.float().cpu().numpy(), oi8.project_bf16(x, q, s)) < 1e-3


def test_int8_golden(pkg, gpu):
    z = np.load(os.path.join(os.path.dirname(__file__), "golden", "int8.npz"))
    qT, sv = pkg.formats.int8_pack(z["q"], z["s"])
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
        qT, sv = pkg.formats.int8_pack(q, s)
        projs.append((torch.from_numpy(qT).cuda(), torch.from_numpy(sv).cuda()))
    many = pkg.int8_project_many(xt, projs, want_f32=True)
    for (q, s), (qT, sv), (yb, yf) in zip(qs, projs, many):
        yb1, yf1 = pkg.int8_project(xt, qT, sv, want_f32=True)
        assert rel_l2(yf.cpu().numpy(), yf1.cpu().numpy()) < 1e-6
        assert rel_l2(yf.cpu().numpy(), oi8.project_f32(x, q, s)) < 1e-5
