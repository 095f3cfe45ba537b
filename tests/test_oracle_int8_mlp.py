"""CPU: pins oracle.int8.mlp_partial_f32 (mlp_partial over int8 leaves, model.py:125-127 with quant8.py:91-99)
against an independent restatement in torch's own bf16 arithmetic -- bf16(f32(q) * s) weights, torch's bf16 matmuls
for g and u (f32 accumulation, bf16 out), F.silu on the clamped f32 values rounded to bf16, then h @ Wd in f32 --
and checks that dropping any one of its bf16 roundings (g, u, h), the plausible mistakes, moves it far beyond the
agreement (planted mistakes, each must fail).  The bf16-leaf form (W [in, out] bf16 itself) is pinned the same way
against torch with bf16 weights, and must equal the int8 form exactly when W = bf16(f32(q) * s)."""
import numpy as np
import pytest
import torch

from oracle import int8 as oi
from oracle.bf16 import rel_l2, round_bf16

AGREE = 1e-5        # observed ~2e-7 (f64 against torch's f32 accumulation)
PLANTED = 1e-3      # observed 1.7e-3 .. 3.2e-3


def _case(seed, limit):
    rng = np.random.default_rng(seed)
    B, D, I = 8, 512, 256
    leaf = lambda n_in, n_out, axis: oi.quantize_array(rng.standard_normal((n_in, n_out)).astype(np.float32) * 0.05,
                                                       axis)
    g, u, d = leaf(D, I, 1), leaf(D, I, 1), leaf(I, D, 0)
    x = round_bf16(rng.standard_normal((B, D)).astype(np.float32) * 2)
    return x, g, u, d, limit


def _torch_mlp(x, g, u, d, limit):
    w = lambda q, s: (torch.tensor(q).float() * torch.tensor(s)).bfloat16()
    xb = torch.tensor(x).bfloat16()
    gg, uu = xb @ w(*g), xb @ w(*u)
    h = (torch.nn.functional.silu(torch.clamp(gg.float(), max=limit)) * torch.clamp(uu.float(), -limit, limit))
    return (h.bfloat16().float() @ w(*d).float()).numpy(), gg.float().numpy(), uu.float().numpy()


@pytest.mark.parametrize("limit", [7.0, 1.5])
def test_mlp_partial_equals_torch_restatement(limit):
    x, g, u, d, L = _case(1, limit)
    want, gg, uu = _torch_mlp(x, g, u, d, L)
    if limit < 2:
        assert (gg > L).mean() > 0.05 and (np.abs(uu) > L).mean() > 0.05      # the clamps engage
    assert rel_l2(oi.mlp_partial_f32(x, g, u, d, L), want) < AGREE


@pytest.mark.parametrize("drop", ["g", "u", "h"])
def test_mlp_partial_planted_rounding_mistakes_fail(drop):
    x, g, u, d, L = _case(2, 7.0)
    want, _, _ = _torch_mlp(x, g, u, d, L)
    assert rel_l2(oi.mlp_partial_f32(x, g, u, d, L, _drop=(drop,)), want) > PLANTED


def _bf16_case(seed, limit, B=8, D=512, I=256):
    rng = np.random.default_rng(seed)
    W = lambda n_in, n_out: round_bf16(rng.standard_normal((n_in, n_out)).astype(np.float32) * 0.05)
    x = round_bf16(rng.standard_normal((B, D)).astype(np.float32) * 2)
    return x, W(D, I), W(D, I), W(I, D), limit


def _torch_mlp_bf16(x, g, u, d, limit):
    t = lambda a: torch.tensor(a).bfloat16()
    xb = t(x)
    gg, uu = xb @ t(g), xb @ t(u)
    h = (torch.nn.functional.silu(torch.clamp(gg.float(), max=limit)) * torch.clamp(uu.float(), -limit, limit))
    return (h.bfloat16().float() @ t(d).float()).numpy(), gg.float().numpy(), uu.float().numpy()


@pytest.mark.parametrize("limit", [7.0, 1.5])
def test_mlp_partial_bf16_leaves_equal_torch_restatement(limit):
    x, g, u, d, L = _bf16_case(3, limit)
    want, gg, uu = _torch_mlp_bf16(x, g, u, d, L)
    if limit < 2:
        assert (gg > L).mean() > 0.05 and (np.abs(uu) > L).mean() > 0.05      # the clamps engage
    assert rel_l2(oi.mlp_partial_f32(x, g, u, d, L), want) < AGREE


@pytest.mark.parametrize("drop", ["g", "u", "h"])
def test_mlp_partial_bf16_leaves_planted_rounding_mistakes_fail(drop):
    x, g, u, d, L = _bf16_case(4, 7.0)
    want, _, _ = _torch_mlp_bf16(x, g, u, d, L)
    assert rel_l2(oi.mlp_partial_f32(x, g, u, d, L, _drop=(drop,)), want) > PLANTED


def test_mlp_partial_bf16_leaves_of_dequantized_int8_equal_int8_form():
    x, g, u, d, L = _case(5, 7.0)
    W = [oi.dequant_bf16(*leaf) for leaf in (g, u, d)]
    assert np.array_equal(oi.mlp_partial_f32(x, *W, L), oi.mlp_partial_f32(x, g, u, d, L))
    assert np.array_equal(oi.project_w_f32(x, W[0]), oi.project_f32(x, *g))


def test_project_w_transposed_operand_fails():
    """A transposed weight (the layout mistake the kernels' wT [out, in] invites) is far from the torch product."""
    x, g, _, _, _ = _bf16_case(6, 7.0, D=256, I=256)
    want = (torch.tensor(x).bfloat16() @ torch.tensor(g).bfloat16()).float().numpy()
    assert rel_l2(oi.project_w_f32(x, g), want) < 1e-2                   # bf16 output rounding only
    assert rel_l2(oi.project_w_f32(x, g.T), want) > 0.5
