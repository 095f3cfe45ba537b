"""Test helpers: seeded expert tables in every format (CB3, IQ2_S, IQ3_S, IQ4_XS, Q2_K, Q3_K), their device planes
and the oracle's view of them."""
import numpy as np

from oracle import cb3 as ocb3, iq2s as oiq2, iq3s as oiq3, iq4xs as oiq4, kquant as okq

MATS = ("gate", "up", "down")


class Layer:
    """E experts x {gate, up, down}; gate/up in ``qtype``, down in ``down_qtype`` (default: the same).  ``deq(name,
    e)`` is the oracle's exact f32 [R, K]."""

    def __init__(self, rng, qtype, E, D, I, scale=0.02, down_qtype=None):
        self.qtype, self.E, self.D, self.I = qtype, E, D, I
        self.qtypes = {"gate": qtype, "up": qtype, "down": down_qtype or qtype}
        self.shapes = {"gate": (I, D), "up": (I, D), "down": (D, I)}
        self.raw = {}
        for name, (R, K) in self.shapes.items():
            qt = self.qtypes[name]
            if qt == "CB3":
                codes, cb = zip(*[ocb3.generate(rng, R, K) for _ in range(E)])
                self.raw[name] = (np.stack(codes), np.stack(cb))
            elif qt == "IQ3_S":
                self.raw[name] = oiq3.random_blocks(rng, E, R, K // 256, scale=scale)
            elif qt == "IQ2_S":
                self.raw[name] = oiq2.random_blocks(rng, E, R, K // 256, scale=scale)
            elif qt in ("Q2_K", "Q3_K"):
                self.raw[name] = okq.random_blocks(rng, qt, E, R, K // 256, scale=scale)
            else:
                self.raw[name] = oiq4.random_blocks(rng, E, R, K // 256, scale=scale)
        self._cache = {}

    def deq(self, name, e):
        key = (name, e)
        if key not in self._cache:
            qt = self.qtypes[name]
            R, K = self.shapes[name]
            if qt == "CB3":
                codes, cb = self.raw[name]
                w = ocb3.dequant(codes[e], cb[e])
            elif qt == "IQ3_S":
                w = oiq3.dequant_blocks(self.raw[name][e]).reshape(R, K)
            elif qt == "IQ2_S":
                w = oiq2.dequant_blocks(self.raw[name][e]).reshape(R, K)
            elif qt in ("Q2_K", "Q3_K"):
                w = okq.dequant_blocks(self.raw[name][e], qt).reshape(R, K)
            else:
                w = oiq4.dequant_blocks(self.raw[name][e]).reshape(R, K)
            if len(self._cache) > 64:
                self._cache.clear()
            self._cache[key] = w
        return self._cache[key]

    def planes(self, name, fm):
        R, K = self.shapes[name]
        qt = self.qtypes[name]
        if qt == "CB3":
            codes, cb = self.raw[name]
            words = np.stack([ocb3.pack_canonical(c) for c in codes])
            return fm.cb3_pack_planes(words, cb, K)
        if qt == "IQ3_S":
            return fm.iq3s_pack_planes(self.raw[name])
        if qt == "IQ2_S":
            return fm.iq2s_pack_planes(self.raw[name])
        if qt in ("Q2_K", "Q3_K"):
            return fm.kq_pack_planes(self.raw[name], qt)
        return fm.iq4xs_pack_planes(self.raw[name])

    def tables(self, pkg, device="cuda"):
        out = {}
        for name in MATS:
            R, K = self.shapes[name]
            out[name] = pkg.ExpertTable(self.qtypes[name], pkg.to_device_planes(self.planes(name, pkg.formats),
                                                                                device), R, K)
        return out


def zipf_routing(rng, N, E, k, s=1.1):
    """Zipf(s)-skewed top-k routing over E experts (random rank -> id permutation), k distinct experts per token via
    Gumbel-top-k on log p; weights = softmax of N(0,1) logits over the chosen k."""
    ranks = np.arange(1, E + 1, dtype=np.float64)
    logp = -s * np.log(ranks)
    perm = rng.permutation(E)
    idx = np.zeros((N, k), np.int32)
    for n in range(N):
        g = logp + rng.gumbel(size=E)
        top = np.argsort(-g)[:k]
        idx[n] = perm[top]
    logits = rng.standard_normal((N, k))
    w = np.exp(logits - logits.max(-1, keepdims=True))
    w = (w / w.sum(-1, keepdims=True)).astype(np.float32)
    return idx, w


def softmax_topk_routing(rng, N, E, k):
    """Router logits ~ N(0,1); softmax; top-k; weights renormalized over the top-k (the benchmark's B=1 routing)."""
    logits = rng.standard_normal((N, E))
    p = np.exp(logits - logits.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    idx = np.argsort(-p, axis=-1)[:, :k].astype(np.int32)
    w = np.take_along_axis(p, idx, -1)
    w = (w / w.sum(-1, keepdims=True)).astype(np.float32)
    return idx, w
