"""float64 model of the ProteinMPNN v_48_020 decoder for bf16 error attribution.

Test infrastructure and analysis, not the product: the encoder and the
teacher-forced decoder (inverse_fold_scalar.cpp:575-663, decoder_layer_scalar.cpp:26-151)
restated in float64 with numpy, with an optional rounding applied to the weights
(w_*) or the inputs (a_*) of each product. Running the decoder on a design
trajectory with one group rounded to bf16 and comparing log_softmax(z / T) with
the unrounded model attributes the low-precision error to products.

    python tests/bf16_error_model.py [L]      # prints the table for L (default 300)
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

from hikoboshi_amd import backbone, weights  # noqa: E402

PRODUCTS = ("W1", "W2", "W3", "in", "out", "log")


def bf16(x):
    """Round to bfloat16 (nearest even) and back."""
    a = np.asarray(x, np.float32).copy()
    u = a.view(np.uint32)
    u += 0x7FFF + ((u >> 16) & 1)
    u &= 0xFFFF0000
    return a.view(np.float32).astype(np.float64)


def fp16(x):
    return np.asarray(x, np.float64).astype(np.float16).astype(np.float64)


def bf16x2(x):
    """Two bf16 terms, hi + lo (about 16 significant bits)."""
    hi = bf16(x)
    return hi + bf16(np.asarray(x, np.float64) - hi)


def exact(x):
    return np.asarray(x, np.float64)


class Model:
    def __init__(self):
        self.W = {k: np.asarray(v, np.float64) for k, v in zip(weights.CANONICAL_TENSORS, weights.load_tensors())}

    def lin(self, x, name, qw=exact, qa=exact, bias=True):
        y = qa(x) @ qw(self.W[name + ".weight"]).T
        if bias and (name + ".bias") in self.W:
            y = y + self.W[name + ".bias"]
        return y

    @staticmethod
    def gelu(x):  # A&S 7.1.26 erf as the reference (gelu.hpp:22-51), exact exp
        v = x * 0.7071067811865475
        a = np.abs(v)
        t = 1.0 / (1.0 + 0.3275911 * a)
        poly = (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t
        erf = np.where(a > 4, np.sign(v), np.sign(v) * (1 - poly * np.exp(-np.minimum(a * a, 16.0))))
        return 0.5 * x * (1 + erf)

    def ln(self, x, name):
        m = x.mean(-1, keepdims=True)
        v = ((x - m) ** 2).mean(-1, keepdims=True)
        return (x - m) / np.sqrt(v + 1e-5) * self.W[name + ".weight"] + self.W[name + ".bias"]

    def encode(self, feats, idx, mask):
        L, K = idx.shape
        S = L * K
        he = self.lin(feats.reshape(S, 416), "features.edge_embedding", bias=False)
        he = self.lin(self.ln(he, "features.norm_edges"), "W_e")
        hv = np.zeros((L, 128))
        valid = idx >= 0
        jj = np.where(valid, idx, 0)
        ma = (mask[:, None] * mask[jj] * valid).reshape(S, 1)
        g = self.gelu
        for layer in range(3):
            p = f"encoder_layers.{layer}."

            def msg_in():
                return np.concatenate([np.repeat(hv, K, 0), he, hv[jj].reshape(S, 128) * valid.reshape(S, 1)], 1)

            m = self.lin(g(self.lin(g(self.lin(msg_in(), p + "W1")), p + "W2")), p + "W3")
            hv = self.ln(hv + (m * ma / 30.0).reshape(L, K, 128).sum(1), p + "norm1")
            f = self.lin(g(self.lin(hv, p + "dense.W_in")), p + "dense.W_out")
            hv = self.ln(hv + f, p + "norm2") * mask[:, None]
            m = self.lin(g(self.lin(g(self.lin(msg_in(), p + "W11")), p + "W12")), p + "W13")
            he = np.where(valid.reshape(S, 1), self.ln(he + m, p + "norm3"), he)
        return he, hv

    def decode(self, he, hv, idx, mask, tokens, order, q=None):
        """Teacher-forced logits [L, 21]; q maps 'w_<product>' / 'a_<product>' to a rounding."""
        q = q or {}
        Q = lambda k: q.get(k, exact)  # noqa: E731
        L, K = idx.shape
        S = L * K
        valid = idx >= 0
        jj = np.where(valid, idx, 0)
        pos = np.empty(L, int)
        pos[order] = np.arange(L)
        bw = (valid & (pos[jj] < pos[:, None])) * mask[:, None]
        fw = (valid & ~(pos[jj] < pos[:, None])) * mask[:, None]
        hs = self.W["W_s.weight"][tokens]
        h0, h = hv.copy(), hv.copy()
        g = self.gelu
        for layer in range(3):
            p = f"decoder_layers.{layer}."
            ctx_bw = np.concatenate([he, hs[jj].reshape(S, 128), h[jj].reshape(S, 128)], 1) * valid.reshape(S, 1)
            ctx_fw = np.concatenate([he, np.zeros((S, 128)), h0[jj].reshape(S, 128)], 1) * valid.reshape(S, 1)
            x = np.concatenate([np.repeat(h, K, 0), bw.reshape(S, 1) * ctx_bw + fw.reshape(S, 1) * ctx_fw], 1)
            x = g(self.lin(x, p + "W1", Q("w_W1"), Q("a_W1")))
            x = g(self.lin(x, p + "W2", Q("w_W2"), Q("a_W2")))
            m = self.lin(x, p + "W3", Q("w_W3"), Q("a_W3"))
            h1 = self.ln(h + (m / 30.0).reshape(L, K, 128).sum(1), p + "norm1")
            f = self.lin(g(self.lin(h1, p + "dense.W_in", Q("w_in"), Q("a_in"))), p + "dense.W_out", Q("w_out"),
                         Q("a_out"))
            h = self.ln(h1 + f, p + "norm2") * mask[:, None]
        return self.lin(h, "W_out", Q("w_log"), Q("a_log"))


def log_softmax(z, T):
    z = z / T
    z = z - z.max(1, keepdims=True)
    return z - np.log(np.exp(z).sum(1, keepdims=True))


def variants():
    """Rounding schemes to compare: each bf16 group alone, the GPU's bf16 decode, fp16, and bf16 pairs."""
    out = {f"bf16 {k[0]}_{p}": {f"{k[0]}_{p}": bf16} for p in PRODUCTS for k in ("weights", "activations")}
    out["bf16 decode as on the GPU (W2 operands, W3/W_in/W_out/logit weights)"] = {
        "w_W2": bf16, "a_W2": bf16, "w_W3": bf16, "w_in": bf16, "w_out": bf16, "w_log": bf16}
    out["fp16 weights and activations of every product"] = {f"{k}_{p}": fp16 for p in PRODUCTS for k in "wa"}
    out["bf16 pairs (hi + lo) for every weight, exact activations"] = {f"w_{p}": bf16x2 for p in PRODUCTS}
    # the split bf16 mode (HKBS_PRECISION_BF16X3): weights and inputs of every product as bf16 pairs
    # (the logits' inputs stay fp32), then the same with the W1 inputs (the E1, Q and R rows) in fp16
    split = {**{f"w_{p}": bf16x2 for p in PRODUCTS}, **{f"a_{p}": bf16x2 for p in PRODUCTS if p != "log"}}
    out["split bf16: bf16 pairs for the weights and inputs of every product"] = split
    out["split bf16 with fp16 message-row inputs (E1, Q, R)"] = {**split, "a_W1": fp16}
    return out


def deviations(L, seeds=(5, 6), T=0.1):
    """max over seeds of max |d log_softmax(z / T)| for every variant, on oracle designs at T = 0.1."""
    from oracle import Oracle

    orc = Oracle(weights.load_tensors())
    model = Model()
    bb = backbone.single_chain(L, 21)
    idx, feats = orc.edge_features(bb)
    mask = np.ones(L)
    he, hv = model.encode(feats, idx, mask)
    res = {}
    for seed in seeds:
        d = orc.inverse_fold(bb, seed=seed, order_seed=seed, temperature=0.1)
        z0 = log_softmax(model.decode(he, hv, idx, mask, d["tokens"], d["order"]), T)
        for name, q in variants().items():
            z = log_softmax(model.decode(he, hv, idx, mask, d["tokens"], d["order"], q), T)
            res[name] = max(res.get(name, 0.0), float(np.abs(z - z0).max()))
    return res


if __name__ == "__main__":
    L = int(sys.argv[1]) if len(sys.argv) > 1 else 300
    for name, v in sorted(deviations(L).items(), key=lambda kv: kv[1]):
        print(f"{v:10.4g}  {name}", flush=True)
