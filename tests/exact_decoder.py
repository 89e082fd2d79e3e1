"""float64 teacher-forced decoder: the arbiter of fp32 rounding differences.

Test infrastructure, not the product. It restates the teacher-forced decoder of
the reference (cpp/modules/mpnn/inverse_fold_scalar.cpp:575-663,
cpp/modules/mpnn/decoder_layer_scalar.cpp:26-151) in float64 with torch on the
CPU, from a given encoder output (h_V, h_E, kNN graph, residue mask), tokens and
decoding order, and returns temperature-scaled log-probs [L, 21].

Two fp32 computations of the same design (the reference's scalar code and the
GPU's restructured one) round differently; where they differ by more than the
fp32 tolerance, this decoder tells which of the two is nearer the value that
exact arithmetic gives on the same inputs. It computes

    W1 [h_t, ctx_tk] + b1 = W1a h_t + b1 + W1b h_E,tk + bw (W1c W_s[s_j] + W1d h_j) + fw W1d h0_j

with the per-residue products formed first (an exact identity; float64
reassociation moves the result by about 1e-15), GELU as the reference's
A&S 7.1.26 form (cpp/include/hikoboshi/primitives/compute/gelu.hpp:22-65) with
exact exp, and LayerNorm with exact mean and variance. tests/bf16_error_model.py
holds the same decoder in plain numpy (the [h_t, ctx] concatenation as the
reference writes it); tests/test_exact_decoder.py pins the two together and this
one to the oracle.
"""
from __future__ import annotations

import numpy as np
import torch

from hikoboshi_amd import weights

_W = None
_ROWS = 64  # residues per block of the edge products


def _weights():
    global _W
    if _W is None:
        _W = {k: torch.from_numpy(np.asarray(v, np.float64)) for k, v in
              zip(weights.CANONICAL_TENSORS, weights.load_tensors())}
    return _W


def _gelu(x):
    v = x * 0.7071067811865475
    a = v.abs()
    t = 1.0 / (1.0 + 0.3275911 * a)
    poly = (((((1.061405429 * t - 1.453152027) * t) + 1.421413741) * t - 0.284496736) * t + 0.254829592) * t
    erf = torch.where(a > 4, torch.sign(v), torch.sign(v) * (1 - poly * torch.exp(-torch.clamp(a * a, max=16.0))))
    return 0.5 * x * (1 + erf)


def _ln(x, W, name):
    m = x.mean(-1, keepdim=True)
    var = ((x - m) ** 2).mean(-1, keepdim=True)
    return (x - m) / torch.sqrt(var + 1e-5) * W[name + ".weight"] + W[name + ".bias"]


def log_probs(enc, tokens, order, temperature):
    """Teacher-forced log_softmax(logits / T) in float64; enc = (mask [L], idx [L,K], h_V [L,128],
    h_E [L,K,128]) as the oracle's encode returns them."""
    W = _weights()
    mask, idx, hv, he = enc
    L, K = idx.shape
    mask = torch.from_numpy(np.asarray(mask, np.float64))
    idx_t = torch.from_numpy(np.asarray(idx, np.int64))
    valid = idx_t >= 0
    jj = torch.where(valid, idx_t, torch.zeros_like(idx_t))
    pos = torch.empty(L, dtype=torch.int64)
    pos[torch.from_numpy(np.asarray(order, np.int64))] = torch.arange(L)
    earlier = pos[jj] < pos[:, None]
    bw = (valid & earlier).double() * mask[:, None]
    fw = (valid & ~earlier).double() * mask[:, None]
    h0 = torch.from_numpy(np.asarray(hv, np.float64))
    he = torch.from_numpy(np.asarray(he, np.float64)).reshape(L, K, 128)
    hs = W["W_s.weight"][torch.from_numpy(np.asarray(tokens, np.int64))]
    h = h0.clone()
    for layer in range(3):
        p = f"decoder_layers.{layer}."
        W1 = W[p + "W1.weight"]
        W1a, W1b, W1c, W1d = W1[:, :128], W1[:, 128:256], W1[:, 256:384], W1[:, 384:]
        A = h @ W1a.T + W[p + "W1.bias"]                         # [L, 128]
        Rb = hs @ W1c.T + h @ W1d.T                               # backward neighbour term [L, 128]
        Qf = h0 @ W1d.T                                           # forward neighbour term
        msum = torch.empty(L, 128, dtype=torch.float64)
        for r0 in range(0, L, _ROWS):  # residue blocks: the [rows, K, 128] temporaries stay in cache
            r = slice(r0, min(L, r0 + _ROWS))
            E = he[r] @ W1b.T                                     # [rows, K, 128]
            # the whole context is zero for an empty slot and for an inactive residue (bw = fw = 0)
            x = A[r, None, :] + (bw[r] + fw[r])[..., None] * E + bw[r, :, None] * Rb[jj[r]] + fw[r, :, None] * Qf[jj[r]]
            g = _gelu(_gelu(x) @ W[p + "W2.weight"].T + W[p + "W2.bias"])
            msum[r] = (g @ W[p + "W3.weight"].T + W[p + "W3.bias"]).sum(1)
        h1 = _ln(h + msum / 30.0, W, p + "norm1")
        f = _gelu(h1 @ W[p + "dense.W_in.weight"].T + W[p + "dense.W_in.bias"])
        f = f @ W[p + "dense.W_out.weight"].T + W[p + "dense.W_out.bias"]
        h = _ln(h1 + f, W, p + "norm2") * mask[:, None]
    z = (h @ W["W_out.weight"].T + W["W_out.bias"]) / temperature
    return torch.log_softmax(z, -1).numpy()
