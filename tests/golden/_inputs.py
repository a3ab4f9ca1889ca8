"""Seeded input generators shared by the golden writer and the tests.

Fixtures in this folder store the generator parameters, a SHA-256 of every
input array and the reference's outputs.  The tests regenerate the inputs
from the parameters (``numpy.random.default_rng``, PCG64) and check the
digests before comparing, so the committed files stay small.

Conventions: activations ~ N(0, 1); weight multivector
components ~ N(0, std) with ``std = 1/sqrt(8 * fan_in)`` (fan_in in
multivectors); "N(0, 0.5)" is read as a standard deviation.
"""

from __future__ import annotations

import hashlib

import numpy as np

F32 = np.float32


def digest(a: np.ndarray) -> str:
    a = np.ascontiguousarray(a)
    h = hashlib.sha256()
    h.update(str(a.dtype).encode())
    h.update(str(a.shape).encode())
    h.update(a.tobytes())
    return h.hexdigest()


def normal(r: np.random.Generator, shape, std=1.0) -> np.ndarray:
    return (r.standard_normal(shape, dtype=np.float32) * np.float32(std)).astype(F32)


def bf16_round(a: np.ndarray) -> np.ndarray:
    """Round fp32 to the nearest bf16 (ties to even) and widen back to fp32."""
    a = np.ascontiguousarray(a, dtype=F32)
    u = a.view(np.uint32).astype(np.uint64)
    lsb = (u >> 16) & 1
    u = ((u + 0x7FFF + lsb) >> 16) << 16
    return u.astype(np.uint32).view(F32).reshape(a.shape)


def expert_weights(r, E, d, F, bias_std=0.0):
    """Per-expert CliffordFFN weights: up (E,F,d,8), down (E,d,F,8), biases."""
    w_up = normal(r, (E, F, d, 8), 1.0 / np.sqrt(8.0 * d))
    w_down = normal(r, (E, d, F, 8), 1.0 / np.sqrt(8.0 * F))
    if bias_std > 0:
        b_up = normal(r, (E, F, 8), bias_std)
        b_down = normal(r, (E, d, 8), bias_std)
    else:
        b_up = np.zeros((E, F, 8), F32)
        b_down = np.zeros((E, d, 8), F32)
    return w_up, b_up, w_down, b_down


def zipf_logits(r, N, E, k, alpha=1.2):
    """Logits whose top-k load follows Zipf(alpha) over a random expert ranking.

    Per token, ``k`` distinct experts are drawn with ``p ∝ rank^-alpha`` and get
    logits ``k, k-1, ..., 1`` plus ``0.1 N(0,1)``; the rest get ``0.1 N(0,1)``.
    """
    ranking = r.permutation(E)
    p = (np.arange(1, E + 1, dtype=np.float64) ** -alpha)
    p /= p.sum()
    logits = normal(r, (N, E), 0.1)
    for t in range(N):
        chosen = r.choice(E, size=k, replace=False, p=p)
        for j, c in enumerate(chosen):
            logits[t, ranking[c]] += F32(k - j)
    return logits


def make_case(params: dict) -> dict:
    """Regenerate the inputs of one fixture case from its parameters."""
    kind = params["kind"]
    r = np.random.default_rng(params["seed"])
    if kind == "geom_matmul":
        M, K, N = params["M"], params["K"], params["N"]
        return {"a": normal(r, (M, K, 8)), "b": normal(r, (K, N, 8))}
    if kind == "route":
        N, E, d = params["N"], params["E"], params["d"]
        return {"logits": normal(r, (N, E)), "x": normal(r, (N, d, 8))}
    if kind in ("layer", "stack"):
        B, T, d, E, F = params["B"], params["T"], params["d"], params["E"], params["F"]
        layers = params.get("layers", 1)
        out = {"x": normal(r, (B, T, d, 8))}
        for li in range(layers):
            pre = f"l{li}_" if kind == "stack" else ""
            out[pre + "router_w"] = normal(r, (E, 4), 0.1)
            out[pre + "router_b"] = normal(r, (E,), params.get("router_bias_std", 0.0)) if params.get("router_bias_std", 0.0) else np.zeros(E, F32)
            wu, bu, wd, bd = expert_weights(r, E, d, F, params.get("bias_std", 0.0))
            out[pre + "w_up"], out[pre + "b_up"], out[pre + "w_down"], out[pre + "b_down"] = wu, bu, wd, bd
            lg = params.get("logits")
            N = B * T
            if lg == "normal":
                out[pre + "logits"] = normal(r, (N, E))
            elif lg == "normal_bias":
                out[pre + "logits"] = (normal(r, (N, E)) + normal(r, (E,), 0.5)[None, :]).astype(F32)
            elif lg == "zipf":
                out[pre + "logits"] = zipf_logits(r, N, E, params["k"])
            elif lg == "clifford_head":
                # CliffordLinear(d -> E) then grade 0 (the reference LM-head pattern)
                out[pre + "head_w"] = normal(r, (E, d, 8), 1.0 / np.sqrt(8.0 * d))
        if params.get("bf16"):
            for key in list(out):
                if key == "x" or "w_up" in key or "w_down" in key or "b_up" in key or "b_down" in key:
                    out[key] = bf16_round(out[key])
        return out
    raise ValueError(kind)
