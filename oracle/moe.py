"""fp32-faithful NumPy restatement of the MoE-HLM expert layer (oracle).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Every function below restates one reference function and cites it.  The
restatement keeps the reference's fp32 operation order (NumPy on the CPU is
the reference's default backend, ``rune/backend.py:19``), so on identical
inputs it reproduces the reference's outputs bit for bit; the committed
goldens in ``tests/golden/`` check exactly that.

Pinning summary (tests named in brackets):

* ``geom_matmul`` -- bit-exact against the reference's compiled
  ``cl3_geom_matmul_flat`` (``oracle/_ref``) [test_oracle_ref_lib]; float64
  brute force; the special cases scalar-only W / scalar-only x reduce to
  ordinary matmuls; equivalence to the dense ``X . L(W)^T`` contraction
  [test_oracle_algebra].
* ``clifford_linear``, ``gelu``/``relu``/``sigmoid`` grade-wise activations,
  ``router_forward``, ``moe_forward_reference`` -- reference goldens
  [test_oracle_golden]; closed forms per grade (scalar-only input is the
  textbook tanh-GELU, grade 3 is ``tanh``) [test_oracle_algebra].
* ``route_topk`` (the build's descending / lowest-index rule), ``dispatch_plan``
  and ``combine`` -- brute force over all slots, and agreement with the
  reference's argsort selection on tie-free inputs [test_oracle_golden,
  test_oracle_routing].
* ``quantize_int8`` -- build-defined (no reference counterpart); pinned by its
  invariants (|q| <= 127, |W - q s| <= s/2, exact on multiples of s)
  [test_oracle_routing].
"""

from __future__ import annotations

import numpy as np

from .cl3 import PRODUCT_IDX, PRODUCT_SIGN, GRADE_SLICES, geom_prod, L_SRC, L_SIGN

F32 = np.float32

# ---------------------------------------------------------------------------
# geometric matmul and CliffordLinear
# ---------------------------------------------------------------------------


def geom_matmul(a: np.ndarray, b: np.ndarray, chunk: int = 64) -> np.ndarray:
    """``out[m, n] = sum_k gp(a[m, k], b[k, n])``; a (M,K,8), b (K,N,8).

    Restates ``rune/ops/batched.py:320-344`` (NumPy fallback: broadcast
    pairwise geometric product, then ``sum(axis=1)``) and
    ``mjolnir/src/cpu/batch_ops.c:56-71``.  Order: the K terms are added
    sequentially, k = 0..K-1, each term being the fp32 geometric product in
    the ``rune/ops/batched.py:72-82`` term order.  Columns are processed in
    chunks of ``chunk`` only to bound memory; that does not change any
    element's operation order.
    """
    a = np.ascontiguousarray(a, dtype=F32)
    b = np.ascontiguousarray(b, dtype=F32)
    assert a.ndim == 3 and b.ndim == 3 and a.shape[2] == 8 and b.shape[2] == 8
    M, K, _ = a.shape
    K2, N, _ = b.shape
    assert K == K2
    out = np.empty((M, N, 8), dtype=F32)
    for n0 in range(0, N, chunk):
        n1 = min(N, n0 + chunk)
        acc = np.zeros((M, n1 - n0, 8), dtype=F32)
        for k in range(K):
            acc += geom_prod(a[:, k, None, :], b[None, k, n0:n1, :])
        out[:, n0:n1] = acc
    return out


def geom_matmul_f64(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """float64 truth for ``geom_matmul`` via the dense ``L(W)`` contraction."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    La = a[..., L_SRC] * L_SIGN.astype(np.float64)  # (M,K,8r,8q)
    return np.einsum("mkrq,knq->mnr", La, b)


def clifford_linear(x: np.ndarray, weight: np.ndarray, bias: np.ndarray | None) -> np.ndarray:
    """CliffordLinear.forward: ``y[..., j] = sum_i W[j, i] * x[..., i] + b[j]``.

    Restates ``holograph/layers/clifford_linear.py:101-123``: flatten to
    (M, d_in, 8), transpose to (d_in, M, 8), ``geom_matmul(W, x_t)``,
    transpose back, then add the bias in fp32.
    """
    x = np.asarray(x, dtype=F32)
    d_out, d_in, _ = weight.shape
    batch = x.shape[:-2]
    assert x.shape[-2] == d_in
    x_t = np.ascontiguousarray(np.transpose(x.reshape(-1, d_in, 8), (1, 0, 2)))
    y = np.transpose(geom_matmul(weight, x_t), (1, 0, 2)).reshape(*batch, d_out, 8)
    if bias is not None:
        y = y + np.asarray(bias, dtype=F32)
    return y


# ---------------------------------------------------------------------------
# grade-wise activations (holograph/layers/activations.py)
# ---------------------------------------------------------------------------


def _gelu(v):
    """tanh-GELU, ``activations.py:15-17``.

    ``np.sqrt(2.0 / np.pi)`` is a float64 NumPy scalar; under NumPy 2 (NEP 50)
    it promotes the tanh argument and the result to float64.  Writing the
    expression the same way keeps that promotion; callers store the result
    into fp32 arrays, which rounds it once, as the reference does.
    """
    return 0.5 * v * (1.0 + np.tanh(np.sqrt(2.0 / np.pi) * (v + 0.044715 * v ** 3)))


def _sigmoid(v):
    """``activations.py:20-24``."""
    return np.where(v >= 0, 1.0 / (1.0 + np.exp(-v)), np.exp(v) / (1.0 + np.exp(v)))


def _magnitude_gate(c, fn):
    """``activations.py:27-38``: ``(c / |c|) * fn(|c|)``, ``|c| = sqrt(sum c^2 + 1e-12)``."""
    mag = np.sqrt(np.sum(c ** 2, axis=-1, keepdims=True) + 1e-12)
    return (c / mag) * fn(mag)


def gelu(data: np.ndarray) -> np.ndarray:
    """clifford_gelu, ``activations.py:41-62``."""
    data = np.asarray(data, dtype=F32)
    out = np.zeros_like(data)
    out[..., 0:1] = _gelu(data[..., 0:1])
    out[..., 1:4] = _magnitude_gate(data[..., 1:4], _gelu)
    out[..., 4:7] = _magnitude_gate(data[..., 4:7], _gelu)
    out[..., 7:8] = np.tanh(data[..., 7:8])
    return out


def relu(data: np.ndarray) -> np.ndarray:
    """clifford_relu with the default zero thresholds, ``activations.py:65-102``."""
    data = np.asarray(data, dtype=F32)
    t = np.zeros(4, dtype=F32)
    out = np.zeros_like(data)
    out[..., 0:1] = np.maximum(data[..., 0:1], t[0])
    for g, sl in ((1, slice(1, 4)), (2, slice(4, 7))):
        c = data[..., sl]
        mag = np.sqrt(np.sum(c ** 2, axis=-1, keepdims=True) + 1e-12)
        out[..., sl] = (c / mag) * np.maximum(mag - t[g], 0.0)
    tv = data[..., 7:8]
    out[..., 7:8] = np.sign(tv) * np.maximum(np.abs(tv) - t[3], 0.0)
    return out


def sigmoid(data: np.ndarray) -> np.ndarray:
    """clifford_sigmoid, ``activations.py:105-128``."""
    data = np.asarray(data, dtype=F32)
    out = np.zeros_like(data)
    out[..., 0:1] = _sigmoid(data[..., 0:1])
    out[..., 1:4] = _magnitude_gate(data[..., 1:4], _sigmoid)
    out[..., 4:7] = _magnitude_gate(data[..., 4:7], _sigmoid)
    out[..., 7:8] = np.tanh(data[..., 7:8])
    return out


ACTIVATIONS = {"gelu": gelu, "relu": relu, "sigmoid": sigmoid, "none": lambda d: np.asarray(d, dtype=F32)}


def clifford_ffn(x, w_up, b_up, w_down, b_down, activation="gelu"):
    """CliffordFFN.forward, ``holograph/models/hlm_block.py:55-61``."""
    h = clifford_linear(x, w_up, b_up)
    h = ACTIVATIONS[activation](h)
    return clifford_linear(h, w_down, b_down)


# ---------------------------------------------------------------------------
# router (holograph/layers/clifford_router.py)
# ---------------------------------------------------------------------------


def softmax(logits: np.ndarray) -> np.ndarray:
    """``clifford_router.py:18-21``: ``exp(l - max) / (sum + 1e-12)`` (fp32)."""
    m = np.max(logits, axis=-1, keepdims=True)
    e = np.exp(logits - m)
    return e / (np.sum(e, axis=-1, keepdims=True) + 1e-12)


def grade_energy(x: np.ndarray) -> np.ndarray:
    """``clifford_router.py:54-69``: per-grade sum of squares over (d, blade)."""
    x = np.asarray(x, dtype=F32)
    energy = np.zeros((*x.shape[:-2], 4), dtype=F32)
    for g in range(4):
        energy[..., g] = np.sum(x[..., GRADE_SLICES[g]] ** 2, axis=(-2, -1))
    return energy


def router_logits(x: np.ndarray, router_weight: np.ndarray, router_bias: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Energy-signature logits, ``clifford_router.py:83-90``. Returns (logits, energy)."""
    energy = grade_energy(x)
    energy_norm = energy / (np.sum(energy, axis=-1, keepdims=True) + 1e-12)
    logits = np.einsum("...g,eg->...e", energy_norm, router_weight) + router_bias
    return logits, energy


def topk_reference(probs: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """Reference selection ``clifford_router.py:95-104``.

    ``argsort`` ascending, last ``k`` columns (so slot ``k-1`` is the argmax),
    then renormalise by ``sum + 1e-12`` summed in that (ascending) slot order.
    Its tie order is NumPy's and is not the build's rule; use only on
    tie-free inputs.
    """
    idx = np.argsort(probs, axis=-1)[..., -k:]
    w = np.take_along_axis(probs, idx, axis=-1)
    w = w / (np.sum(w, axis=-1, keepdims=True) + 1e-12)
    return idx, w


def route_topk(probs: np.ndarray, k: int) -> tuple[np.ndarray, np.ndarray]:
    """The build's routing rule on top of the reference's probabilities.

    Slot 0 holds the most probable expert; equal probabilities are ordered by
    the lower expert index first (so at the k-th place the lower index wins).
    The renormalising sum is accumulated from the least probable selected
    slot to the most probable one -- the order the reference sums its
    ascending argsort output in (``clifford_router.py:104``) -- so on
    tie-free inputs the weights are bit-identical to the reference's.
    """
    probs = np.asarray(probs, dtype=F32)
    N, E = probs.shape
    # lexsort: last key is primary -> (-prob, index)
    order = np.lexsort((np.broadcast_to(np.arange(E), (N, E)), -probs), axis=-1)
    idx = order[:, :k].astype(np.int32)
    w = np.take_along_axis(probs, idx, axis=-1)
    s = np.zeros(N, dtype=F32)
    for j in range(k - 1, -1, -1):
        s = s + w[:, j]
    w = w / (s[:, None] + F32(1e-12))
    return idx, w.astype(F32)


def router_forward(x, router_weight, router_bias, k):
    """``CliffordRouter.forward`` (``clifford_router.py:71-106``), reference slot order."""
    logits, energy = router_logits(x, router_weight, router_bias)
    probs = softmax(logits)
    idx, w = topk_reference(probs, k)
    return idx, w, energy


# ---------------------------------------------------------------------------
# dispatch / combine (holograph/models/hlm_block.py:154-183)
# ---------------------------------------------------------------------------


def dispatch_plan(idx: np.ndarray, n_experts: int):
    """Counts, offsets, permutation and slot positions for a routing.

    ``_moe_forward`` visits experts in ascending order and, within one, the
    flat slots ``t*k + s`` in ascending order (``hlm_block.py:165-178``).
    That is a stable counting sort of the flat slots by expert: ``perm[p]`` is
    the token of the p-th sorted row and ``slot_pos[t, s]`` is the sorted row
    of slot ``(t, s)``.  A token never holds one expert twice, so within an
    expert the rows are in ascending token order.
    """
    idx = np.asarray(idx)
    N, k = idx.shape
    flat = idx.reshape(-1)
    counts = np.bincount(flat, minlength=n_experts).astype(np.int32)
    offsets = np.zeros(n_experts + 1, dtype=np.int32)
    offsets[1:] = np.cumsum(counts)
    order = np.argsort(flat, kind="stable")  # flat slot ids grouped by expert
    perm = (order // k).astype(np.int32)
    slot_pos = np.empty(N * k, dtype=np.int32)
    slot_pos[order] = np.arange(N * k, dtype=np.int32)
    return counts, offsets, perm, slot_pos.reshape(N, k)


def combine(y_sorted: np.ndarray, idx: np.ndarray, w: np.ndarray, slot_pos: np.ndarray) -> np.ndarray:
    """Weighted combine in the reference's order (``hlm_block.py:180-181``).

    ``out[t] = ((0 + w_a y_a) + w_b y_b) + ...`` over the token's experts in
    ascending expert order, each ``w * y`` rounded to fp32 before the add --
    what ``np.add.at`` does when it is called once per expert in ascending
    order.
    """
    N, k = idx.shape
    order = np.argsort(idx, axis=-1, kind="stable")
    out = np.zeros((N,) + y_sorted.shape[1:], dtype=F32)
    for j in range(k):
        s = order[:, j]
        rows = slot_pos[np.arange(N), s]
        ws = w[np.arange(N), s].astype(F32)
        term = ws.reshape((N,) + (1,) * (y_sorted.ndim - 1)) * y_sorted[rows].astype(F32)
        out = out + term
    return out


def moe_forward_reference(x, router_weight, router_bias, experts, k, activation="gelu", logits=None):
    """``HLMBlock._moe_forward`` (``hlm_block.py:154-183``) restated.

    ``x``: (B, T, d, 8).  ``experts``: list of (w_up, b_up, w_down, b_down).
    If ``logits`` (N, E) is given it replaces the router's energy logits
    (route-from-logits entry, configs 2-5); softmax, selection and
    renormalisation are the reference's either way.  Returns
    ``(out, info)`` with the reference's own ``idx``/``w`` (ascending slot
    order), counts and the expert-grouped token order.
    """
    x = np.asarray(x, dtype=F32)
    B, T, d, _ = x.shape
    N = B * T
    flat_x = x.reshape(N, d, 8)
    out = np.zeros_like(flat_x)
    if logits is None:
        logits, energy = router_logits(flat_x, router_weight, router_bias)
    else:
        energy = None
    probs = softmax(np.asarray(logits, dtype=F32))
    idx, w = topk_reference(probs, k)
    flat_idx = idx.reshape(-1)
    flat_w = w.reshape(-1)
    flat_tok = np.broadcast_to(np.arange(N, dtype=np.int32)[:, None], idx.shape).reshape(-1)
    counts = np.zeros(len(experts), dtype=np.int32)
    perm = []
    for e, (wu, bu, wd, bd) in enumerate(experts):
        mask = flat_idx == e
        counts[e] = int(mask.sum())
        if not mask.any():
            continue
        tok = flat_tok[mask]
        perm.append(tok)
        y = clifford_ffn(flat_x[tok], wu, bu, wd, bd, activation)
        np.add.at(out, tok, flat_w[mask][:, None, None] * y)
    perm = np.concatenate(perm).astype(np.int32) if perm else np.zeros(0, np.int32)
    info = dict(logits=logits, probs=probs, idx=idx, w=w, energy=energy, counts=counts, perm=perm)
    return out.reshape(B, T, d, 8), info


# ---------------------------------------------------------------------------
# int8 weights (build-defined; conventions of bifrost/quantization)
# ---------------------------------------------------------------------------


def quantize_int8(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-output-channel int8 for CliffordLinear weights.

    ``w``: (..., d_out, d_in, 8).  One scale per output multivector channel
    ``j`` (it factors out of every row ``(j, r)`` of ``L(W)``):
    ``s = max(absmax_j, 1e-12) / 127`` (computed in float64, stored fp32),
    ``q = clip(rint(w / s), -127, 127)``.  Conventions from
    ``bifrost/quantization/grade_quantize.py:85-117`` (symmetric absmax/qmax,
    ``1e-12`` floor) and ``:198-203`` (round half to even, clip).
    """
    w64 = np.asarray(w, dtype=np.float64)
    absmax = np.max(np.abs(w64), axis=(-2, -1))
    s = (np.maximum(absmax, 1e-12) / 127.0).astype(F32)
    q = np.clip(np.rint(w64 / s.astype(np.float64)[..., None, None]), -127, 127).astype(np.int8)
    return q, s


def dequantize_int8(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """``q * s`` rounded to fp32 -- the weights the int8 path is checked against."""
    return (q.astype(np.float64) * s.astype(np.float64)[..., None, None]).astype(F32)


# ---- int8 Pauli weights (weight format 5) -----------------------------------------------
# A Cl(3,0) multivector s + v1 e1 + v2 e2 + v3 e3 + b12 e12 + b13 e13 + b23 e23 + t e123 is
# the 2x2 complex matrix s I + v1 sx + v2 sy + v3 sz + b12 sx sy + b13 sx sz + b23 sy sz
# + t sx sy sz (sx, sy, sz the Pauli matrices), and the geometric product is the matrix
# product.  Its eight real entries, ordered [U00, V00, U01, V01, U10, V10, U11, V11]
# (entry (a, c) of U + iV), are what format 5 quantizes.


def pauli_entries(w: np.ndarray) -> np.ndarray:
    """Blade-order multivectors (..., 8) -> their matrices' real entries (..., 8), float64."""
    w = np.asarray(w, dtype=np.float64)
    s, v1, v2, v3, b12, b13, b23, t = (w[..., i] for i in range(8))
    return np.stack([s + v3, t + b12, v1 - b13, b23 - v2, v1 + b13, b23 + v2, s - v3, t - b12], axis=-1)


def from_pauli_entries(p: np.ndarray) -> np.ndarray:
    """Inverse of :func:`pauli_entries` (float64; exact up to the halving)."""
    p = np.asarray(p, dtype=np.float64)
    u00, v00, u01, v01, u10, v10, u11, v11 = (p[..., i] for i in range(8))
    return 0.5 * np.stack([u00 + u11, u10 + u01, v10 - v01, u00 - u11, v00 - v11, u10 - u01, v10 + v01,
                           v00 + v11], axis=-1)


def quantize_int8_pauli(w: np.ndarray) -> tuple[np.ndarray, np.ndarray]:
    """Symmetric per-output-channel int8 of the weights' matrix entries (format 5).

    ``w``: (..., d_out, d_in, 8) blade order.  Per output channel ``j``:
    ``s = max(max |entries of W_j.|, 1e-12) / 127`` (float64, stored fp32) and
    ``q = clip(rint(entries / s), -127, 127)`` -- the conventions of
    :func:`quantize_int8` (``grade_quantize.py:85-117,198-203``) applied in the
    matrix basis.  Returns ``q`` (..., d_out, d_in, 8) int8 in entry order and ``s``.
    """
    p = pauli_entries(w)
    absmax = np.max(np.abs(p), axis=(-2, -1))
    s = (np.maximum(absmax, 1e-12) / 127.0).astype(F32)
    q = np.clip(np.rint(p / s.astype(np.float64)[..., None, None]), -127, 127).astype(np.int8)
    return q, s


def dequantize_int8_pauli(q: np.ndarray, s: np.ndarray) -> np.ndarray:
    """The blade-order weights (float64, exact) that format-5 codes ``q`` with scales ``s`` hold."""
    return from_pauli_entries(q.astype(np.float64) * s.astype(np.float64)[..., None, None])
