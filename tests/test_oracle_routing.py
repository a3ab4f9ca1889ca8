"""Pin the oracle's routing rule, dispatch plan, combine and int8 quantizer by brute force."""

import itertools

import numpy as np
import pytest

from oracle import moe


def brute_topk(probs_row, k):
    """Pick k experts one at a time: highest probability, lowest index on ties."""
    chosen = []
    for _ in range(k):
        best = None
        for e, p in enumerate(probs_row):
            if e in chosen:
                continue
            if best is None or p > probs_row[best]:
                best = e
        chosen.append(best)
    return chosen


@pytest.mark.parametrize("E,k", [(4, 1), (8, 2), (16, 2), (32, 4), (64, 8)])
def test_route_topk_brute_force_with_ties(E, k):
    r = np.random.default_rng(E * 10 + k)
    # few distinct values -> many exact ties
    probs = r.integers(0, 4, size=(300, E)).astype(np.float32) / 4
    idx, _ = moe.route_topk(probs, k)
    for t in range(probs.shape[0]):
        assert list(idx[t]) == brute_topk(probs[t], k)


def test_route_weights_renormalised_in_ascending_probability_order():
    r = np.random.default_rng(11)
    probs = moe.softmax(r.standard_normal((500, 16), dtype=np.float32))
    idx, w = moe.route_topk(probs, 4)
    for t in range(0, 500, 7):
        sel = probs[t, idx[t]]
        s = np.float32(0)
        for v in sel[::-1]:
            s = np.float32(s + v)
        assert np.array_equal(w[t], (sel / (s + np.float32(1e-12))).astype(np.float32))


def test_tie_rule_differs_from_stable_ascending_argsort():
    # Documented divergence: with a stable ascending sort, the reference's
    # "last k" would keep the HIGHER index of a tie at the k-th place.
    probs = np.array([[0.25, 0.25, 0.25, 0.25]], np.float32)
    idx, _ = moe.route_topk(probs, 2)
    assert list(idx[0]) == [0, 1]
    assert list(np.argsort(probs[0], kind="stable")[-2:]) == [2, 3]


@pytest.mark.parametrize("N,E,k", [(1, 1, 1), (37, 5, 2), (200, 16, 4), (64, 32, 2)])
def test_dispatch_plan_brute_force(N, E, k):
    r = np.random.default_rng(N + E + k)
    idx = np.stack([r.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    counts, offsets, perm, slot_pos = moe.dispatch_plan(idx, E)
    rows = []
    for e in range(E):  # the reference's loop order: expert, then token
        for t in range(N):
            for s in range(k):
                if idx[t, s] == e:
                    rows.append((e, t, s))
    assert counts.sum() == N * k and offsets[-1] == N * k
    for p, (e, t, s) in enumerate(rows):
        assert perm[p] == t and slot_pos[t, s] == p
        assert offsets[e] <= p < offsets[e + 1]


def test_combine_brute_force_order():
    r = np.random.default_rng(12)
    N, E, k = 50, 8, 3
    idx = np.stack([r.permutation(E)[:k] for _ in range(N)]).astype(np.int32)
    w = r.random((N, k)).astype(np.float32)
    _, _, perm, slot_pos = moe.dispatch_plan(idx, E)
    y = r.standard_normal((N * k, 4, 8)).astype(np.float32)
    out = moe.combine(y, idx, w, slot_pos)
    for t in range(N):
        acc = np.zeros((4, 8), np.float32)
        for s in np.argsort(idx[t]):
            acc = (acc + (w[t, s] * y[slot_pos[t, s]]).astype(np.float32)).astype(np.float32)
        assert np.array_equal(out[t], acc)
    # identity expert: combine of dispatched rows is the convex mix of the token itself
    x = r.standard_normal((N, 4, 8)).astype(np.float32)
    wn = w / w.sum(1, keepdims=True)
    out = moe.combine(x[perm], idx, wn.astype(np.float32), slot_pos)
    assert np.allclose(out, x, rtol=1e-5, atol=1e-6)


def test_quantize_int8_invariants():
    r = np.random.default_rng(13)
    w = r.standard_normal((3, 6, 5, 8)).astype(np.float32)
    w[1, 2] = 0  # an all-zero output channel
    q, s = moe.quantize_int8(w)
    assert q.dtype == np.int8 and s.shape == (3, 6)
    assert np.abs(q.astype(int)).max() <= 127
    assert (np.abs(q.astype(int)).max(axis=(-2, -1))[s > 1e-10] == 127).all()
    deq = moe.dequantize_int8(q, s)
    assert (np.abs(deq - w) <= s[..., None, None] * 0.5 + 1e-7).all()
    assert (q[1, 2] == 0).all()
    # exact on multiples of the scale
    w2 = (np.arange(-127, 128, dtype=np.float32) * np.float32(0.01)).reshape(1, 1, -1, 1).repeat(8, -1)
    q2, s2 = moe.quantize_int8(w2)
    assert np.array_equal(q2[0, 0, :, 0], np.arange(-127, 128))


def test_quantize_int8_pauli_invariants():
    """Format 5: codes in range, the channel's largest entry at +-127, half-step error on the
    matrix entries, the dequantized blade weights within the step of the weights, exact on
    multiples of the scale, zero channels zero."""
    r = np.random.default_rng(17)
    w = r.standard_normal((3, 6, 5, 8)).astype(np.float32)
    w[2, 4] = 0
    q, s = moe.quantize_int8_pauli(w)
    assert q.dtype == np.int8 and q.shape == w.shape and s.shape == (3, 6) and s.dtype == np.float32
    assert np.abs(q.astype(int)).max() <= 127
    assert (np.abs(q.astype(int)).max(axis=(-2, -1))[s > 1e-10] == 127).all()
    p = moe.pauli_entries(w)
    assert (np.abs(q * s.astype(np.float64)[..., None, None] - p) <= s[..., None, None] * 0.5 + 1e-12).all()
    # the scale is the channel's largest entry over 127, entries being sums of two blades
    assert np.array_equal(s, (np.abs(p).max(axis=(-2, -1)) / 127.0).clip(1e-12 / 127.0).astype(np.float32))
    deq = moe.dequantize_int8_pauli(q, s)
    assert (np.abs(deq - w) <= s[..., None, None] * 0.5 + 1e-7).all()
    assert (q[2, 4] == 0).all()
    # exact on multiples of the scale: weights whose entries are integers times 0.01
    codes = r.integers(-127, 128, size=(1, 2, 7, 8))
    codes[0, :, 0, 0] = 127  # pin each channel's scale to 0.01
    wq = moe.from_pauli_entries(codes * 0.01)
    q3, s3 = moe.quantize_int8_pauli(wq)
    assert np.array_equal(q3, codes) and np.array_equal(s3, np.full((1, 2), 0.01, np.float32))
