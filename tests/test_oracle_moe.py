"""Pins of the QMoE oracle (oracle/moe.py) on the CPU.

* explicit upstream outputs: the top-1 tie case ([16, 32], tolerance 0), the
  zero-intermediate case (exact zeros) and the empty-token case
  (kernels/_provenance/upstream/com.microsoft.QMoE/build/webgpu/test.json);
* ``expert_weights`` against an element-by-element loop over the shader's
  ``expertWeight`` formula, and against the independently pinned MatMulNBits
  dequantisation with the midpoint zero point (same low-first layout);
* routing against a sort by (logit, expert index) descending with ties;
* ReLU experts against two chained MatMulNBits products (k = 1, one expert);
* SwiGLU wiring (gate rows 2j, linear rows 2j + 1, alpha/beta placement, the
  limit clamps) on weights whose projections are known integers.
"""
import math

import numpy as np
import pytest

from oracle import moe as Q
from oracle import oracle as O
from tests import fixture_util as F

OP = "com.microsoft.QMoE"


def _attrs(case):
    a = case["attrs"]
    return dict(k=a.get("k", 1), activation=a.get("activation_type", "relu"), swiglu_fusion=a.get("swiglu_fusion", 0),
                bits=a.get("expert_weight_bits", 4), block_size=a.get("block_size", 0),
                alpha=a.get("activation_alpha", 1.0), beta=a.get("activation_beta", 0.0),
                swiglu_limit=a.get("swiglu_limit"))


def run_case(case, substitute=False):
    i = F.case_inputs(case, substitute)
    return Q.qmoe(i["inputT"], i["routerT"], i["fc1T"], i["fc1ScalesT"], i["fc2T"], i["fc2ScalesT"], **_attrs(case))


@pytest.mark.parametrize("name", ["q4_top1_tie_selects_higher_expert", "q4_zero_inter", "empty_zero_dim"])
def test_explicit_outputs(name):
    case = F.find(OP, name)
    want = F.materialize(case["outputs"]["outputT"])
    got = run_case(case)
    atol, rtol = F.case_tolerance(case, "outputT")
    assert got.shape == want.shape
    assert F.reference_compare(got, want, atol, rtol)


def test_tie_selects_higher_expert_exactly():
    got = run_case(F.find(OP, "q4_top1_tie_selects_higher_expert"))
    assert np.array_equal(got, np.array([[16.0, 32.0]], np.float32))


@pytest.mark.parametrize("bits,block", [(4, 0), (4, 16), (8, 0), (8, 32)])
def test_expert_weights_elementwise(bits, block):
    rng = np.random.default_rng(bits + block)
    E, rows, cols = 2, 5, 64
    packed = rng.integers(0, 256, (E, rows, cols * bits // 8), dtype=np.uint8)
    scales = rng.uniform(0.01, 0.3, (E, rows, cols // block) if block else (E, rows)).astype(np.float32)
    W = Q.expert_weights(packed, scales, rows, cols, bits, block)
    per_row = scales.size // (E * rows)
    flat_s = scales.reshape(-1)
    for e in range(E):
        for r in range(rows):
            for c in range(cols):
                byte = int(packed[e, r, (c * bits) // 8])
                q = (byte >> ((c * bits) % 8)) & ((1 << bits) - 1)
                si = (e * rows + r) * per_row + (c // max(1, block) if per_row > 1 else 0)
                want = np.float32(np.float32(q) - np.float32(1 << (bits - 1))) * flat_s[si]
                assert W[e, r, c] == np.float32(want)


@pytest.mark.parametrize("bits,block", [(4, 16), (4, 0), (8, 32)])
def test_expert_weights_match_matmul_nbits_dequantisation(bits, block):
    rng = np.random.default_rng(7 * bits + block)
    E, rows, cols = 3, 6, 96
    packed = rng.integers(0, 256, (E, rows, cols * bits // 8), dtype=np.uint8)
    bs = block or cols
    scales = rng.uniform(0.01, 0.3, (E, rows, cols // bs)).astype(np.float32)
    W = Q.expert_weights(packed, scales if block else scales[:, :, 0], rows, cols, bits, block)
    for e in range(E):
        ref = O.dequantize(packed[e].reshape(rows, cols // bs, bs * bits // 8), scales[e], None, cols, bits, bs)
        assert np.array_equal(W[e], ref)


def _sorted_topk(logits, k):
    out = []
    for row in np.asarray(logits, np.float32):
        order = sorted(range(len(row)), key=lambda e: (float(row[e]), e), reverse=True)
        out.append(set(order[:k]))
    return out


@pytest.mark.parametrize("k", [1, 2, 3])
def test_routing_matches_sort_with_ties(k):
    rng = np.random.default_rng(k)
    logits = rng.integers(-2, 3, (64, 6)).astype(np.float32)  # many ties
    sel, w = Q.route(logits, k)
    for t, want in enumerate(_sorted_topk(logits, k)):
        assert set(np.nonzero(sel[t])[0]) == want
        chosen = sorted(want)
        e = np.exp(logits[t, chosen].astype(np.float64) - logits[t, chosen].max())
        assert np.allclose(w[t, chosen], e / e.sum(), rtol=0, atol=1e-15)
        assert abs(w[t].sum() - 1.0) < 1e-12


def test_relu_expert_is_two_chained_matmuls():
    rng = np.random.default_rng(11)
    T, H, I = 3, 64, 32
    x = rng.standard_normal((T, H)).astype(np.float32)
    fc1 = rng.integers(0, 256, (1, I, H // 2), dtype=np.uint8)
    fc2 = rng.integers(0, 256, (1, H, I // 2), dtype=np.uint8)
    s1 = rng.uniform(0.01, 0.1, (1, I)).astype(np.float32)
    s2 = rng.uniform(0.01, 0.1, (1, H)).astype(np.float32)
    got = Q.qmoe(x, np.zeros((T, 1), np.float32), fc1, s1, fc2, s2)
    h = O.matmul_nbits(x, fc1[0].reshape(I, 1, H // 2), s1[0].reshape(I, 1), K=H, N=I, block_size=H,
                       out_dtype=np.float64)
    y = O.matmul_nbits(np.maximum(h, 0), fc2[0].reshape(H, 1, I // 2), s2[0].reshape(H, 1), K=I, N=H,
                       block_size=I, out_dtype=np.float64)
    assert np.allclose(got, y.astype(np.float32), rtol=1e-6, atol=1e-6)


def test_swiglu_wiring_on_known_projections():
    # One expert, x = e_0: projection row r equals weight (r, col 0) = (q - 8) * 1.
    H, I = 2, 3
    gate_codes, lin_codes = [12, 3, 9], [10, 14, 1]
    fc1 = np.zeros((1, 2 * I, 1), np.uint8)
    for j in range(I):
        fc1[0, 2 * j, 0] = gate_codes[j] | (8 << 4)   # row 2j: gate
        fc1[0, 2 * j + 1, 0] = lin_codes[j] | (8 << 4)  # row 2j + 1: linear
    fc2 = np.full((1, H, 2), 0x88, np.uint8)
    fc2[0, 0, 0] = 9 | (9 << 4)   # output 0 = sum of h[0] + h[1]
    fc2[0, 0, 1] = 9 | (8 << 4)   # + h[2]
    s1 = np.ones((1, 2 * I), np.float32)
    s2 = np.ones((1, H), np.float32)
    x = np.array([[1.0, 0.0]], np.float32)
    alpha, beta, lim = 1.5, 0.25, 2.5
    got = Q.qmoe(x, np.zeros((1, 1), np.float32), fc1, s1, fc2, s2, activation="swiglu", swiglu_fusion=1,
                 alpha=alpha, beta=beta, swiglu_limit=lim)
    h = []
    for j in range(I):
        g = min(float(gate_codes[j] - 8), lim)
        lin = max(-lim, min(float(lin_codes[j] - 8), lim))
        h.append(g / (1 + math.exp(-alpha * g)) * (lin + beta))
    assert got[0, 0] == pytest.approx(sum(h), rel=1e-6)
    assert got[0, 1] == 0.0
