"""NumPy oracle for com.microsoft.QMoE, opcode 1030 (test infrastructure only).

This module is the oracle, test infrastructure and never the product: only ``tests/``,
``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline`` may import it.

It restates, on the CPU, the arithmetic of xrGPU's serial Vulkan shader for the
quantized mixture of experts:

* ``expertWeight`` kernels/_shared/extended/shaders/complex_kernel.glsl:158
  (codes low-first within a byte, ``(float(q) - 2^(bits-1)) * scale`` in
  float32, ``scalesPerRow = size(scales) / (experts * rows)`` with the block
  ``col / block_size`` when a row has several scales);
* ``expertRank`` complex_kernel.glsl:159 (an expert's rank counts the experts
  with a larger logit, or an equal logit and a larger index);
* ``moe`` complex_kernel.glsl:160 (softmax over the top-k experts only; FC1
  rows ``2j`` / ``2j + 1`` for interleaved SwiGLU, ``j`` for ReLU; SwiGLU
  ``gate * logistic(alpha * gate) * (linear + beta)`` with the optional
  ``swiglu_limit`` clamps; experts summed in ascending index order);
* planner defaults and checks kernels/_shared/extended/complex_plan.cpp:121-128
  (k 1, bits 4, block_size 0, activation relu, alpha 1, beta 0).

Sums are float64, rounded once to float32 (the reference sums serially in
float32). Pins: ``tests/test_oracle_moe.py``.
"""
from __future__ import annotations

import numpy as np

from .oracle import logistic

ACT_RELU = 1
ACT_SWIGLU = 6


def expert_weights(packed, scales, rows: int, cols: int, bits: int, block_size: int) -> np.ndarray:
    """``expertWeight`` for every (expert, row, col): float32 ``[E, rows, cols]``."""
    packed = np.asarray(packed, dtype=np.uint8)
    experts = packed.shape[0]
    if rows == 0 or cols == 0:
        return np.zeros((experts, rows, cols), np.float32)
    per_byte = 8 // bits
    flat = packed.reshape(experts, rows, -1)
    shifts = (np.arange(cols) * bits) % 8
    byte_idx = (np.arange(cols) * bits) // 8
    q = (flat[:, :, byte_idx].astype(np.uint32) >> shifts.astype(np.uint32)) & ((1 << bits) - 1)
    assert per_byte * flat.shape[2] >= cols
    value = q.astype(np.float32) - np.float32(1 << (bits - 1))
    s = np.asarray(scales, dtype=np.float32).reshape(experts, rows, -1)
    per_row = s.shape[2]
    idx = (np.arange(cols) // max(1, block_size)) if per_row > 1 else np.zeros(cols, np.int64)
    return (value * s[:, :, idx]).astype(np.float32)  # one float32 rounding per weight


def expert_rank(logits: np.ndarray) -> np.ndarray:
    """``expertRank``: rank[t, e] = #{e2: l[t,e2] > l[t,e] or (l[t,e2] == l[t,e] and e2 > e)}."""
    l = np.asarray(logits, dtype=np.float32)
    T, E = l.shape
    a = l[:, None, :]   # other (e2)
    b = l[:, :, None]   # this (e)
    e2 = np.arange(E)[None, None, :]
    e1 = np.arange(E)[None, :, None]
    return np.sum((a > b) | ((a == b) & (e2 > e1)), axis=2)


def route(logits, k: int):
    """Selected mask [T, E] and softmax weights over the selected experts (float64)."""
    l = np.asarray(logits, dtype=np.float32).astype(np.float64)
    sel = expert_rank(logits) < k
    masked = np.where(sel, l, -np.inf)
    mx = masked.max(axis=1, keepdims=True) if l.size else np.zeros((l.shape[0], 1))
    e = np.where(sel, np.exp(l - mx), 0.0)
    den = e.sum(axis=1, keepdims=True)
    return sel, e / np.where(den == 0, 1, den)


def qmoe(x, router, fc1, fc1_scales, fc2, fc2_scales, *, k: int = 1, activation: str = "relu",
         swiglu_fusion: int = 0, bits: int = 4, block_size: int = 0, alpha: float = 1.0,
         beta: float = 0.0, swiglu_limit=None) -> np.ndarray:
    """com.microsoft.QMoE forward, output float32 of ``x``'s shape."""
    x = np.asarray(x, dtype=np.float32)
    shape = x.shape
    H = shape[-1]
    xr = x.reshape(-1, H).astype(np.float64)
    E = np.asarray(router).shape[1]
    F1 = np.asarray(fc1).shape[1]
    act = ACT_SWIGLU if activation == "swiglu" else ACT_RELU
    fusion = 2 if (act == ACT_SWIGLU and swiglu_fusion) else 1
    inter = F1 // fusion
    fc1 = np.asarray(fc1, np.uint8)
    fc2 = np.asarray(fc2, np.uint8)
    s1 = np.asarray(fc1_scales, np.float32)
    s2 = np.asarray(fc2_scales, np.float32)
    cache = {}

    def weights(e):  # dequantised per selected expert only (bounded memory)
        if e not in cache:
            cache[e] = (expert_weights(fc1[e:e + 1], s1[e:e + 1], F1, H, bits, block_size)[0].astype(np.float64),
                        expert_weights(fc2[e:e + 1], s2[e:e + 1], H, inter, bits, block_size)[0].astype(np.float64))
        return cache[e]
    sel, w = route(router, k)
    a = np.float64(np.float32(alpha))
    bta = np.float64(np.float32(beta))
    out = np.zeros_like(xr)
    for t in range(xr.shape[0]):
        for e in range(E):  # ascending expert index, as the shader
            if not sel[t, e]:
                continue
            W1e, W2e = weights(e)
            proj = W1e @ xr[t]
            if act == ACT_SWIGLU:
                gate = proj[0::2] if fusion == 2 else proj[:inter]
                lin = proj[1::2] if fusion == 2 else np.zeros(inter)
                if swiglu_limit is not None:
                    lim = np.float64(np.float32(swiglu_limit))
                    gate = np.minimum(gate, lim)
                    lin = np.clip(lin, -lim, lim)
                h = gate * logistic(a * gate) * (lin + bta)
            else:
                h = np.maximum(proj[:inter], 0.0)
            out[t] += w[t, e] * (W2e @ h)
    return out.astype(np.float32).reshape(shape)
