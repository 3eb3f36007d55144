"""Seeded synthetic inputs for the five MatMulNBits-family workloads.

Every workload draws from ``numpy.random.default_rng(seed)`` in a fixed order
so the benchmark, the GPU tests and the CPU baseline see identical bytes.
Packed weights are uniform random bytes (both nibbles independent and uniform
on 0..15); scales are U(0.001, 0.02); activations N(0, 1).

=====================  =====================================================
name                   shape
=====================  =====================================================
``cpu_f32_k2048``      MatMulNBits f32, M=1, K=N=2048, bs=32, packed zp, seed 0
``decode_up_m1``       MatMulNBits f16, M=1, K=4096, N=14336, bs=32, no zp, seed 1
                       (Llama-3-8B FFN up-projection decode GEMV)
``qkv_gqa_m4``         MatMulNBitsQkv f16, M=4, K=4096, Nq=4096, Nkv=1024,
                       bs=64, packed zp, gamma=1, eps=1e-6, seed 2
``mlp_swiglu_m16``     MatMulNBitsMlp f16, M=16, K=4096, N=14336, bs=32,
                       silu(gate)*up, no zp/bias/norm, seed 3
``prefill_m2048``      MatMulNBits f16, M=2048, K=4096, N=14336, bs=128,
                       packed zp, bias N(0, 0.01), seed 4
=====================  =====================================================
"""
from __future__ import annotations

import numpy as np

WORKLOADS = ("cpu_f32_k2048", "decode_up_m1", "qkv_gqa_m4", "mlp_swiglu_m16", "prefill_m2048")


def _packed(rng, n, kb, blob):
    return rng.integers(0, 256, size=(n, kb, blob), dtype=np.uint8)


def _scales(rng, shape, dtype):
    return rng.uniform(0.001, 0.02, size=shape).astype(dtype)


def make(name: str, scale_down: int = 1) -> dict:
    """Inputs and attributes for a workload.

    ``scale_down`` divides N (and M for the prefill workload) so tests can run
    the same generator at a size the CPU oracle finishes in seconds.
    """
    if name == "cpu_f32_k2048":
        rng = np.random.default_rng(0)
        K, N, bs = 2048, 2048 // scale_down, 32
        kb = K // bs
        A = rng.standard_normal((1, K)).astype(np.float32)
        B = _packed(rng, N, kb, bs // 2)
        S = _scales(rng, (N, kb), np.float32)
        Z = rng.integers(0, 256, size=(N, (kb + 1) // 2), dtype=np.uint8)
        return dict(op="com.microsoft.MatMulNBits", inputs=dict(aT=A, bT=B, scalesT=S, zeroPointsT=Z),
                    attrs=dict(K=K, N=N, bits=4, block_size=bs))
    if name == "decode_up_m1":
        rng = np.random.default_rng(1)
        K, N, bs = 4096, 14336 // scale_down, 32
        kb = K // bs
        A = rng.standard_normal((1, K)).astype(np.float16)
        B = _packed(rng, N, kb, bs // 2)
        S = _scales(rng, (N, kb), np.float16)
        return dict(op="com.microsoft.MatMulNBits", inputs=dict(aT=A, bT=B, scalesT=S),
                    attrs=dict(K=K, N=N, bits=4, block_size=bs))
    if name == "qkv_gqa_m4":
        rng = np.random.default_rng(2)
        K, Nq, Nkv, bs = 4096, 4096 // scale_down, 1024 // scale_down, 64
        kb = K // bs
        A = rng.standard_normal((4, K)).astype(np.float16)
        gamma = np.ones(K, np.float16)
        ins = dict(aT=A, normScaleT=gamma)
        for p, n in (("q", Nq), ("k", Nkv), ("v", Nkv)):
            ins[p + "BT"] = _packed(rng, n, kb, bs // 2)
            ins[p + "ScalesT"] = _scales(rng, (n, kb), np.float16)
            ins[p + "ZeroPointsT"] = rng.integers(0, 256, size=(n, (kb + 1) // 2), dtype=np.uint8)
        return dict(op="com.microsoft.MatMulNBitsQkv", inputs=ins,
                    attrs=dict(K=K, Nq=Nq, Nkv=Nkv, bits=4, block_size=bs, epsilon=1e-6))
    if name == "mlp_swiglu_m16":
        rng = np.random.default_rng(3)
        K, N, bs = 4096, 14336 // scale_down, 32
        kb = K // bs
        A = rng.standard_normal((16, K)).astype(np.float16)
        ins = dict(aT=A)
        for p in ("gate", "up"):
            ins[p + "BT"] = _packed(rng, N, kb, bs // 2)
            ins[p + "ScalesT"] = _scales(rng, (N, kb), np.float16)
        return dict(op="com.microsoft.MatMulNBitsMlp", inputs=ins,
                    attrs=dict(K=K, N=N, bits=4, block_size=bs, activation="silu"))
    if name == "prefill_m2048":
        rng = np.random.default_rng(4)
        M, K, N, bs = 2048 // scale_down, 4096, 14336 // scale_down, 128
        kb = K // bs
        A = rng.standard_normal((M, K)).astype(np.float16)
        B = _packed(rng, N, kb, bs // 2)
        S = _scales(rng, (N, kb), np.float16)
        Z = rng.integers(0, 256, size=(N, (kb + 1) // 2), dtype=np.uint8)
        bias = (rng.standard_normal(N) * 0.01).astype(np.float16)
        return dict(op="com.microsoft.MatMulNBits", inputs=dict(aT=A, bT=B, scalesT=S, zeroPointsT=Z, biasT=bias),
                    attrs=dict(K=K, N=N, bits=4, block_size=bs))
    raise KeyError(name)


def algorithmic_bytes(w: dict) -> int:
    """Bytes each tensor contributes when read or written once (inputs + outputs)."""
    total = sum(int(np.asarray(v).nbytes) for v in w["inputs"].values())
    a = w["inputs"]["aT"]
    rows = a.size // a.shape[-1]
    item = a.dtype.itemsize
    at = w["attrs"]
    if w["op"] == "com.microsoft.MatMulNBitsQkv":
        total += rows * (at["Nq"] + 2 * at["Nkv"]) * item
    else:
        total += rows * at["N"] * item
    return total


def flops(w: dict) -> int:
    a = w["inputs"]["aT"]
    rows = a.size // a.shape[-1]
    at = w["attrs"]
    if w["op"] == "com.microsoft.MatMulNBitsQkv":
        n = at["Nq"] + 2 * at["Nkv"]
    elif w["op"] == "com.microsoft.MatMulNBitsMlp":
        n = 2 * at["N"]
    else:
        n = at["N"]
    return 2 * rows * at["K"] * n
