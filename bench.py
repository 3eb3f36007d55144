"""Benchmark of the MatMulNBits hot path on one MI355X.

Headline (``value``): achieved HBM GB/s of the int4 dequant-GEMV of the
Llama-3-8B FFN up-projection decode (MatMulNBits fp16, M=1, K=4096, N=14336,
block_size=32, no zero points). A step is one operator call on one batch of
synthetic input that is already resident in HBM. Weight replicas rotate so the
working set (>= 10 x 33 MB) exceeds the 256 MB Infinity Cache and every step
reads its weights from HBM.

The same JSON line also carries the prefill GEMM (M=2048, K=4096, N=14336,
block_size=128, packed zero points, bias) in TFLOP/s, the fused Qkv and Mlp
decode workloads in GB/s, the roofline of the dominant kernel and the CPU
baseline (the NumPy oracle on this host's cores, a bounded sample).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0       # MI355X HBM3E, published
FP16_PEAK_TFLOPS = 2500.0   # MI355X dense fp16 MFMA, published
PROFILES = os.path.join(ROOT, "profiles")
SEEDS = {"decode_up_m1": 1, "qkv_gqa_m4": 2, "mlp_swiglu_m16": 3, "prefill_m2048": 4, "qmoe_mixtral_t1": 6,
         "bnb4_nf4_m1": 7, "gbq_embed_t2048": 8, "int8a_decode_m1": 1, "f32_k2048_m1": 0,
         "mlp_prefill_m64": 9, "prefill_m2048_prepacked": 4, "down_proj_m64": 10, "mlp_prefill_m2048": 13,
         "qkv_prefill_m2048": 14, "q8_f32_decode_m1": 15, "f32_prefill_m64": 16, "qmoe_prefill_t256": 17,
         "q8_f16_decode_m1": 18, "f32_prefill_m512": 19, "q2_f16_prefill_m128": 20, "f32_qkv_decode_m1": 21,
         "f32_mlp_prefill_m64": 22}
# The CPU-oracle workload on the GPU: MatMulNBits float32, M=1, K=N=2048,
# block_size 32, packed zero points (2,703,360 algorithmic bytes per call)
F32 = dict(M=1, K=2048, N=2048, bs=32)
# MatMulNBitsMlp prefill: 64 rows, K=2048, N=5632 (the TinyLlama-1.1B FFN),
# block_size 32, normScale, SiLU; 2*2*M*K*N flops per call
MLP64 = dict(M=64, K=2048, N=5632, bs=32)
# MatMulNBits with float32 activations and 8-bit codes: the upstream
# qwen3-qproj-decode-m1-q8g32 case (M=1, K=2560, N=4096, block_size 32, float32
# scales)
Q8F32 = dict(M=1, K=2560, N=4096, bs=32, bits=8)
# float32 MatMulNBits for 64 rows (K=N=4096, block_size 32, 4-bit codes)
F32P = dict(M=64, K=4096, N=4096, bs=32, bits=4)
# float32 MatMulNBits prefill: the upstream qwen3-qproj-prefill-m512-q4g64 case
# (M=512, K=2560, N=4096, block_size 64, float32 scales)
F32P512 = dict(M=512, K=2560, N=4096, bs=64, bits=4)
# float16 MatMulNBits prefill with 2-bit codes: the upstream
# bonsai2-ffn-gate-prefill-m128-q2g128-k5120-n17408 case (block_size 128)
Q2F16 = dict(M=128, K=5120, N=17408, bs=128, bits=2)
# the MatMulNBits legs with float32 arithmetic (float32 activations, or
# float16 with 2- or 8-bit codes)
# float32 MatMulNBitsQkv decode and MatMulNBitsMlp prefill: the upstream
# qkv-q4-llama-decode-k4096-nq4096-nkv4096 and mlp-q4-prefill-m64-k2048-n5632
# cases (float32 activations, scales and outputs, block_size 32, normScale;
# Mlp SiLU)
F32QKV = dict(M=1, K=4096, Nq=4096, Nkv=4096, bs=32)
F32MLP = dict(M=64, K=2048, N=5632, bs=32)
WIDE_LEGS = {"q8_f32_decode_m1": Q8F32, "q8_f16_decode_m1": Q8F32, "f32_prefill_m64": F32P, "f32_prefill_m512": F32P512,
             "q2_f16_prefill_m128": Q2F16}
# MatMulNBitsMlp prefill of the Llama-3-8B FFN: 2048 rows, K=4096, N=14336,
# block_size 32, normScale, SiLU (gate and up: 2*2*M*K*N flops per call)
MLP2K = dict(M=2048, K=4096, N=14336, bs=32)
# MatMulNBitsQkv prefill, the GQA layout: 2048 rows, K=4096, Nq=4096,
# Nkv=1024, block_size 64, packed zero points, normScale
QKV2K = dict(M=2048, K=4096, Nq=4096, Nkv=1024, bs=64)
# MatMulNBits down projection of the Llama-3-8B FFN for 64 tokens (K=14336,
# N=4096, block_size 32, packed zero points): 32 output tiles for 256 CUs, the
# split-K GEMM's case
DOWN64 = dict(M=64, K=14336, N=4096, bs=32)
# com.microsoft.MatMulBnb4 decode: the FFN up-projection shape in NF4, blocks of 64
BNB4 = dict(M=1, K=4096, N=14336, bs=64)
# com.microsoft.GatherBlockQuantized: a 128256 x 4096 4-bit embedding table
# (blocks of 32, float32 scales) gathered for 2048 tokens
GBQ = dict(rows=128256, width=4096, bs=32, n=2048)
# com.microsoft.QMoE decode, Mixtral-8x7B expert geometry: T=1, H=4096, I=14336,
# E=8, k=2, 4-bit codes, float32 scales per block of 64, interleaved SwiGLU
QMOE = dict(T=1, H=4096, I=14336, E=8, k=2, bits=4, bs=64)
# com.microsoft.QMoE prefill, the same expert geometry for 256 tokens with
# float32 scales per row (block_size 0): the grouped-expert GEMMs,
# 2 * T * k * 3 * H * I flops per call
QMOE_PF = dict(T=256, H=4096, I=14336, E=8, k=2, bits=4, bs=0)


def qmoe_algorithmic_bytes(T=1, H=4096, I=14336, k=2, bits=4, bs=64, **_):
    """Bytes one call must move: the k selected experts' codes and scales of
    FC1 (2I x H) and FC2 (H x I), the activations, the router row and the
    output (the float32 intermediate h is the implementation's own)."""
    fc1 = 2 * I * H * bits // 8 + 2 * I * (H // bs) * 4
    fc2 = H * I * bits // 8 + H * (I // bs) * 4
    return k * (fc1 + fc2) + T * (2 * H * 4 + QMOE["E"] * 4)


def _gen_weights(torch, g, n, kb, blob, dev):
    return torch.randint(0, 256, (n, kb, blob), dtype=torch.uint8, device=dev, generator=g)


def _scales(torch, g, shape, dev):
    return (torch.rand(shape, device=dev, generator=g) * 0.019 + 0.001).half()


def make_replicas(torch, name, R, dev, seed):
    """R independent weight sets of a workload, generated on the device."""
    g = torch.Generator(device=dev)
    g.manual_seed(seed)
    reps = []
    if name in ("decode_up_m1", "int8a_decode_m1"):
        K, N, bs = 4096, 14336, 32
        A = torch.randn((1, K), device=dev, generator=g).half()
        for _ in range(R):
            reps.append(dict(B=_gen_weights(torch, g, N, K // bs, bs // 2, dev), S=_scales(torch, g, (N, K // bs), dev)))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs)
    if name == "f32_k2048_m1":
        q = F32
        K, N, bs = q["K"], q["N"], q["bs"]
        kb = K // bs
        A = torch.randn((q["M"], K), device=dev, generator=g)
        for _ in range(R):
            reps.append(dict(B=_gen_weights(torch, g, N, kb, bs // 2, dev),
                             S=torch.rand((N, kb), device=dev, generator=g) * 0.019 + 0.001,
                             Z=torch.randint(0, 256, (N, (kb + 1) // 2), dtype=torch.uint8, device=dev, generator=g)))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs)
    if name in ("prefill_m2048", "prefill_m2048_prepacked"):
        M, K, N, bs = 2048, 4096, 14336, 128
        kb = K // bs
        A = torch.randn((M, K), device=dev, generator=g).half()
        for _ in range(R):
            reps.append(dict(B=_gen_weights(torch, g, N, kb, bs // 2, dev), S=_scales(torch, g, (N, kb), dev),
                             Z=torch.randint(0, 256, (N, (kb + 1) // 2), dtype=torch.uint8, device=dev, generator=g),
                             bias=(torch.randn(N, device=dev, generator=g) * 0.01).half()))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs, M=M)
    if name == "qkv_gqa_m4":
        K, Nq, Nkv, bs = 4096, 4096, 1024, 64
        kb = K // bs
        A = torch.randn((4, K), device=dev, generator=g).half()
        gamma = torch.ones(K, device=dev).half()
        for _ in range(R):
            r = {}
            for p, n in (("q", Nq), ("k", Nkv), ("v", Nkv)):
                r[p + "B"] = _gen_weights(torch, g, n, kb, bs // 2, dev)
                r[p + "S"] = _scales(torch, g, (n, kb), dev)
                r[p + "Z"] = torch.randint(0, 256, (n, (kb + 1) // 2), dtype=torch.uint8, device=dev, generator=g)
            reps.append(r)
        return dict(A=A, gamma=gamma, reps=reps, K=K, Nq=Nq, Nkv=Nkv, bs=bs)
    if name == "qmoe_mixtral_t1":
        q = QMOE
        H, I, E, bits, bs = q["H"], q["I"], q["E"], q["bits"], q["bs"]
        x = torch.randn((q["T"], H), device=dev, generator=g) * 0.5
        # router rows selecting experts {0,1}, {2,3}, {4,5}, {6,7} with unequal weights
        routers = []
        for j in range(E // 2):
            r = torch.full((q["T"], E), -4.0, device=dev)
            r[:, 2 * j], r[:, 2 * j + 1] = 1.0, 0.25
            routers.append(r)
        for _ in range(R):
            reps.append(dict(
                fc1=torch.randint(0, 256, (E, 2 * I, H * bits // 8), dtype=torch.uint8, device=dev, generator=g),
                s1=torch.rand((E, 2 * I, H // bs), device=dev, generator=g) * 0.019 + 0.001,
                fc2=torch.randint(0, 256, (E, H, I * bits // 8), dtype=torch.uint8, device=dev, generator=g),
                s2=torch.rand((E, H, I // bs), device=dev, generator=g) * 0.019 + 0.001))
        return dict(A=x, routers=routers, reps=reps)
    if name == "qmoe_prefill_t256":
        q = QMOE_PF
        T, H, I, E = q["T"], q["H"], q["I"], q["E"]
        x = torch.randn((T, H), device=dev, generator=g) * 0.5
        router = torch.randn((T, E), device=dev, generator=g)
        for _ in range(R):
            reps.append(dict(
                fc1=torch.randint(0, 256, (E, 2 * I, H // 2), dtype=torch.uint8, device=dev, generator=g),
                s1=torch.rand((E, 2 * I), device=dev, generator=g) * 0.019 + 0.001,
                fc2=torch.randint(0, 256, (E, H, I // 2), dtype=torch.uint8, device=dev, generator=g),
                s2=torch.rand((E, H), device=dev, generator=g) * 0.019 + 0.001))
        return dict(A=x, router=router, reps=reps)
    if name == "bnb4_nf4_m1":
        q = BNB4
        A = torch.randn((q["M"], q["K"]), device=dev, generator=g).half()
        for _ in range(R):
            reps.append(dict(B=torch.randint(0, 256, (q["N"] * q["K"] // 2,), dtype=torch.uint8, device=dev, generator=g),
                             S=(torch.rand(q["N"] * q["K"] // q["bs"], device=dev, generator=g) + 0.05).half()))
        return dict(A=A, reps=reps)
    if name == "gbq_embed_t2048":
        q = GBQ
        data = torch.randint(0, 256, (q["rows"], q["width"] // 2), dtype=torch.uint8, device=dev, generator=g)
        scales = torch.rand((q["rows"], q["width"] // q["bs"]), device=dev, generator=g) * 0.02
        idx = [torch.randint(0, q["rows"], (q["n"],), dtype=torch.int32, device=dev, generator=g) for _ in range(R)]
        return dict(A=data, scales=scales, reps=idx)
    if name == "down_proj_m64":
        q = DOWN64
        K, N, bs = q["K"], q["N"], q["bs"]
        kb = K // bs
        A = torch.randn((q["M"], K), device=dev, generator=g).half()
        for _ in range(R):
            reps.append(dict(B=_gen_weights(torch, g, N, kb, bs // 2, dev), S=_scales(torch, g, (N, kb), dev),
                             Z=torch.randint(0, 256, (N, (kb + 1) // 2), dtype=torch.uint8, device=dev, generator=g)))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs)
    if name == "mlp_prefill_m64":
        q = MLP64
        K, N, bs = q["K"], q["N"], q["bs"]
        A = torch.randn((q["M"], K), device=dev, generator=g).half()
        gamma = (torch.rand((K,), device=dev, generator=g) + 0.5).half()
        for _ in range(R):
            reps.append(dict(gB=_gen_weights(torch, g, N, K // bs, bs // 2, dev), gS=_scales(torch, g, (N, K // bs), dev),
                             uB=_gen_weights(torch, g, N, K // bs, bs // 2, dev), uS=_scales(torch, g, (N, K // bs), dev)))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs, gamma=gamma)
    if name in WIDE_LEGS:
        q = WIDE_LEGS[name]
        dt = torch.float16 if "f16" in name else torch.float32
        K, N, bs, bits = q["K"], q["N"], q["bs"], q["bits"]
        kb = K // bs
        A = torch.randn((q["M"], K), device=dev, generator=g).to(dt)
        for _ in range(R):
            reps.append(dict(B=torch.randint(0, 256, (N, kb, bs * bits // 8), dtype=torch.uint8, device=dev, generator=g),
                             S=(torch.rand((N, kb), device=dev, generator=g) * 0.01 + 0.04).to(dt)))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs, bits=bits)
    if name in ("f32_qkv_decode_m1", "f32_mlp_prefill_m64"):
        q = F32QKV if name == "f32_qkv_decode_m1" else F32MLP
        K, bs = q["K"], q["bs"]
        kb = K // bs
        A = torch.randn((q["M"], K), device=dev, generator=g) * 0.2
        gamma = torch.rand((K,), device=dev, generator=g) + 0.5
        shapes = (("q", q["Nq"]), ("k", q["Nkv"]), ("v", q["Nkv"])) if "qkv" in name else (("g", q["N"]), ("u", q["N"]))
        for _ in range(R):
            r = {}
            for p, n in shapes:
                r[p + "B"] = _gen_weights(torch, g, n, kb, bs // 2, dev)
                r[p + "S"] = _scales(torch, g, (n, kb), dev).float()
            reps.append(r)
        return dict(A=A, reps=reps, K=K, bs=bs, gamma=gamma, q=q)
    if name == "mlp_prefill_m2048":
        q = MLP2K
        K, N, bs = q["K"], q["N"], q["bs"]
        A = torch.randn((q["M"], K), device=dev, generator=g).half()
        gamma = (torch.rand((K,), device=dev, generator=g) + 0.5).half()
        for _ in range(R):
            reps.append(dict(gB=_gen_weights(torch, g, N, K // bs, bs // 2, dev), gS=_scales(torch, g, (N, K // bs), dev),
                             uB=_gen_weights(torch, g, N, K // bs, bs // 2, dev), uS=_scales(torch, g, (N, K // bs), dev)))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs, gamma=gamma)
    if name == "qkv_prefill_m2048":
        q = QKV2K
        K, bs = q["K"], q["bs"]
        kb = K // bs
        A = torch.randn((q["M"], K), device=dev, generator=g).half()
        gamma = (torch.rand((K,), device=dev, generator=g) + 0.5).half()
        for _ in range(R):
            r = {}
            for p, n in (("q", q["Nq"]), ("k", q["Nkv"]), ("v", q["Nkv"])):
                r[p + "B"] = _gen_weights(torch, g, n, kb, bs // 2, dev)
                r[p + "S"] = _scales(torch, g, (n, kb), dev)
                r[p + "Z"] = torch.randint(0, 256, (n, (kb + 1) // 2), dtype=torch.uint8, device=dev, generator=g)
            reps.append(r)
        return dict(A=A, gamma=gamma, reps=reps)
    if name == "mlp_swiglu_m16":
        K, N, bs = 4096, 14336, 32
        A = torch.randn((16, K), device=dev, generator=g).half()
        for _ in range(R):
            reps.append(dict(gB=_gen_weights(torch, g, N, K // bs, bs // 2, dev), gS=_scales(torch, g, (N, K // bs), dev),
                             uB=_gen_weights(torch, g, N, K // bs, bs // 2, dev), uS=_scales(torch, g, (N, K // bs), dev)))
        return dict(A=A, reps=reps, K=K, N=N, bs=bs)
    raise KeyError(name)


def step_fn(ops, name, w):
    """A callable running step i on replica i % R (outputs preallocated)."""
    torch = sys.modules["torch"]
    reps, A = w["reps"], w["A"]
    if name == "decode_up_m1":
        Y = torch.empty((1, w["N"]), dtype=torch.float16, device=A.device)
        return lambda i: ops.matmul_nbits(A, reps[i % len(reps)]["B"], reps[i % len(reps)]["S"], block_size=w["bs"], out=Y)
    if name == "f32_k2048_m1":
        Y = torch.empty((1, w["N"]), dtype=torch.float32, device=A.device)

        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits(A, r["B"], r["S"], r["Z"], block_size=w["bs"], out=Y)
        return f
    if name == "prefill_m2048":
        Y = torch.empty((w["M"], w["N"]), dtype=torch.float16, device=A.device)

        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits(A, r["B"], r["S"], r["Z"], r["bias"], block_size=w["bs"], out=Y)
        return f
    if name == "prefill_m2048_prepacked":
        # the weights are prepacked once, before any timing (the request
        # lifecycle does the same at prepare)
        Y = torch.empty((w["M"], w["N"]), dtype=torch.float16, device=A.device)
        packed = [ops.prepack_weights(r["B"], K=w["K"], block_size=w["bs"]) for r in reps]
        for r in reps:
            del r["B"]

        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits_prepacked(A, packed[i % len(reps)], r["S"], r["Z"], r["bias"], K=w["K"],
                                              N=w["N"], block_size=w["bs"], out=Y)
        return f
    if name == "qkv_gqa_m4":
        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits_qkv(A, r["qB"], r["qS"], r["kB"], r["kS"], r["vB"], r["vS"], norm_scale=w["gamma"],
                                        block_size=w["bs"], q_zero_points=r["qZ"], k_zero_points=r["kZ"],
                                        v_zero_points=r["vZ"], want_residual=False)
        return f
    if name == "down_proj_m64":
        Y = torch.empty((DOWN64["M"], w["N"]), dtype=torch.float16, device=A.device)
        # the split-K workspace, zero-filled once outside the timed graph (a
        # captured call without one runs unsplit)
        ws = torch.zeros(ops.matmul_nbits_workspace_bytes(DOWN64["M"], w["K"], w["N"], 4, w["bs"]), dtype=torch.uint8,
                         device=A.device)

        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits(A, r["B"], r["S"], r["Z"], block_size=w["bs"], out=Y, workspace=ws)
        return f
    if name == "mlp_prefill_m64":
        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits_mlp(A, r["gB"], r["gS"], r["uB"], r["uS"], norm_scale=w["gamma"],
                                        block_size=w["bs"])
        return f
    if name in WIDE_LEGS:
        Y = torch.empty((A.shape[0], w["N"]), dtype=A.dtype, device=A.device)
        # the float32 prefill GEMM's workspace (row exponents), zero-filled once
        # outside the timed graph (a captured call without one takes the GEMV)
        nws = ops.matmul_nbits_workspace_bytes(A.shape[0], w["K"], w["N"], w["bits"], w["bs"], A.dtype)
        ws = torch.zeros(nws, dtype=torch.uint8, device=A.device) if nws else None

        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits(A, r["B"], r["S"], block_size=w["bs"], bits=w["bits"], out=Y, workspace=ws)
        return f
    if name in ("f32_qkv_decode_m1", "f32_mlp_prefill_m64"):
        q = w["q"]
        # the workspace (x, gate / up rows, the projections' GEMM workspace),
        # allocated once outside the timed graph
        if "qkv" in name:
            ws = torch.empty(max(1, ops.fused_workspace_bytes("qkv", q["M"], q["K"], q["Nq"], q["Nkv"], 4, w["bs"],
                                                              torch.float32)), dtype=torch.uint8, device=A.device)

            def f(i):
                r = reps[i % len(reps)]
                return ops.matmul_nbits_qkv(A, r["qB"], r["qS"], r["kB"], r["kS"], r["vB"], r["vS"], norm_scale=w["gamma"],
                                            block_size=w["bs"], want_residual=False, workspace=ws)
        else:
            ws = torch.empty(max(1, ops.fused_workspace_bytes("mlp", q["M"], q["K"], q["N"], 0, 4, w["bs"], torch.float32)),
                             dtype=torch.uint8, device=A.device)

            def f(i):
                r = reps[i % len(reps)]
                return ops.matmul_nbits_mlp(A, r["gB"], r["gS"], r["uB"], r["uS"], norm_scale=w["gamma"],
                                            block_size=w["bs"], workspace=ws)
        return f
    if name == "mlp_prefill_m2048":
        # one workspace for the normalised rows, allocated once (the front end
        # would otherwise take it from torch's caching allocator per call)
        ws = torch.empty(ops.fused_workspace_bytes("mlp", MLP2K["M"], w["K"], w["N"], block_size=w["bs"]),
                         dtype=torch.uint8, device=A.device)

        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits_mlp(A, r["gB"], r["gS"], r["uB"], r["uS"], norm_scale=w["gamma"],
                                        block_size=w["bs"], workspace=ws)
        return f
    if name == "qkv_prefill_m2048":
        q = QKV2K
        ws = torch.empty(ops.fused_workspace_bytes("qkv", q["M"], q["K"], q["Nq"], q["Nkv"], block_size=q["bs"]),
                         dtype=torch.uint8, device=A.device)

        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits_qkv(A, r["qB"], r["qS"], r["kB"], r["kS"], r["vB"], r["vS"], norm_scale=w["gamma"],
                                        block_size=q["bs"], q_zero_points=r["qZ"], k_zero_points=r["kZ"],
                                        v_zero_points=r["vZ"], want_residual=False, workspace=ws)
        return f
    if name == "mlp_swiglu_m16":
        def f(i):
            r = reps[i % len(reps)]
            return ops.matmul_nbits_mlp(A, r["gB"], r["gS"], r["uB"], r["uS"], block_size=w["bs"])
        return f
    if name == "qmoe_mixtral_t1":
        routers, q = w["routers"], QMOE
        ws = torch.empty(ops.qmoe_workspace_bytes(q["T"], q["k"], q["H"], q["I"]), dtype=torch.uint8, device=A.device)

        def f(i):
            # consecutive steps route to disjoint expert pairs of rotating weight
            # sets, so no step finds its experts in the 256 MB Infinity Cache
            r = reps[(i // len(routers)) % len(reps)]
            return ops.qmoe(A, routers[i % len(routers)], r["fc1"], r["s1"], r["fc2"], r["s2"], k=q["k"],
                            activation="swiglu", swiglu_fusion=1, expert_weight_bits=q["bits"], block_size=q["bs"],
                            workspace=ws)
        return f
    if name == "qmoe_prefill_t256":
        q = QMOE_PF
        ws = torch.empty(ops.qmoe_workspace_bytes(q["T"], q["k"], q["H"], q["I"]), dtype=torch.uint8, device=A.device)

        def f(i):
            r = reps[i % len(reps)]
            return ops.qmoe(A, w["router"], r["fc1"], r["s1"], r["fc2"], r["s2"], k=q["k"], activation="swiglu",
                            swiglu_fusion=1, expert_weight_bits=q["bits"], block_size=q["bs"], workspace=ws)
        return f
    if name == "int8a_decode_m1":
        Y = torch.empty((1, w["N"]), dtype=torch.float16, device=A.device)
        ws = torch.empty(ops.int8a_workspace_bytes(1, w["K"]), dtype=torch.uint8, device=A.device)
        return lambda i: ops.matmul_nbits_int8a(A, reps[i % len(reps)]["B"], reps[i % len(reps)]["S"], K=w["K"],
                                                N=w["N"], block_size=w["bs"], out=Y, workspace=ws)
    if name == "bnb4_nf4_m1":
        q = BNB4
        Y = torch.empty((q["M"], q["N"]), dtype=torch.float16, device=A.device)
        return lambda i: ops.matmul_bnb4(A, reps[i % len(reps)]["B"], reps[i % len(reps)]["S"], K=q["K"], N=q["N"],
                                         block_size=q["bs"], quant_type=1, out=Y)
    if name == "gbq_embed_t2048":
        status = torch.zeros(1, dtype=torch.int32, device=A.device)
        return lambda i: ops.gather_block_quantized(A, reps[i % len(reps)], w["scales"], bits=4, block_size=GBQ["bs"],
                                                    status=status, check=False)
    raise KeyError(name)


def time_steps(torch, fn, steps, warmup):
    """Device time per step over K steps with HIP events on the launch stream.

    The K steps are captured once into a HIP graph (torch.cuda.CUDAGraph) and
    the timed region replays it, so back-to-back kernels are not separated by
    the Python/ctypes launch overhead of each call (about 10 us, longer than
    a decode kernel). Every step is still one operator call on its own weight
    replica. Returns (graph ms/step, eager ms/step, host wall ms/call).
    """
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    # eager: event-timed and host-timed, for reference
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record(stream)
    for i in range(steps):
        fn(warmup + i)
    end.record(stream)
    wall = (time.perf_counter() - t0) / steps * 1e3
    torch.cuda.synchronize()
    eager = start.elapsed_time(end) / steps
    # graph of the same K steps
    side = torch.cuda.Stream()
    side.wait_stream(stream)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        with torch.cuda.graph(g, stream=side):
            for i in range(steps):
                fn(i)
    torch.cuda.synchronize()
    # untimed replays for about 100 ms first: a box's first launches run at a
    # lower clock (the decode step measured 8.3 us in a fresh process and
    # 7.7 us in the next one on the same box), and one timed replay of K
    # steps lasts only K x the step time
    t_end = time.perf_counter() + 0.1
    while time.perf_counter() < t_end:
        g.replay()
        torch.cuda.synchronize()
    start.record(stream)
    g.replay()
    end.record(stream)
    torch.cuda.synchronize()
    ms = start.elapsed_time(end) / steps
    del g
    return ms, eager, wall


def per_launch_percentiles(torch, fn, n, warmup):
    """Per-launch event timing (p10/p50/p90 ms); each launch bracketed alone."""
    stream = torch.cuda.current_stream()
    for i in range(warmup):
        fn(i)
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(n)]
    for i, (a, b) in enumerate(ev):
        a.record(stream)
        fn(i)
        b.record(stream)
    torch.cuda.synchronize()
    t = sorted(a.elapsed_time(b) for a, b in ev)
    return t[len(t) // 10], t[len(t) // 2], t[(9 * len(t)) // 10]


def dense_fp16_reference(torch, steps: int = 30):
    """torch.matmul (hipBLASLt) on the prefill shape with dense fp16 weights and
    random data: the vendor library's dense rate, the context for the fused
    dequant GEMM's MFMA fraction (it does no dequantisation)."""
    M, K, N = 2048, 4096, 14336
    g = torch.Generator(device="cuda")
    g.manual_seed(5)
    A = torch.randn((M, K), device="cuda", generator=g).half()
    Ws = [torch.randn((N, K), device="cuda", generator=g).half() for _ in range(2)]
    for i in range(5):
        A @ Ws[i % 2].t()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for i in range(steps):
        A @ Ws[i % 2].t()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / steps
    return {"what": "torch.matmul fp16 (hipBLASLt), same shape, dense fp16 weights, random data, no dequantisation",
            "us": round(ms * 1e3, 1), "tflops": round(2 * M * K * N / (ms * 1e-3) / 1e12, 1)}


def _cpu_model() -> str:
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, runs=5, budget_s=8.0):
    """Median wall time of ``fn`` over up to ``runs`` runs after one warm-up,
    stopping early once ``budget_s`` is spent."""
    import numpy as np
    fn()
    times, t_start = [], time.perf_counter()
    while len(times) < runs and (not times or time.perf_counter() - t_start < budget_s):
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
    return float(np.median(times)), len(times)


def cpu_baseline():
    """The NumPy oracle on this host's cores, three legs per workload (bounded).

    For the decode workload (M=1 K=4096 N=14336, fp16, no zp) and the
    CPU-oracle workload (M=1 K=N=2048, fp32, packed zp): (i) end to end
    (unpack + float32 dequantise + float64 matvec + one rounding), (ii) the
    matvec alone on a pre-dequantised float64 W, (iii) end to end with one BLAS
    thread. ``value`` is leg (i) of the decode workload, the headline's
    workload."""
    import numpy as np
    from oracle import oracle as O
    from xrgpu_amd import workloads
    try:
        from threadpoolctl import threadpool_info, threadpool_limits
        info = threadpool_info()
        threads = max([p.get("num_threads", 1) for p in info] or [1])
        blas = sorted({f"{p.get('internal_api')} {p.get('version')}" for p in info if p.get("user_api") == "blas"})
    except Exception:
        threadpool_limits, threads, blas = None, 1, []
    legs = {}
    for wname in ("decode_up_m1", "cpu_f32_k2048"):
        w = workloads.make(wname)
        i, at = w["inputs"], w["attrs"]
        Z = i.get("zeroPointsT")
        nbytes = workloads.algorithmic_bytes(w)

        def e2e():
            return O.matmul_nbits(i["aT"], i["bT"], i["scalesT"], Z, K=at["K"], N=at["N"], block_size=at["block_size"])
        W = O.dequantize(i["bT"], i["scalesT"], Z, at["K"], 4, at["block_size"]).astype(np.float64)
        x = i["aT"].astype(np.float64)
        t1, n1 = _median_time(e2e)
        t2, n2 = _median_time(lambda: x @ W.T)
        if threadpool_limits is not None:
            with threadpool_limits(limits=1):
                t3, n3 = _median_time(e2e)
        else:
            t3, n3 = t1, n1
        del W
        legs[wname] = {"bytes": nbytes,
                       "end_to_end": {"ms": round(t1 * 1e3, 3), "GBps": round(nbytes / t1 / 1e9, 4), "runs": n1},
                       "matmul_only": {"ms": round(t2 * 1e3, 3), "GBps": round(nbytes / t2 / 1e9, 4), "runs": n2},
                       "one_thread": {"ms": round(t3 * 1e3, 3), "GBps": round(nbytes / t3 / 1e9, 4), "runs": n3}}
    d = legs["decode_up_m1"]["end_to_end"]
    return {"value": d["GBps"], "unit": "GB/s", "cores": int(threads), "kind": "port",
            "sample": f"NumPy oracle (unpack + fp32 dequant + fp64 matvec) on the full decode GEMV M=1 K=4096 "
                      f"N=14336, median of {d['runs']} runs, {d['ms']} ms/call; three legs on it and on the "
                      f"fp32 K=N=2048 workload in 'legs'",
            "legs": legs, "blas": blas, "blas_threads": int(threads), "host_cores": len(os.sched_getaffinity(0)),
            "cpu_model": _cpu_model()}


def stream_ceiling(torch, ops, steps, warmup, nbytes=33_067_008, R=10):
    """The plain read of the decode workload's bytes: R rotating buffers of
    ``nbytes`` (330 MB, beyond the Infinity Cache), one buffer read per step
    by xrmm_stream_read_ex, timed like the decode leg. Swept over the one-shot
    grid (every lane issues 1, 2, 4 or 8 loads and retires) and persistent
    grids of 4 or 8 workgroups per CU walking the buffer, each with
    non-temporal and default-policy loads; the best is the ceiling."""
    g = torch.Generator(device="cuda")
    g.manual_seed(11)
    bufs = [torch.randint(0, 256, (nbytes,), dtype=torch.uint8, device="cuda", generator=g) for _ in range(R)]
    sink = torch.zeros(1, dtype=torch.int32, device="cuda")
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    variants = [("oneshot_nt", u, True, 0) for u in (1, 2, 4, 8)]
    variants += [("oneshot_default", u, False, 0) for u in (1, 4)]
    variants += [(f"persistent{wpc}_{'nt' if nt else 'default'}", u, nt, wpc * cus)
                 for wpc in (4, 8) for nt in (True, False) for u in (2, 4)]
    per = {}
    for kind, u, nt, wg in variants:
        ms, _, _ = time_steps(torch, lambda i, u=u, nt=nt, wg=wg: ops.stream_read(
            bufs[i % R], loads_per_lane=u, sink=sink, nontemporal=nt, workgroups=wg), steps, warmup)
        per[f"{kind}_u{u}"] = ms
    best = min(per, key=per.get)
    ms = per[best]
    del bufs
    torch.cuda.empty_cache()
    return {"what": f"plain 16-byte read of {nbytes} B (the decode GEMV's bytes), {R} rotating buffers, "
                    f"best of one-shot and persistent grids, non-temporal and default loads",
            "us": round(ms * 1e3, 3), "gbs": round(nbytes / (ms * 1e-3) / 1e9, 2),
            "frac_hbm": round(nbytes / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "best": best,
            "us_by_variant": {k: round(v * 1e3, 3) for k, v in per.items()}}


def mfma_ceiling(torch, ops, launches=6, target_ms=2.0):
    """The sustained v_mfma_f32_32x32x16_f16 rate on this box: back-to-back
    MFMAs on random N(0, 1) binary16 operands (a GEMM's switching activity)
    on every CU, swept over 4, 8 and 16 waves per CU and 4 or 8 independent
    accumulators, then the best shape again on all-zero operands. Every wave
    records its loop's shader-clock cycles (s_memtime) and the constant-rate
    counter (s_memrealtime, 100 MHz) at its start and end, which give the
    clock the MFMAs ran at and the MFMA issue interval per SIMD. The
    ceiling is the best random-operand rate."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    nb = ops.mfma_peak_operand_bytes()
    g = torch.Generator(device="cuda")
    g.manual_seed(12)
    rnd = torch.randn(nb // 2, device="cuda", generator=g).half()
    zero = torch.zeros(nb // 2, device="cuda", dtype=torch.float16)

    def run(opnd, wpc, nacc, iters):
        wg, waves = cus * wpc // 4, 4
        clocks = torch.zeros(4 * wg * waves, dtype=torch.int64, device="cuda")
        for _ in range(2):
            ops.mfma_peak(opnd, clocks, workgroups=wg, waves=waves, accumulators=nacc, iters=iters)
        torch.cuda.synchronize()
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(launches):
            ops.mfma_peak(opnd, clocks, workgroups=wg, waves=waves, accumulators=nacc, iters=iters)
        e.record()
        torch.cuda.synchronize()
        ms = s.elapsed_time(e) / launches
        c = clocks.view(-1, 4).double()
        cyc, r0, r1 = c[:, 0], c[:, 1], c[:, 2]
        span = float(r1.max() - r0.min())            # ticks of 10 ns over all waves of the last launch
        sclk = float(cyc.sum() / (r1 - r0).sum()) * 0.1  # GHz: shader cycles per 10 ns tick / 10
        fl = ops.mfma_peak_flops(wg, waves, iters)
        tf = fl / (ms * 1e-3) / 1e12
        mfma_per_simd = wg * waves * 16 * iters / (cus * 4)
        return {"waves_per_cu": wpc, "accumulators": nacc, "iters": iters, "us_per_launch": round(ms * 1e3, 1),
                "tflops": round(tf, 1), "frac_of_2500": round(tf / FP16_PEAK_TFLOPS, 4), "sclk_ghz": round(sclk, 3),
                "wave_span_over_launch": round(span * 1e-5 / ms, 3),
                "mean_wave_loop_over_span": round(float((r1 - r0).mean()) / span, 3),
                "cycles_per_mfma_per_simd": round(span * sclk * 10 / mfma_per_simd, 2)}

    sweep = []
    for wpc in (4, 8, 16):
        for nacc in (4, 8):
            # about target_ms per launch at 1.3 PFLOP/s
            iters = max(64, int(target_ms * 1e-3 * 1.3e15 / (cus * wpc * 16 * 32768)))
            sweep.append(run(rnd, wpc, nacc, iters))
    best = max(sweep, key=lambda r: r["tflops"])
    zero_run = run(zero, best["waves_per_cu"], best["accumulators"], best["iters"])
    del rnd, zero
    return {"mfma": "v_mfma_f32_32x32x16_f16", "operands": "random N(0,1) binary16", "tflops": best["tflops"],
            "frac_of_2500": best["frac_of_2500"], "sclk_ghz": best["sclk_ghz"], "best": best,
            "sweep": sweep, "zero_operands": zero_run}


def copy_calibration():
    """Counter calibration for rocprofv3 byte counters: five device copies of
    256 MiB (each reads and writes exactly 268435456 bytes). Run under
    ``rocprofv3 --pmc FETCH_SIZE`` / ``--pmc WRITE_SIZE``; the copy kernel's
    counter values give the counter-to-bytes factors rocprof_summary uses."""
    import torch
    nbytes = 256 << 20
    x = torch.ones(nbytes // 4, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    for _ in range(5):
        y.copy_(x)
    torch.cuda.synchronize()
    print(f"copy calibration: {nbytes} bytes read and written per dispatch", flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--replicas", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--only", default="")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="only run the rocprofv3 byte-counter calibration copies and exit")
    args = ap.parse_args()
    if args.copy_calibration:
        copy_calibration()
        return
    if args.gpus != 1:
        print("bench.py measures one GPU: the MatMulNBits family runs on a single device here; "
              "multi-GPU sharding is a design note only.", file=sys.stderr)
        sys.exit(2)

    import torch
    from xrgpu_amd import ops, workloads

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    results = {}
    names = ["decode_up_m1", "prefill_m2048", "prefill_m2048_prepacked", "qkv_gqa_m4", "mlp_swiglu_m16",
             "mlp_prefill_m64", "down_proj_m64", "mlp_prefill_m2048", "qkv_prefill_m2048", "f32_k2048_m1",
             "q8_f32_decode_m1", "q8_f16_decode_m1", "f32_prefill_m64", "f32_prefill_m512", "q2_f16_prefill_m128",
             "f32_qkv_decode_m1", "f32_mlp_prefill_m64",
             "qmoe_mixtral_t1", "qmoe_prefill_t256", "bnb4_nf4_m1", "gbq_embed_t2048", "int8a_decode_m1"]
    if args.only:
        names = [n for n in names if n in args.only.split(",")]
    for name in names:
        # every leg rotates more weight bytes than the 256 MB Infinity Cache
        # holds (Qkv: 24 x 13.7 MB = 328 MB)
        # (prefill legs: 8 replicas, 8 x 30-66 MB of weights and scales)
        R = {"prefill_m2048": 8, "prefill_m2048_prepacked": 8, "mlp_prefill_m2048": 8, "qkv_prefill_m2048": 24,
             "qmoe_mixtral_t1": 2, "qmoe_prefill_t256": 1, "gbq_embed_t2048": 8, "qkv_gqa_m4": 24,
             "f32_k2048_m1": 100, "mlp_prefill_m64": 24, "down_proj_m64": 12, "q8_f32_decode_m1": 24, "q8_f16_decode_m1": 24,
             "f32_prefill_m64": 24, "f32_prefill_m512": 24, "q2_f16_prefill_m128": 12, "f32_qkv_decode_m1": 12,
             "f32_mlp_prefill_m64": 24}.get(name, args.replicas)
        w = make_replicas(torch, name, R, dev, seed=SEEDS[name])
        fn = step_fn(ops, name, w)
        steps = args.steps if "prefill_m2048" not in name and name != "qmoe_prefill_t256" else max(10, args.steps // 10)
        ms, eager_ms, wall_ms = time_steps(torch, fn, steps, args.warmup)
        p10, p50, p90 = per_launch_percentiles(torch, fn, min(100, steps), 5)
        wl = workloads.make(name, scale_down=1) if name == "decode_up_m1" else None
        results[name] = dict(ms=ms, eager_ms=eager_ms, wall_ms=wall_ms, p10=p10, p50=p50, p90=p90, steps=steps, replicas=R)
        print(f"[bench] {name}: {ms * 1e3:.3f} us/step over {steps} steps", file=sys.stderr, flush=True)
        del w, fn, wl
        torch.cuda.empty_cache()

    def traffic_of(summary, dispatch_name):
        """Calibrated HBM bytes per launch from the committed rocprofv3 summary,
        when it describes the kernel the dispatcher runs now."""
        from xrgpu_amd.rocprof_summary import read_field
        path = os.path.join(PROFILES, summary)
        if read_field(path, "dispatch_name") != dispatch_name:
            return None
        v = read_field(path, "traffic_bytes_per_launch")
        return int(float(v)) if v else None

    out = {}
    ceiling = stream_ceiling(torch, ops, args.steps, args.warmup) if "decode_up_m1" in results else None
    if "decode_up_m1" in results:
        r = results["decode_up_m1"]
        decode_kernel = ops.select_kernel("MatMulNBits", 1, 4096, 14336, 4, 32)
        nbytes = 33_067_008
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out = {
            "metric": "int4 GEMV µs + HBM GB/s (M=1,K=4096,N=14336); prefill TFLOP/s (M=2048)",
            "value": round(gbs, 2), "unit": "GB/s", "n_gpus": 1, "steps": r["steps"], "warmup": args.warmup,
            "ms_per_step": round(r["ms"], 6), "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
            "dtype": "f16 (int4 weights, fp32 accumulate)", "data": "synthetic",
            "config": {"workload": "decode_up_m1: MatMulNBits M=1 K=4096 N=14336 bits=4 block_size=32 no zp, "
                                   "Llama-3-8B FFN up-projection", "replicas": r["replicas"],
                       "parallelism": "single GPU"},
            "gemv_us": round(r["ms"] * 1e3, 3),
            "gemv_us_per_launch_p10_p50_p90": [round(x * 1e3, 3) for x in (r["p10"], r["p50"], r["p90"])],
            "eager_us_per_call": round(r["eager_ms"] * 1e3, 3),
            "host_wall_us_per_call": round(r["wall_ms"] * 1e3, 3),
            "timing": "HIP events around a graph replay of K steps (each step one operator call on its own replica)",
            "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(gbs / HBM_PEAK_GBS, 4),
                         "traffic": traffic_of("decode_up_m1_gemv.md", decode_kernel),
                         "kernel": decode_kernel, "bytes_per_launch": nbytes},
            "stream_ceiling": ceiling,
            "decode_over_stream_ceiling": round(ceiling["us"] / (r["ms"] * 1e3), 4),
        }
    mceil = mfma_ceiling(torch, ops) if any("prefill_m2048" in n for n in results) else None
    if "prefill_m2048" in results:
        r = results["prefill_m2048"]
        fl = 2 * 2048 * 4096 * 14336
        tf = fl / (r["ms"] * 1e-3) / 1e12
        out["prefill"] = {"workload": "prefill_m2048: MatMulNBits M=2048 K=4096 N=14336 bs=128 packed zp bias",
                          "us": round(r["ms"] * 1e3, 2), "tflops": round(tf, 2),
                          "roofline": {"bound": "mfma", "achieved": round(tf, 2), "peak": FP16_PEAK_TFLOPS,
                                       "unit": "TFLOP/s", "frac": round(tf / FP16_PEAK_TFLOPS, 4),
                                       "flops_per_launch": fl,
                                       "kernel": ops.select_kernel("MatMulNBits", 2048, 4096, 14336, 4, 128, zp="packed"),
                                       "traffic": traffic_of("prefill_m2048_gemm.md", ops.select_kernel(
                                           "MatMulNBits", 2048, 4096, 14336, 4, 128, zp="packed"))},
                          "dense_fp16_library": dense_fp16_reference(torch),
                          "mfma_ceiling": mceil,
                          "frac_of_mfma_ceiling": round(tf / mceil["tflops"], 4)}
    if "prefill_m2048_prepacked" in results:
        r = results["prefill_m2048_prepacked"]
        fl = 2 * 2048 * 4096 * 14336
        tf = fl / (r["ms"] * 1e-3) / 1e12
        out.setdefault("prefill", {})["prepacked"] = {
            "workload": "the same call on weights prepacked once by xrmm_prepack_weights (what the request "
                        "lifecycle does at prepare)",
            "us": round(r["ms"] * 1e3, 2), "tflops": round(tf, 2), "frac": round(tf / FP16_PEAK_TFLOPS, 4),
            "frac_of_mfma_ceiling": round(tf / mceil["tflops"], 4),
            "kernel": "gemm_q4_big (prepacked weights)",
            "traffic": traffic_of("prefill_m2048_prepacked_gemm.md", "gemm_q4_big_prepacked")}
    for name, nbytes, summary, kern in (
            ("qkv_gqa_m4", 13_656_064, "qkv_gqa_m4_gemv.md",
             ops.select_kernel("MatMulNBitsQkv", 4, 4096, 4096, 4, 64, zp="packed")),
            ("mlp_swiglu_m16", 66_650_112, "mlp_swiglu_m16_gemv.md", ops.select_kernel("MatMulNBitsMlp", 16, 4096, 14336, 4, 32))):
        if name in results:
            r = results[name]
            gbs = nbytes / (r["ms"] * 1e-3) / 1e9
            out[name] = {"us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                         "bytes_per_launch": nbytes, "replicas": r["replicas"],
                         "rotated_bytes": nbytes * r["replicas"], "kernel": kern, "traffic": traffic_of(summary, kern)}
    if "mlp_prefill_m64" in results:
        r, q = results["mlp_prefill_m64"], MLP64
        fl = 2 * 2 * q["M"] * q["K"] * q["N"]
        nbytes = 2 * q["N"] * (q["K"] // 2 + q["K"] // q["bs"] * 2) + q["M"] * (q["K"] + q["N"]) * 2 + q["K"] * 2
        tf = fl / (r["ms"] * 1e-3) / 1e12
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out["mlp_prefill_m64"] = {
            "workload": "MatMulNBitsMlp fp16 M=64 K=2048 N=5632 bs=32 normScale SiLU (TinyLlama-1.1B FFN prefill)",
            "us": round(r["ms"] * 1e3, 3), "tflops": round(tf, 2), "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 4),
            "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "flops_per_launch": fl,
            "bytes_per_launch": nbytes, "replicas": r["replicas"],
            "kernel": ops.select_kernel("MatMulNBitsMlp", q["M"], q["K"], q["N"], 4, q["bs"]),
            "traffic": traffic_of("mlp_prefill_m64_thin.md", ops.select_kernel("MatMulNBitsMlp", q["M"], q["K"], q["N"], 4, q["bs"]))}
    for name, q, kern_args in (("mlp_prefill_m2048", MLP2K, ("MatMulNBitsMlp", MLP2K["M"], MLP2K["K"], MLP2K["N"], 4,
                                                             MLP2K["bs"])),
                               ("qkv_prefill_m2048", QKV2K, ("MatMulNBitsQkv", QKV2K["M"], QKV2K["K"], QKV2K["Nq"], 4,
                                                             QKV2K["bs"]))):
        if name not in results:
            continue
        r = results[name]
        if name.startswith("mlp"):
            fl = 2 * 2 * q["M"] * q["K"] * q["N"]
            what = "MatMulNBitsMlp fp16 M=2048 K=4096 N=14336 bs=32 normScale SiLU (Llama-3-8B FFN gate/up prefill)"
            kern = ops.select_kernel(*kern_args)
        else:
            fl = 2 * q["M"] * q["K"] * (q["Nq"] + 2 * q["Nkv"])
            what = "MatMulNBitsQkv fp16 M=2048 K=4096 Nq=4096 Nkv=1024 bs=64 packed zp normScale (GQA prefill)"
            kern = ops.select_kernel(*kern_args, zp="packed")
        tf = fl / (r["ms"] * 1e-3) / 1e12
        out[name] = {"workload": what, "us": round(r["ms"] * 1e3, 2), "tflops": round(tf, 2),
                     "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 4), "flops_per_launch": fl, "replicas": r["replicas"],
                     "kernel": "rms prologue + " + kern}
        if mceil:
            out[name]["frac_of_mfma_ceiling"] = round(tf / mceil["tflops"], 4)
    if "down_proj_m64" in results:
        r, q = results["down_proj_m64"], DOWN64
        fl = 2 * q["M"] * q["K"] * q["N"]
        kb = q["K"] // q["bs"]
        nbytes = q["N"] * (q["K"] // 2 + kb * 2 + (kb + 1) // 2) + q["M"] * (q["K"] + q["N"]) * 2
        tf = fl / (r["ms"] * 1e-3) / 1e12
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out["down_proj_m64"] = {
            "workload": "MatMulNBits fp16 M=64 K=14336 N=4096 bs=32 packed zp (Llama-3-8B FFN down projection, 64 tokens)",
            "us": round(r["ms"] * 1e3, 3), "tflops": round(tf, 2), "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 4),
            "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "bytes_per_launch": nbytes,
            "replicas": r["replicas"],
            "kernel": ops.select_kernel("MatMulNBits", q["M"], q["K"], q["N"], 4, q["bs"], zp="packed") + " (split-K)",
            "traffic": traffic_of("down_proj_m64_gemm.md",
                                  ops.select_kernel("MatMulNBits", q["M"], q["K"], q["N"], 4, q["bs"], zp="packed"))}
    for name, q, what in (("q8_f32_decode_m1", Q8F32, "MatMulNBits float32 M=1 K=2560 N=4096 bits=8 bs=32 (upstream "
                                                     "qwen3-qproj-decode-m1-q8g32 geometry)"),
                          ("q8_f16_decode_m1", Q8F32, "MatMulNBits float16 M=1 K=2560 N=4096 bits=8 bs=32 (upstream "
                                                      "qwen3-qproj-decode-m1-q8g32, float32 arithmetic)"),
                          ("f32_prefill_m64", F32P, "MatMulNBits float32 M=64 K=4096 N=4096 bits=4 bs=32"),
                          ("f32_prefill_m512", F32P512, "MatMulNBits float32 M=512 K=2560 N=4096 bits=4 bs=64 (upstream "
                                                        "qwen3-qproj-prefill-m512-q4g64 geometry)"),
                          ("q2_f16_prefill_m128", Q2F16, "MatMulNBits float16 M=128 K=5120 N=17408 bits=2 bs=128 "
                                                         "(upstream bonsai2-ffn-gate-prefill-m128-q2g128 geometry, "
                                                         "float32 arithmetic)")):
        if name not in results:
            continue
        r = results[name]
        kb = q["K"] // q["bs"]
        esz = 2 if "f16" in name else 4
        nbytes = q["N"] * (q["K"] * q["bits"] // 8 + kb * esz) + q["M"] * (q["K"] + q["N"]) * esz
        fl = 2 * q["M"] * q["K"] * q["N"]
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out[name] = {"workload": what, "us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2),
                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "tflops": round(fl / (r["ms"] * 1e-3) / 1e12, 2),
                     "bytes_per_launch": nbytes, "replicas": r["replicas"],
                     "kernel": ops.select_kernel("MatMulNBits", q["M"], q["K"], q["N"], q["bits"], q["bs"],
                                                 torch.float16 if esz == 2 else torch.float32)}
    for name, q in (("f32_qkv_decode_m1", F32QKV), ("f32_mlp_prefill_m64", F32MLP)):
        if name not in results:
            continue
        r = results[name]
        kb = q["K"] // q["bs"]
        ncols = q["Nq"] + 2 * q["Nkv"] if "qkv" in name else 2 * q["N"]
        nout = ncols if "qkv" in name else q["N"]
        nbytes = ncols * (q["K"] // 2 + kb * 4) + q["M"] * (q["K"] + nout) * 4 + q["K"] * 4
        fl = 2 * q["M"] * q["K"] * ncols
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        what = ("MatMulNBitsQkv float32 M=1 K=4096 Nq=Nkv=4096 bs=32 normScale (upstream qkv-q4-llama-decode-k4096)"
                if "qkv" in name else
                "MatMulNBitsMlp float32 M=64 K=2048 N=5632 bs=32 normScale SiLU (upstream mlp-q4-prefill-m64-k2048-n5632)")
        out[name] = {"workload": what, "us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2),
                     "frac_hbm": round(gbs / HBM_PEAK_GBS, 4), "tflops": round(fl / (r["ms"] * 1e-3) / 1e12, 2),
                     "bytes_per_launch": nbytes, "replicas": r["replicas"],
                     "kernel": ops.select_kernel("MatMulNBitsQkv" if "qkv" in name else "MatMulNBitsMlp", q["M"], q["K"],
                                                 q["Nq"] if "qkv" in name else q["N"], 4, q["bs"], torch.float32)}
    if "f32_k2048_m1" in results:
        r, q = results["f32_k2048_m1"], F32
        nbytes = 2_703_360
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out["f32_k2048_m1"] = {
            "workload": "MatMulNBits float32 M=1 K=2048 N=2048 bs=32 packed zp (the CPU-oracle workload, on the GPU)",
            "us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_launch": nbytes, "replicas": r["replicas"],
            "kernel": ops.select_kernel("MatMulNBits", q["M"], q["K"], q["N"], 4, q["bs"], torch.float32, zp="packed"),
            "traffic": traffic_of("f32_k2048_m1_gemv.md", ops.select_kernel("MatMulNBits", q["M"], q["K"], q["N"], 4, q["bs"],
                                                                              torch.float32, zp="packed"))}
    if "qmoe_mixtral_t1" in results:
        r, q = results["qmoe_mixtral_t1"], QMOE
        nbytes = qmoe_algorithmic_bytes(**q)
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out["qmoe_mixtral_t1"] = {
            "workload": "QMoE T=1 H=4096 I=14336 E=8 k=2 bits=4 block_size=64 interleaved SwiGLU (Mixtral-8x7B experts)",
            "us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_launch": nbytes, "kernel": ops.qmoe_kernel(q["T"], q["H"], q["E"], 2 * q["I"], q["k"], q["bits"],
                                                                   q["bs"], "swiglu", 1)}
    if "qmoe_prefill_t256" in results:
        r, q = results["qmoe_prefill_t256"], QMOE_PF
        flops = 2 * q["T"] * q["k"] * 3 * q["H"] * q["I"]
        tf = flops / (r["ms"] * 1e-3) / 1e12
        out["qmoe_prefill_t256"] = {
            "workload": "QMoE T=256 H=4096 I=14336 E=8 k=2 bits=4 row scales, interleaved SwiGLU (Mixtral-8x7B experts)",
            "us": round(r["ms"] * 1e3, 3), "tflops": round(tf, 2), "frac_mfma": round(tf / FP16_PEAK_TFLOPS, 4),
            "flops_per_launch": flops,
            "numerics": "float32 activations as two binary16 terms: two fp16 MFMAs per product",
            "kernel": ops.qmoe_kernel(q["T"], q["H"], q["E"], 2 * q["I"], q["k"], q["bits"], q["bs"], "swiglu", 1)}
    if "bnb4_nf4_m1" in results:
        r, q = results["bnb4_nf4_m1"], BNB4
        nbytes = q["N"] * q["K"] // 2 + q["N"] * q["K"] // q["bs"] * 2 + q["M"] * (q["K"] + q["N"]) * 2
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out["bnb4_nf4_m1"] = {
            "workload": "MatMulBnb4 fp16 M=1 K=4096 N=14336 NF4 block_size=64 (codes + fp16 absmax)",
            "us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_launch": nbytes, "kernel": ops.bnb4_kernel(q["M"], q["K"], q["N"], q["bs"], 1, 1)}
    if "int8a_decode_m1" in results:
        r = results["int8a_decode_m1"]
        nbytes = 33_067_008
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out["int8a_decode_m1"] = {
            "workload": "opt-in int8 activations (accuracy_level 4), MatMulNBits fp16 M=1 K=4096 N=14336 bs=32",
            "us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_launch": nbytes, "numerics": "not the reference's float32 arithmetic (opt-in)"}
    if "gbq_embed_t2048" in results:
        r, q = results["gbq_embed_t2048"], GBQ
        nbytes = q["n"] * (q["width"] // 2 + q["width"] // q["bs"] * 4 + q["width"] * 4 + 4)
        gbs = nbytes / (r["ms"] * 1e-3) / 1e9
        out["gbq_embed_t2048"] = {
            "workload": "GatherBlockQuantized 2048 rows of a 128256 x 4096 4-bit table, block_size=32, fp32 out",
            "us": round(r["ms"] * 1e3, 3), "gbs": round(gbs, 2), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
            "bytes_per_launch": nbytes}
    if not args.no_cpu:
        print("[bench] CPU baseline (NumPy oracle)", file=sys.stderr, flush=True)
        out["cpu_baseline"] = cpu_baseline()
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
