"""GPU: each operator driven through its kernel-catalog binding
(xrgpu_amd/catalog.py): the request lifecycle and the zero-copy call the
entry names, against the oracle."""
import numpy as np
import pytest

from oracle import oracle as O
from xrgpu_amd import catalog
from xrgpu_amd import operator as op

pytestmark = pytest.mark.gpu


def _weights(rng, N, K, bs):
    kb = K // bs
    return (rng.integers(0, 256, (N, kb, bs // 2), dtype=np.uint8),
            rng.uniform(0.001, 0.02, (N, kb)).astype(np.float16))


def test_matmul_nbits_through_the_catalog(gpu):
    import torch
    rng = np.random.default_rng(31)
    M, K, N, bs = 3, 256, 96, 32
    A = rng.standard_normal((M, K)).astype(np.float16)
    B, S = _weights(rng, N, K, bs)
    ref = O.matmul_nbits(A, B, S, None, None, K=K, N=N, block_size=bs)
    b = catalog.bind("com.microsoft.MatMulNBits")
    req = b.request([op.Tensor("aT", A), op.Tensor("bT", B), op.Tensor("scalesT", S)], {"N": N, "block_size": bs})
    with b.Operator.prepare("", req) as o:
        o.run()
        (y,) = o.read_outputs()
    assert O.tolerance_ok(y.data, ref, np.float16)[0]
    yz = b.zero_copy(torch.from_numpy(A).to(gpu), torch.from_numpy(B).to(gpu), torch.from_numpy(S).to(gpu),
                     block_size=bs).cpu().numpy()
    assert O.tolerance_ok(yz, ref, np.float16)[0]


def test_qkv_and_mlp_through_the_catalog(gpu):
    import torch
    rng = np.random.default_rng(32)
    M, K, N, bs = 2, 128, 64, 32
    A = rng.standard_normal((M, K)).astype(np.float16)
    g = rng.uniform(0.5, 1.5, K).astype(np.float16)
    W = {p: _weights(rng, N, K, bs) for p in ("q", "k", "v", "gate", "up")}
    res = O.matmul_nbits_qkv(A, *W["q"], *W["k"], *W["v"], K=K, Nq=N, Nkv=N, norm_scale=g, block_size=bs)
    q, k, v = res[0], res[1], res[2]
    b = catalog.bind("com.microsoft.MatMulNBitsQkv")
    ins = [op.Tensor("aT", A), op.Tensor("normScaleT", g)]
    for p in ("q", "k", "v"):
        ins += [op.Tensor(p + "BT", W[p][0]), op.Tensor(p + "ScalesT", W[p][1])]
    with b.Operator.prepare("", b.request(ins, {"Nq": N, "Nkv": N, "block_size": bs})) as o:
        o.run()
        outs = {t.name: t.data for t in o.read_outputs()}
    for name, ref in (("qT", q), ("kT", k), ("vT", v)):
        assert O.tolerance_ok(outs[name], ref, np.float16)[0], name
    y = O.matmul_nbits_mlp(A, *W["gate"], *W["up"], K=K, N=N, block_size=bs)
    y = y[0] if isinstance(y, tuple) else y
    b = catalog.bind("com.microsoft.MatMulNBitsMlp")
    d = lambda x: torch.from_numpy(x).to(gpu)
    yz = b.zero_copy(d(A), d(W["gate"][0]), d(W["gate"][1]), d(W["up"][0]), d(W["up"][1]), block_size=bs)
    yz = (yz[0] if isinstance(yz, tuple) else yz).cpu().numpy()
    assert O.tolerance_ok(yz, y, np.float16)[0]
