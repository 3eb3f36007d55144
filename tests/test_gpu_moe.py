"""GPU parity of com.microsoft.QMoE (libxrmm's xrmm_qmoe) against the oracle.

Every upstream fixture case (kernels/_provenance/upstream/com.microsoft.QMoE/
build/webgpu/test.json) runs with its own attributes and tolerance; inputs the
reference's harness cannot materialise (``fillFloat32``) get seeded values of
the same shape, and explicit outputs are checked as given. Seeded shapes cover
both kernel families (16-byte rows: ``qmoe_rows``; anything else:
``qmoe_scalar``), 4 and 8 bits, row and block scales (16, 32, 64), ReLU and
SwiGLU with and without the limit, k = 1..3, rank-3 input and no tokens. Bar:
the fixture's own atol/rtol on the reference's own inputs; float32
``max|d| <= 1e-5 * max|Y_ref|`` where seeded stand-ins replace them (their
outputs reach 1e4..1e6, where an absolute 5e-5 is below one ulp).
"""
import numpy as np
import pytest

from oracle import moe as Q
from oracle import oracle as O
from tests import fixture_util as F

pytestmark = pytest.mark.gpu
torch = pytest.importorskip("torch")
OP = "com.microsoft.QMoE"


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def ops():
    from xrgpu_amd import ops as _ops
    return _ops


def _attrs(a):
    return dict(k=a.get("k", 1), activation=a.get("activation_type", "relu"), swiglu_fusion=a.get("swiglu_fusion", 0),
                bits=a.get("expert_weight_bits", 4), block_size=a.get("block_size", 0),
                alpha=a.get("activation_alpha", 1.0), beta=a.get("activation_beta", 0.0),
                swiglu_limit=a.get("swiglu_limit"))


def run_gpu(i, at):
    return ops().qmoe(dev(i["inputT"]), dev(i["routerT"]), dev(i["fc1T"]), dev(i["fc1ScalesT"]), dev(i["fc2T"]),
                      dev(i["fc2ScalesT"]), k=at["k"], activation=at["activation"], swiglu_fusion=at["swiglu_fusion"],
                      expert_weight_bits=at["bits"], block_size=at["block_size"], activation_alpha=at["alpha"],
                      activation_beta=at["beta"], swiglu_limit=at["swiglu_limit"]).cpu().numpy()


def run_oracle(i, at):
    return Q.qmoe(i["inputT"], i["routerT"], i["fc1T"], i["fc1ScalesT"], i["fc2T"], i["fc2ScalesT"], **at)


@pytest.mark.parametrize("name", [c["name"] for c in F.load_cases() if c["operation"] == OP])
def test_fixture_cases(gpu, name):
    case = F.find(OP, name)
    i = F.case_inputs(case, substitute=True)
    substituted = not F.materializable(case)
    at = _attrs(case["attrs"])
    got = run_gpu(i, at)
    ref = run_oracle(i, at)
    atol, rtol = F.case_tolerance(case, "outputT")
    assert got.shape == ref.shape
    fixture_ok = F.reference_compare(got, ref, max(atol, 1e-6), rtol)
    if substituted:
        # seeded stand-ins (standard normal scales) reach outputs of 1e4..1e6, where
        # the fixture's absolute tolerance is below one float32 ulp: relative bar
        ok, err, lim = O.tolerance_ok(got, ref, np.float32)
        assert ok or fixture_ok, f"{name}: max|d|={err} limit={lim}"
    else:
        assert fixture_ok, f"{name}: max|d|={np.max(np.abs(got - ref))}"
    if "outputT" in case["explicit"]:
        want = F.materialize(case["outputs"]["outputT"])
        assert F.reference_compare(got, want, atol, rtol)


def rand_case(rng, T, H, I, E, bits, bs, swiglu):
    F1 = 2 * I if swiglu else I
    x = (rng.standard_normal((T, H)) * 0.5).astype(np.float32)
    router = rng.standard_normal((T, E)).astype(np.float32)
    fc1 = rng.integers(0, 256, (E, F1, H * bits // 8), dtype=np.uint8)
    fc2 = rng.integers(0, 256, (E, H, I * bits // 8), dtype=np.uint8)
    s1 = rng.uniform(0.01, 0.05, (E, F1, H // bs) if bs else (E, F1)).astype(np.float32)
    s2 = rng.uniform(0.01, 0.05, (E, H, I // bs) if bs else (E, H)).astype(np.float32)
    return {"inputT": x, "routerT": router, "fc1T": fc1, "fc1ScalesT": s1, "fc2T": fc2, "fc2ScalesT": s2}


RAND = [
    # T, H, I, E, k, bits, bs, activation, limit, kernel
    (3, 256, 512, 4, 2, 4, 0, "swiglu", None, "qmoe_rows"),
    (5, 512, 256, 8, 2, 4, 32, "swiglu", 1.5, "qmoe_rows"),
    (2, 256, 256, 4, 1, 4, 16, "relu", None, "qmoe_rows"),
    (4, 256, 384, 3, 3, 8, 64, "swiglu", None, "qmoe_rows"),
    (1, 4096, 1024, 8, 2, 4, 32, "swiglu", None, "qmoe_rows"),   # the decode layout, narrower
    (7, 2048, 512, 6, 2, 8, 0, "relu", None, "qmoe_rows"),
    (2, 96, 40, 3, 2, 4, 0, "swiglu", None, "qmoe_scalar"),       # rows of 48 / 20 bytes
    (3, 72, 40, 4, 1, 8, 0, "relu", None, "qmoe_scalar"),         # rows of 72 / 40 bytes
    (3, 80, 48, 4, 1, 8, 16, "relu", None, "qmoe_rows"),          # 8-bit block 16: one scale per chunk
    # long FC1 / FC2 rows: several row groups per wave in FC1, FC2 reductions
    # split into segments combined by the last workgroup of each row tile
    (1, 1024, 16384, 4, 2, 4, 64, "swiglu", None, "qmoe_rows"),
    (2, 512, 8192, 4, 2, 8, 0, "relu", None, "qmoe_rows"),
    (1, 256, 20480, 3, 3, 4, 16, "swiglu", 4.0, "qmoe_rows"),
    (1, 256, 4096, 2, 1, 4, 32, "swiglu", None, "qmoe_rows"),     # k = 1: segments only
]


@pytest.mark.parametrize("T,H,I,E,k,bits,bs,act,limit,kernel", RAND)
def test_seeded_shapes(gpu, T, H, I, E, k, bits, bs, act, limit, kernel):
    rng = np.random.default_rng(T * 131 + H + I + E + bits + bs)
    sw = act == "swiglu"
    i = rand_case(rng, T, H, I, E, bits, bs, sw)
    at = dict(k=k, activation=act, swiglu_fusion=1 if sw else 0, bits=bits, block_size=bs, alpha=1.702 if sw else 1.0,
              beta=1.0 if sw else 0.0, swiglu_limit=limit)
    assert ops().qmoe_kernel(T, H, E, 2 * I if sw else I, k, bits, bs, act, 1 if sw else 0) == kernel
    got = run_gpu(i, at)
    ref = run_oracle(i, at)
    ok, err, lim = O.tolerance_ok(got, ref, np.float32)
    assert ok, f"max|d|={err} > {lim}"


def test_split_reduction_is_deterministic(gpu):
    # the combined FC2 partials are summed in a fixed order: repeated calls
    # (fresh and reused workspaces) give identical bits
    rng = np.random.default_rng(99)
    i = rand_case(rng, 1, 1024, 16384, 4, 4, 64, True)
    at = dict(k=2, activation="swiglu", swiglu_fusion=1, bits=4, block_size=64, alpha=1.0, beta=0.0, swiglu_limit=None)
    first = run_gpu(i, at)
    d = {n: dev(v) for n, v in i.items()}
    ws = torch.empty(ops().qmoe_workspace_bytes(1, 2, 1024, 16384), dtype=torch.uint8, device="cuda")
    for _ in range(3):
        again = ops().qmoe(d["inputT"], d["routerT"], d["fc1T"], d["fc1ScalesT"], d["fc2T"], d["fc2ScalesT"], k=2,
                           activation="swiglu", swiglu_fusion=1, expert_weight_bits=4, block_size=64,
                           workspace=ws).cpu().numpy()
        assert np.array_equal(first, again)


def test_rank3_and_empty(gpu):
    rng = np.random.default_rng(3)
    i = rand_case(rng, 6, 256, 256, 4, 4, 0, False)
    i3 = dict(i, inputT=i["inputT"].reshape(2, 3, 256))
    at = dict(k=2, activation="relu", swiglu_fusion=0, bits=4, block_size=0, alpha=1.0, beta=0.0, swiglu_limit=None)
    got = run_gpu(i3, at)
    assert got.shape == (2, 3, 256)
    ok, err, lim = O.tolerance_ok(got, run_oracle(i3, at), np.float32)
    assert ok
    e = dict(i, inputT=i["inputT"][:0], routerT=i["routerT"][:0])
    assert run_gpu(e, at).shape == (0, 256)


def test_invalid_geometry_raises(gpu):
    from xrgpu_amd import _native as nat
    rng = np.random.default_rng(5)
    i = rand_case(rng, 2, 256, 256, 4, 4, 0, False)
    at = dict(k=5, activation="relu", swiglu_fusion=0, bits=4, block_size=0, alpha=1.0, beta=0.0, swiglu_limit=None)
    with pytest.raises(nat.XrmmInvalid, match="routing geometry"):
        run_gpu(i, at)
    with pytest.raises(nat.XrmmInvalid, match="SwiGLU fusion"):
        run_gpu(i, dict(at, k=1, swiglu_fusion=1))


GROUPED = [
    # T, H, I, E, k, activation, limit, x scale: the grouped-expert GEMMs
    # (4-bit codes, row scales, at least 32 (token, slot) pairs)
    (48, 1024, 1024, 8, 2, "swiglu", None, 0.2),    # the upstream prefill-band geometry
    (64, 256, 128, 64, 8, "swiglu", 7.0, 1.0),      # many experts and slots, SwiGLU limit
    (40, 512, 192, 6, 3, "relu", None, 1.0),        # ReLU, k = 3, a partial column tile (F1 = 192)
    (33, 256, 320, 5, 1, "swiglu", None, 3e5),      # x far beyond binary16: the row exponent scales it down
    (96, 128, 64, 16, 4, "swiglu", None, 1e-3),     # small x: scaled up before the binary16 split
    (40, 256, 2048, 4, 2, "swiglu", None, 1.0),      # FC2 over two K splits (few tiles)
    (36, 256, 4096, 3, 2, "relu", 5.0, 1.0),         # FC2 over four K splits
]


@pytest.mark.parametrize("T,H,I,E,k,act,limit,xs", GROUPED)
def test_grouped_experts(gpu, T, H, I, E, k, act, limit, xs):
    """Float32 bar max|d| <= 1e-5 max|Y_ref| against the oracle, and
    bitwise-repeatable outputs (the pair lists' order changes no row)."""
    rng = np.random.default_rng(T * 7 + H + I + E + k)
    sw = act == "swiglu"
    i = rand_case(rng, T, H, I, E, 4, 0, sw)
    i["inputT"] = (i["inputT"] * np.float32(xs / max(float(np.abs(i["inputT"]).max()), 1e-30))).astype(np.float32)
    at = dict(k=k, activation=act, swiglu_fusion=1 if sw else 0, bits=4, block_size=0, alpha=1.702 if sw else 1.0,
              beta=1.0 if sw else 0.0, swiglu_limit=limit)
    assert ops().qmoe_kernel(T, H, E, 2 * I if sw else I, k, 4, 0, act, 1 if sw else 0) == "qmoe_grouped"
    got = run_gpu(i, at)
    ok, err, lim = O.tolerance_ok(got, run_oracle(i, at), np.float32)
    assert ok, f"max|d|={err} > {lim}"
    assert np.array_equal(got, run_gpu(i, at))


GROUPED_BLOCKS = [
    # T, H, I, E, k, activation, bits, block_size: block scales and 8-bit
    # codes on the grouped-expert GEMMs
    (48, 512, 512, 6, 2, "swiglu", 4, 32),      # two blocks per K step
    (40, 256, 1024, 4, 2, "relu", 8, 64),       # 8-bit codes, one block per step
    (36, 256, 2048, 3, 2, "swiglu", 4, 128),    # a block over two steps; FC2 in two K splits
    (33, 128, 256, 5, 1, "relu", 8, 32),        # 8-bit, two blocks per K step
    (64, 256, 4096, 2, 2, "relu", 4, 256),      # FC2 in four K splits of whole blocks
    (36, 2048, 4096, 2, 2, "relu", 4, 2048),    # splits past the last block hold zero partials
    (72, 384, 640, 9, 3, "swiglu", 8, 32),      # 8-bit, odd tile counts
]


@pytest.mark.parametrize("T,H,I,E,k,act,bits,bs", GROUPED_BLOCKS)
def test_grouped_block_scales(gpu, T, H, I, E, k, act, bits, bs):
    """Float32 bar against the oracle with per-block scales (each block's sum
    scaled before it joins the row's sum) and 8-bit codes (c - 128 exact in
    binary16), plus bitwise-repeatable outputs."""
    rng = np.random.default_rng(T * 5 + H + I + E + k + bits + bs)
    sw = act == "swiglu"
    i = rand_case(rng, T, H, I, E, bits, bs, sw)
    at = dict(k=k, activation=act, swiglu_fusion=1 if sw else 0, bits=bits, block_size=bs, alpha=1.702 if sw else 1.0,
              beta=1.0 if sw else 0.0, swiglu_limit=None)
    assert ops().qmoe_kernel(T, H, E, 2 * I if sw else I, k, bits, bs, act, 1 if sw else 0) == "qmoe_grouped"
    got = run_gpu(i, at)
    ok, err, lim = O.tolerance_ok(got, run_oracle(i, at), np.float32)
    assert ok, f"max|d|={err} > {lim}"
    assert np.array_equal(got, run_gpu(i, at))


def test_grouped_nonfinite_rows(gpu):
    """+-Inf and NaN activations reach the sums as the reference's float32
    products do (the binary16 split keeps lo = 0 for them); other tokens are
    unaffected."""
    rng = np.random.default_rng(17)
    T, H, I, E = 48, 256, 128, 4
    i = rand_case(rng, T, H, I, E, 4, 0, True)
    i["inputT"][3, 5] = np.inf
    i["inputT"][7, 0] = np.nan
    at = dict(k=2, activation="swiglu", swiglu_fusion=1, bits=4, block_size=0, alpha=1.702, beta=1.0, swiglu_limit=None)
    assert ops().qmoe_kernel(T, H, E, 2 * I, 2, 4, 0, "swiglu", 1) == "qmoe_grouped"
    got, ref = run_gpu(i, at), run_oracle(i, at)
    assert not np.isfinite(ref[3]).all() and not np.isfinite(ref[7]).all()
    ok, err, lim = O.tolerance_ok(got, ref, np.float32)
    assert ok, f"max|d|={err} > {lim}"
