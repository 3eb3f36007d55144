"""PyTorch-ROCm front end of the zero-copy entry points.

Tensors stay on the GPU; the library receives their device pointers and the
current HIP stream. PyTorch only provides memory and streams here: every
operator runs a HIP kernel of libxrmm.so, and a missing library raises.

Shapes follow the operator contracts (kernels/com.microsoft.MatMulNBits*/
contract.json): A ``[..., K]`` (leading axes fold into rows), B
``[N, ceil(K/bs), ceil(bs*bits/8)]`` uint8, scales ``[N, ceil(K/bs)]``,
float zero points ``[N, ceil(K/bs)]`` or packed uint8 zero points
``[N, ceil(ceil(K/bs)*bits/8)]``.
"""
from __future__ import annotations

import torch

from . import _native as nat

_T1 = {torch.float32: nat.F32, torch.float16: nat.F16}


def _ptr(t):
    return None if t is None else t.data_ptr()


# The current stream's raw handle without building a torch.cuda.Stream object
# (a per-call cost of several microseconds on the eager path).
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream(stream=None, device=None):
    if stream is not None:
        return stream.cuda_stream
    if _raw_stream is not None:
        return _raw_stream(device if device is not None and device >= 0 else torch.cuda.current_device())
    return torch.cuda.current_stream().cuda_stream


def _check_dev(*ts):
    """Every tensor on one GPU and contiguous; returns the device index."""
    dev = -2
    for t in ts:
        if t is None:
            continue
        d = t.get_device()  # -1 on the CPU
        if d < 0:
            raise nat.XrmmInvalid("tensors must be on the GPU")
        if not t.is_contiguous():
            raise nat.XrmmInvalid("tensors must be contiguous")
        if dev == -2:
            dev = d
        elif d != dev:
            raise nat.XrmmInvalid("tensors must share one device")
    return dev


def _zp_dtype(zp):
    if zp is None:
        return nat.UNSPECIFIED
    if zp.dtype == torch.uint8:
        return nat.U8
    if zp.dtype in _T1:
        return _T1[zp.dtype]
    raise nat.XrmmInvalid("zero points must be float32, float16 or uint8")


def _t1(A):
    if A.dtype not in _T1:
        raise nat.XrmmInvalid("A must be float32 or float16")
    return _T1[A.dtype]


def _geometry(K, bits, block_size):
    kb = (K + block_size - 1) // block_size
    blob = (block_size * bits + 7) // 8
    return kb, blob, (kb * bits + 7) // 8


def _check_weights(B, S, Z, N, K, bits, bs, dtype, name=""):
    kb, blob, zrow = _geometry(K, bits, bs)
    if B.dtype != torch.uint8 or tuple(B.shape) != (N, kb, blob):
        raise nat.XrmmInvalid(f"{name}B must be uint8 [{N}, {kb}, {blob}], got {B.dtype} {tuple(B.shape)}")
    if S.dtype != dtype or tuple(S.shape) != (N, kb):
        raise nat.XrmmInvalid(f"{name}scales must be {dtype} [{N}, {kb}], got {S.dtype} {tuple(S.shape)}")
    if Z is not None:
        want = (N, zrow) if Z.dtype == torch.uint8 else (N, kb)
        if tuple(Z.shape) != want:
            raise nat.XrmmInvalid(f"{name}zero points must have shape {list(want)}, got {tuple(Z.shape)}")


def _check_out(out, shape, dtype, name="out"):
    """A caller-supplied output must match what the kernels write through its pointer."""
    if out is not None and (out.dtype != dtype or tuple(out.shape) != tuple(shape)):
        raise nat.XrmmInvalid(f"{name} must be {dtype} {list(shape)}, got {out.dtype} {tuple(out.shape)}")


def _check_aux(t, shape, dtype, name):
    """skip / normScale / biases: the kernels read them with A's dtype and the given element count."""
    if t is not None and (t.dtype != dtype or t.numel() != _numel(shape) or (len(shape) == 1 and t.dim() != 1)):
        raise nat.XrmmInvalid(f"{name} must be {dtype} with shape {list(shape)}, got {t.dtype} {tuple(t.shape)}")


def _numel(shape):
    n = 1
    for d in shape:
        n *= int(d)
    return n


def _one_zp_dtype(zps, what):
    present = [z for z in zps if z is not None]
    zdt = _zp_dtype(present[0]) if present else nat.UNSPECIFIED
    if any(_zp_dtype(z) != zdt for z in present):
        raise nat.XrmmInvalid(f"zero points of the {what} projections must share a dtype")
    return zdt


def matmul_nbits(A, B, scales, zero_points=None, bias=None, *, K=None, N=None, bits=4,
                 block_size=32, out=None, workspace=None, stream=None):
    """com.microsoft.MatMulNBits on the GPU. Returns Y ``A.shape[:-1] + [N]``.

    Geometries with few output tiles split K across workgroups on a workspace
    (``matmul_nbits_workspace_bytes``), and float32 activations with more than
    16 rows (from 5 or 12 rows for weight matrices of 2^25 or 2^24 codes) run
    the float32 matrix-core GEMM, whose row exponents (and split partials)
    live there too. Eager calls use one zero-filled
    workspace per (device, stream) kept by this module. A caller may pass its
    own ``workspace`` (uint8, 256-byte aligned, its first 4096 bytes zero
    before first use; every call leaves them zero); calls that may overlap
    need different workspaces. Under HIP graph capture without a caller
    workspace the call runs unsplit, so a captured graph never depends on a
    workspace this module might replace or share with another graph."""
    K = int(K if K is not None else A.shape[-1])
    N = int(N if N is not None else B.shape[0])
    if A.shape[-1] != K:
        raise nat.XrmmInvalid("A's last dimension must equal K")
    _check_weights(B, scales, zero_points, N, K, bits, block_size, A.dtype)
    if bias is not None and (bias.dtype != A.dtype or tuple(bias.shape) != (N,)):
        raise nat.XrmmInvalid("bias must be [N] of A's dtype")
    M = A.numel() // K
    _check_out(out, tuple(A.shape[:-1]) + (N,), A.dtype)
    dev = _check_dev(A, B, scales, zero_points, bias, out)
    if out is None:
        out = torch.empty(tuple(A.shape[:-1]) + (N,), dtype=A.dtype, device=A.device)
    lib = nat.lib()
    s = _stream(stream, dev)
    need = lib.xrmm_matmul_nbits_workspace_bytes(M, K, N, bits, block_size, _t1(A)) if M > 4 else 0
    if need > 0 and workspace is not None:
        if workspace.dtype != torch.uint8 or workspace.numel() < need or workspace.get_device() != dev:
            raise nat.XrmmInvalid(f"workspace must be uint8 with at least {need} bytes on A's device")
        ws = workspace
    elif need > 0 and not torch.cuda.is_current_stream_capturing():
        ws = _workspace(A.device, s, need, stream)
    else:
        need = 0
    if need > 0:
        nat.check(lib.xrmm_matmul_nbits_ws(_ptr(A), _ptr(B), _ptr(scales), _ptr(zero_points), _zp_dtype(zero_points),
                                           _ptr(bias), _ptr(out), M, K, N, bits, block_size, _t1(A), _ptr(ws),
                                           ws.numel(), s))
        return out
    nat.check(lib.xrmm_matmul_nbits(_ptr(A), _ptr(B), _ptr(scales), _ptr(zero_points),
                                    _zp_dtype(zero_points), _ptr(bias), _ptr(out), M, K, N,
                                    bits, block_size, _t1(A), s))
    return out


# Split-K workspaces of matmul_nbits, one per (device, stream): zero-filled when
# allocated, and every call leaves them zero-filled, so consecutive calls on a
# stream share one; calls on different streams never share.
_WORKSPACES = {}


def _workspace(device, stream_handle, nbytes, stream=None):
    key = (device.index, stream_handle)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.numel() < nbytes:
        size = max(nbytes, 0 if ws is None else 2 * ws.numel())
        if stream is None:  # the current stream: the one the call enqueues on
            ws = torch.zeros(size, dtype=torch.uint8, device=device)
        else:
            with torch.cuda.stream(stream):  # zero-filled in the stream that will use it
                ws = torch.zeros(size, dtype=torch.uint8, device=device)
        _WORKSPACES[key] = ws
    return ws


def matmul_nbits_workspace_bytes(M, K, N, bits=4, block_size=32, dtype=torch.float16):
    """Bytes of the split-K workspace a MatMulNBits geometry uses (0: none)."""
    return int(nat.lib().xrmm_matmul_nbits_workspace_bytes(int(M), int(K), int(N), int(bits), int(block_size),
                                                            nat.F16 if dtype == torch.float16 else nat.F32))


def prepacked_bytes(N, K, bits=4, block_size=32):
    """Bytes of B prepacked for the prefill GEMM (0: the geometry has no prepacked layout)."""
    return int(nat.lib().xrmm_prepacked_bytes(int(N), int(K), int(bits), int(block_size)))


def prepack_weights(B, *, K, N=None, bits=4, block_size=32, stream=None):
    """B [N, ceil(K/bs), bs/2] uint8 -> the prepacked layout (a flat uint8 tensor) that
    matmul_nbits_prepacked reads: K-step-major, codes reordered inside each word."""
    N = int(N if N is not None else B.shape[0])
    K = int(K)
    kb, blob, _ = _geometry(K, bits, block_size)
    if B.dtype != torch.uint8 or tuple(B.shape) != (N, kb, blob):
        raise nat.XrmmInvalid(f"B must be uint8 [{N}, {kb}, {blob}], got {B.dtype} {tuple(B.shape)}")
    nbytes = prepacked_bytes(N, K, bits, block_size)
    if nbytes == 0:
        raise nat.XrmmInvalid("prepacked weights need 4-bit codes and whole 32-code chunks per column")
    out = torch.empty(nbytes, dtype=torch.uint8, device=B.device)
    dev = _check_dev(B, out)
    nat.check(nat.lib().xrmm_prepack_weights(_ptr(B), _ptr(out), N, K, bits, block_size, _stream(stream, dev)))
    return out


def matmul_nbits_prepacked(A, packed, scales, zero_points=None, bias=None, *, K=None, N, bits=4, block_size=32,
                           out=None, stream=None):
    """MatMulNBits with B prepacked by prepack_weights (the prefill GEMM for every M)."""
    K = int(K if K is not None else A.shape[-1])
    N = int(N)
    if A.shape[-1] != K:
        raise nat.XrmmInvalid("A's last dimension must equal K")
    if packed.dtype != torch.uint8 or packed.numel() != prepacked_bytes(N, K, bits, block_size):
        raise nat.XrmmInvalid("packed must be the uint8 output of prepack_weights for this N, K and block_size")
    kb, _, zrow = _geometry(K, bits, block_size)
    if scales.dtype != A.dtype or tuple(scales.shape) != (N, kb):
        raise nat.XrmmInvalid(f"scales must be {A.dtype} [{N}, {kb}], got {scales.dtype} {tuple(scales.shape)}")
    if zero_points is not None:
        want = (N, zrow) if zero_points.dtype == torch.uint8 else (N, kb)
        if tuple(zero_points.shape) != want:
            raise nat.XrmmInvalid(f"zero points must have shape {list(want)}, got {tuple(zero_points.shape)}")
    if bias is not None and (bias.dtype != A.dtype or tuple(bias.shape) != (N,)):
        raise nat.XrmmInvalid("bias must be [N] of A's dtype")
    M = A.numel() // K
    _check_out(out, tuple(A.shape[:-1]) + (N,), A.dtype)
    dev = _check_dev(A, packed, scales, zero_points, bias, out)
    if out is None:
        out = torch.empty(tuple(A.shape[:-1]) + (N,), dtype=A.dtype, device=A.device)
    nat.check(nat.lib().xrmm_matmul_nbits_prepacked(_ptr(A), _ptr(packed), _ptr(scales), _ptr(zero_points),
                                                    _zp_dtype(zero_points), _ptr(bias), _ptr(out), M, K, N, bits,
                                                    block_size, _t1(A), _stream(stream, dev)))
    return out


def _fused_workspace(op, A, M, K, N, Nkv, bits, block_size, skip, norm_scale, workspace):
    """The normalised-activation workspace of a Qkv / Mlp prefill call: the
    caller's, checked, or a fresh one from torch's caching allocator (under
    HIP graph capture it comes from the graph's own pool); (None, 0) when the
    geometry needs none. Nothing in it needs clearing."""
    need = int(nat.lib().xrmm_matmul_nbits_fused_workspace_bytes(op, M, K, N, Nkv, bits, block_size, _t1(A),
                                                                 int(skip is not None), int(norm_scale is not None)))
    if need <= 0:
        return None, 0
    if workspace is not None:
        if workspace.dtype != torch.uint8 or workspace.numel() < need or workspace.get_device() != A.get_device():
            raise nat.XrmmInvalid(f"workspace must be uint8 with at least {need} bytes on A's device")
        return workspace, workspace.numel()
    return torch.empty(need, dtype=torch.uint8, device=A.device), need


def fused_workspace_bytes(op, M, K, N, Nkv=0, bits=4, block_size=32, dtype=torch.float16, skip=False,
                          norm_scale=True):
    """Bytes of the Qkv ("qkv") / Mlp ("mlp") prefill workspace (0: none)."""
    code = {"qkv": 1, "mlp": 2}[op]
    return int(nat.lib().xrmm_matmul_nbits_fused_workspace_bytes(
        code, int(M), int(K), int(N), int(Nkv), int(bits), int(block_size),
        nat.F16 if dtype == torch.float16 else nat.F32, int(bool(skip)), int(bool(norm_scale))))


def matmul_nbits_qkv(A, q_B, q_scales, k_B, k_scales, v_B, v_scales, *, norm_scale, skip=None,
                     K=None, Nq=None, Nkv=None, bits=4, block_size=32, epsilon=1e-6,
                     q_zero_points=None, k_zero_points=None, v_zero_points=None,
                     want_residual=True, workspace=None, stream=None):
    """com.microsoft.MatMulNBitsQkv. Returns ``(Q, K, V, residual-or-None)``.

    Prefill geometries normalise the rows once into a workspace
    (``fused_workspace_bytes``); pass ``workspace`` to supply it, else one is
    taken from torch's caching allocator."""
    K = int(K if K is not None else A.shape[-1])
    Nq = int(Nq if Nq is not None else q_B.shape[0])
    Nkv = int(Nkv if Nkv is not None else k_B.shape[0])
    zps = (q_zero_points, k_zero_points, v_zero_points)
    for (Bm, S, Z, n, nm) in ((q_B, q_scales, zps[0], Nq, "q_"), (k_B, k_scales, zps[1], Nkv, "k_"),
                              (v_B, v_scales, zps[2], Nkv, "v_")):
        _check_weights(Bm, S, Z, n, K, bits, block_size, A.dtype, nm)
    zdt = _one_zp_dtype(zps, "three")
    if A.shape[-1] != K:
        raise nat.XrmmInvalid("A's last dimension must equal K")
    M = A.numel() // K
    _check_aux(skip, (M, K), A.dtype, "skip")
    if norm_scale is None:
        raise nat.XrmmInvalid("Missing complex input: normScaleT")
    _check_aux(norm_scale, (K,), A.dtype, "norm_scale")
    dev = _check_dev(A, skip, norm_scale, q_B, q_scales, k_B, k_scales, v_B, v_scales, *zps)
    lead = tuple(A.shape[:-1])
    Q = torch.empty(lead + (Nq,), dtype=A.dtype, device=A.device)
    Ko = torch.empty(lead + (Nkv,), dtype=A.dtype, device=A.device)
    V = torch.empty(lead + (Nkv,), dtype=A.dtype, device=A.device)
    R = torch.empty_like(A) if want_residual else None
    ws, nws = _fused_workspace(1, A, M, K, Nq, Nkv, bits, block_size, skip, norm_scale, workspace)
    nat.check(nat.lib().xrmm_matmul_nbits_qkv_ws(
        _ptr(A), _ptr(skip), _ptr(norm_scale), _ptr(q_B), _ptr(q_scales), _ptr(zps[0]), _ptr(k_B),
        _ptr(k_scales), _ptr(zps[1]), _ptr(v_B), _ptr(v_scales), _ptr(zps[2]), zdt, _ptr(Q), _ptr(Ko),
        _ptr(V), _ptr(R), M, K, Nq, Nkv, bits, block_size, float(epsilon), _t1(A), _ptr(ws), nws,
        _stream(stream, dev)))
    return Q, Ko, V, R


def matmul_nbits_mlp(A, gate_B, gate_scales, up_B, up_scales, *, skip=None, norm_scale=None,
                     gate_bias=None, up_bias=None, K=None, N=None, bits=4, block_size=32,
                     epsilon=1e-5, activation="silu", gate_zero_points=None, up_zero_points=None,
                     want_residual=False, workspace=None, stream=None):
    """com.microsoft.MatMulNBitsMlp. Returns ``(Y, residual-or-None)``.

    Prefill geometries with skip or norm_scale normalise the rows once into a
    workspace (``fused_workspace_bytes``); pass ``workspace`` to supply it,
    else one is taken from torch's caching allocator."""
    K = int(K if K is not None else A.shape[-1])
    N = int(N if N is not None else gate_B.shape[0])
    if activation not in nat.ACT:
        raise nat.XrmmInvalid("Unknown fused activation: " + str(activation))
    _check_weights(gate_B, gate_scales, gate_zero_points, N, K, bits, block_size, A.dtype, "gate_")
    _check_weights(up_B, up_scales, up_zero_points, N, K, bits, block_size, A.dtype, "up_")
    zdt = _one_zp_dtype((gate_zero_points, up_zero_points), "gate and up")
    if A.shape[-1] != K:
        raise nat.XrmmInvalid("A's last dimension must equal K")
    M = A.numel() // K
    _check_aux(skip, (M, K), A.dtype, "skip")
    _check_aux(norm_scale, (K,), A.dtype, "norm_scale")
    _check_aux(gate_bias, (N,), A.dtype, "gate_bias")
    _check_aux(up_bias, (N,), A.dtype, "up_bias")
    dev = _check_dev(A, skip, norm_scale, gate_B, gate_scales, up_B, up_scales, gate_bias, up_bias,
               gate_zero_points, up_zero_points)
    Y = torch.empty(tuple(A.shape[:-1]) + (N,), dtype=A.dtype, device=A.device)
    R = torch.empty_like(A) if want_residual else None
    ws, nws = _fused_workspace(2, A, M, K, N, 0, bits, block_size, skip, norm_scale, workspace)
    nat.check(nat.lib().xrmm_matmul_nbits_mlp_ws(
        _ptr(A), _ptr(skip), _ptr(norm_scale), _ptr(gate_B), _ptr(gate_scales), _ptr(gate_zero_points),
        _ptr(gate_bias), _ptr(up_B), _ptr(up_scales), _ptr(up_zero_points), _ptr(up_bias), zdt, _ptr(Y),
        _ptr(R), M, K, N, bits, block_size, float(epsilon), nat.ACT[activation], _t1(A), _ptr(ws), nws,
        _stream(stream, dev)))
    return Y, R


def dequantize(B, scales, zero_points=None, *, K, bits=4, block_size=32, out_dtype=torch.float32,
               stream=None):
    """Dequantized ``W[N, K]``: float32 reference value or its one-rounding fp16."""
    N = int(B.shape[0])
    dev = _check_dev(B, scales, zero_points)
    _check_weights(B, scales, zero_points, N, K, bits, block_size, scales.dtype)
    W = torch.empty((N, K), dtype=out_dtype, device=B.device)
    nat.check(nat.lib().xrmm_dequantize(_ptr(B), _ptr(scales), _ptr(zero_points), _zp_dtype(zero_points),
                                        _ptr(W), N, K, bits, block_size, _T1[scales.dtype], _T1[out_dtype],
                                        _stream(stream, dev)))
    return W


def select_kernel(op: str, M, K, N, bits=4, block_size=32, dtype=torch.float16, zp=None, zp_dtype=None) -> str:
    """The kernel family a call takes (with the workspaces this module
    supplies). ``zp``: None, "packed" (uint8) or "float" (zero points of
    ``zp_dtype``, by default the activations' dtype)."""
    code = {"MatMulNBits": 0, "MatMulNBitsQkv": 1, "MatMulNBitsMlp": 2}[op]
    zdt = nat.UNSPECIFIED if zp is None else nat.U8 if zp == "packed" else _T1[zp_dtype or dtype]
    r = nat.lib().xrmm_select_kernel(code, M, K, N, bits, block_size, _T1[dtype], zdt)
    if r is None:
        raise nat.XrmmInvalid(nat.last_error())
    return r.decode()


def qmoe(x, router, fc1, fc1_scales, fc2, fc2_scales, *, k=1, activation="relu", swiglu_fusion=0,
         expert_weight_bits=4, block_size=0, activation_alpha=1.0, activation_beta=0.0, swiglu_limit=None,
         workspace=None, stream=None):
    """com.microsoft.QMoE: ``output`` of ``x``'s shape (float32).

    x ``[..., H]`` float32, router ``[T, E]`` float32, fc1 ``[E, F1, H*bits/8]``
    and fc2 ``[E, H, I*bits/8]`` uint8, float32 scales ``[E, rows]`` or
    ``[E, rows, cols/block_size]``. ``workspace`` (uint8 device tensor) is
    allocated per call when not given.
    """
    if activation not in ("relu", "swiglu"):
        raise nat.XrmmInvalid("Invalid quantized SwiGLU fusion")
    dev = _check_dev(x, router, fc1, fc1_scales, fc2, fc2_scales, workspace)
    for t, dt, nm in ((x, torch.float32, "input"), (router, torch.float32, "router"), (fc1, torch.uint8, "fc1"),
                      (fc2, torch.uint8, "fc2"), (fc1_scales, torch.float32, "fc1 scales"),
                      (fc2_scales, torch.float32, "fc2 scales")):
        if t.dtype != dt:
            raise nat.XrmmInvalid(f"{nm} has the wrong dtype")
    H = int(x.shape[-1])
    T = x.numel() // H if H else 0
    E = int(router.shape[1])
    F1 = int(fc1.shape[1])
    act = nat.ACT[activation]
    fusion = 2 if (activation == "swiglu" and swiglu_fusion) else 1
    inter = F1 // fusion
    if int(router.shape[0]) != T or fc1.shape[0] != E or fc2.shape[0] != E or fc2.shape[1] != H:
        raise nat.XrmmInvalid("Invalid MoE weight geometry")
    per = 8 // int(expert_weight_bits)
    if fc1.dim() != 3 or fc2.dim() != 3 or fc1.shape[2] * per != H or fc2.shape[2] * per != inter:
        raise nat.XrmmInvalid("Invalid packed expert projection")
    for sc, rows, cols in ((fc1_scales, F1, H), (fc2_scales, H, inter)):
        want = (E, rows, cols // block_size) if block_size else (E, rows)
        if tuple(sc.shape) != want:
            raise nat.XrmmInvalid("Invalid quantized expert scales")
    y = torch.empty_like(x)
    if workspace is None:
        workspace = torch.empty(qmoe_workspace_bytes(T, k, H, inter), dtype=torch.uint8, device=x.device)
    nat.check(nat.lib().xrmm_qmoe(
        _ptr(x), _ptr(router), _ptr(fc1), _ptr(fc1_scales), _ptr(fc2), _ptr(fc2_scales), _ptr(y), _ptr(workspace),
        workspace.numel(), T, H, E, F1, int(k), int(expert_weight_bits), int(block_size), act, int(swiglu_fusion),
        float(activation_alpha), float(activation_beta), float(swiglu_limit or 0.0), int(swiglu_limit is not None),
        _stream(stream, dev)))
    return y


def qmoe_workspace_bytes(T, k, hidden, inter) -> int:
    """Bytes of device workspace ``qmoe`` needs (routing table, h, FC2 partials)."""
    return max(int(nat.lib().xrmm_qmoe_workspace_bytes(int(T), int(k), int(hidden), int(inter))), 1)


def qmoe_kernel(T, H, E, F1, k=1, bits=4, block_size=0, activation="relu", swiglu_fusion=0) -> str:
    r = nat.lib().xrmm_qmoe_kernel(T, H, E, F1, k, bits, block_size, nat.ACT[activation], swiglu_fusion)
    return r.decode() if r else ""


_IDX = {torch.int32: nat.I32, torch.int64: nat.I64}


def gather_block_quantized(data, indices, scales, zero_points=None, *, bits=4, block_size=128, status=None,
                           check=True, stream=None):
    """com.microsoft.GatherBlockQuantized: float32 ``[len(indices), width]``.

    data ``[rows, packed_cols]`` uint8, indices int32/int64 ``[n]``, float32
    scales ``[rows, blocks]``, optional packed uint8 zero points. An index out
    of range leaves its row zero and raises the device word ``status`` (uint32,
    allocated here when not given) to 55; with ``check`` the call waits for the
    stream and raises ``XrmmError`` ("GPU operator contract validation failed:
    code 55") as the reference's run does.
    """
    if status is not None and (status.dtype not in (torch.int32, torch.uint32) or status.numel() < 1):
        raise nat.XrmmInvalid("status must be an int32 or uint32 tensor of at least one element")
    if data.dtype != torch.uint8 or (zero_points is not None and zero_points.dtype != torch.uint8):
        raise nat.XrmmInvalid("Logical dtype outside frozen contract: dataT")
    if scales.dtype != torch.float32:
        raise nat.XrmmInvalid("Logical dtype outside frozen contract: scalesT")
    if indices.dtype not in _IDX:
        raise nat.XrmmInvalid("Logical dtype outside frozen contract: indicesT")
    if data.dim() != 2 or indices.dim() != 1:
        raise nat.XrmmInvalid("Unsupported GatherBlockQuantized geometry")
    rows, pcols = int(data.shape[0]), int(data.shape[1])
    width = pcols * (8 // int(bits)) if bits in (4, 8) else 0
    blocks = (width + block_size - 1) // block_size if block_size > 0 else 0
    if tuple(scales.shape) != (rows, blocks):
        raise nat.XrmmInvalid("Unsupported GatherBlockQuantized geometry")
    if zero_points is not None and tuple(zero_points.shape) != (rows, (blocks * bits + 7) // 8):
        raise nat.XrmmInvalid("Unsupported GatherBlockQuantized geometry")
    dev = _check_dev(data, indices, scales, zero_points, status)
    data, indices, scales = data.contiguous(), indices.contiguous(), scales.contiguous()
    out = torch.empty((int(indices.shape[0]), width), dtype=torch.float32, device=data.device)
    if status is None:
        status = torch.zeros(1, dtype=torch.int32, device=data.device)
    nat.check(nat.lib().xrmm_gather_block_quantized(
        _ptr(data), _ptr(indices), _IDX[indices.dtype], _ptr(scales), _ptr(zero_points), _ptr(out), _ptr(status),
        rows, pcols, int(indices.shape[0]), int(bits), int(block_size), _stream(stream, dev)))
    if check:
        code = int(status.item())
        if code:
            raise nat.XrmmError(f"GPU operator contract validation failed: code {code}")
    return out


def matmul_bnb4(A, B, absmax, *, K, N, block_size=32, quant_type=1, trans_b=1, out=None, stream=None):
    """com.microsoft.MatMulBnb4: ``Y = A @ dequant(B)`` in A's dtype, ``[M, N]``.

    A ``[M, K]`` float32/float16, B uint8 ``ceil(N*K/2)`` bytes (even flat index
    in the high nibble), absmax ``ceil(N*K/block_size)`` in A's dtype.
    """
    if A.dtype not in _T1 or absmax.dtype != A.dtype:
        raise nat.XrmmInvalid("Logical dtype outside frozen contract: aT")
    if B.dtype != torch.uint8:
        raise nat.XrmmInvalid("Logical dtype outside frozen contract: bT")
    if A.dim() != 2 or int(A.shape[1]) != K:
        raise nat.XrmmInvalid("Invalid packed matmul geometry")
    if B.numel() < (N * K + 1) // 2 or absmax.numel() < (N * K + block_size - 1) // max(block_size, 1):
        raise nat.XrmmInvalid("Invalid packed matmul geometry")
    M = int(A.shape[0])
    _check_out(out, (M, N), A.dtype)
    dev = _check_dev(A, B, absmax, out)
    A, B, absmax = A.contiguous(), B.contiguous(), absmax.contiguous()
    Y = out if out is not None else torch.empty((M, N), dtype=A.dtype, device=A.device)
    nat.check(nat.lib().xrmm_matmul_bnb4(_ptr(A), _ptr(B), _ptr(absmax), _ptr(Y), M, K, N, int(block_size),
                                         int(quant_type), int(trans_b), _T1[A.dtype], _stream(stream, dev)))
    return Y


def bnb4_kernel(M, K, N, block_size=32, quant_type=1, trans_b=1, dtype=torch.float16) -> str:
    r = nat.lib().xrmm_matmul_bnb4_kernel(M, K, N, block_size, quant_type, trans_b, _T1[dtype])
    if r is None:
        raise nat.XrmmInvalid(nat.last_error())
    return r.decode()


def matmul_nbits_int8a(A, B, scales, zero_points=None, bias=None, *, K, N, bits=4, block_size=32, out=None,
                       workspace=None, stream=None):
    """Opt-in int8-activation MatMulNBits (the upstream operator's
    accuracy_level 4, not the reference's float32 arithmetic): rows of A are
    quantized per 128 (max|a| / 127) and multiplied with the 4-bit weights as
    exact int32 dot products. Packed uint8 zero points only."""
    if A.dtype not in _T1 or scales.dtype != A.dtype:
        raise nat.XrmmInvalid("T1 must be float32 or float16")
    if zero_points is not None and zero_points.dtype != torch.uint8:
        raise nat.XrmmInvalid("int8-activation path: zero points must be absent or packed uint8")
    _check_weights(B, scales, zero_points, N, K, bits, block_size, scales.dtype)
    if A.shape[-1] != K:
        raise nat.XrmmInvalid("A's last dimension must equal K")
    if bias is not None and (bias.dtype != A.dtype or tuple(bias.shape) != (N,)):
        raise nat.XrmmInvalid("bias must be [N] of A's dtype")
    A2 = A.reshape(-1, K).contiguous()
    M = int(A2.shape[0])
    _check_out(out, tuple(A.shape[:-1]) + (N,), A.dtype)
    dev = _check_dev(A, B, scales, zero_points, bias, out, workspace)
    Y = out if out is not None else torch.empty(tuple(A.shape[:-1]) + (N,), dtype=A.dtype, device=A.device)
    need = int(nat.lib().xrmm_matmul_nbits_int8a_workspace_bytes(M, K))
    if need < 0:
        raise nat.XrmmInvalid("int8-activation path: K must be a positive multiple of 128, at most 16384")
    if workspace is None:
        workspace = torch.empty(max(need, 16), dtype=torch.uint8, device=A.device)
    nat.check(nat.lib().xrmm_matmul_nbits_int8a(
        _ptr(A2), _ptr(B), _ptr(scales), _ptr(zero_points), nat.U8 if zero_points is not None else nat.UNSPECIFIED,
        _ptr(bias), _ptr(Y), _ptr(workspace), workspace.numel(), M, K, N, bits, block_size, _T1[A.dtype],
        _stream(stream, dev)))
    return Y


def matmul_nbits_int8a_noalloc(A, B, scales, zero_points=None, bias=None, *, K, N, bits=4, block_size=32, out=None,
                               stream=None):
    """``matmul_nbits_int8a`` without a workspace: the library's static 2 MiB
    device scratch holds the activation codes (nothing is allocated by the
    library; ``out`` avoids the one torch allocation here). Calls overlapping on
    one GPU share that scratch and race."""
    if A.dtype not in _T1 or scales.dtype != A.dtype:
        raise nat.XrmmInvalid("T1 must be float32 or float16")
    if zero_points is not None and zero_points.dtype != torch.uint8:
        raise nat.XrmmInvalid("int8-activation path: zero points must be absent or packed uint8")
    _check_weights(B, scales, zero_points, N, K, bits, block_size, scales.dtype)
    if A.shape[-1] != K:
        raise nat.XrmmInvalid("A's last dimension must equal K")
    if bias is not None and (bias.dtype != A.dtype or tuple(bias.shape) != (N,)):
        raise nat.XrmmInvalid("bias must be [N] of A's dtype")
    M = A.numel() // K
    _check_out(out, tuple(A.shape[:-1]) + (N,), A.dtype)
    dev = _check_dev(A, B, scales, zero_points, bias, out)
    Y = out if out is not None else torch.empty(tuple(A.shape[:-1]) + (N,), dtype=A.dtype, device=A.device)
    nat.check(nat.lib().xrmm_matmul_nbits_int8a_noalloc(
        _ptr(A), _ptr(B), _ptr(scales), _ptr(zero_points), nat.U8 if zero_points is not None else nat.UNSPECIFIED,
        _ptr(bias), _ptr(Y), M, K, N, bits, block_size, _T1[A.dtype], _stream(stream, dev)))
    return Y


def int8a_workspace_bytes(M, K) -> int:
    """Workspace bytes of ``matmul_nbits_int8a`` (activation codes and scales)."""
    n = int(nat.lib().xrmm_matmul_nbits_int8a_workspace_bytes(int(M), int(K)))
    if n < 0:
        raise nat.XrmmInvalid("int8-activation path: K must be a positive multiple of 128, at most 16384")
    return max(n, 16)


def stream_read(buf, *, loads_per_lane=4, sink=None, nontemporal=True, workgroups=0, stream=None):
    """Read ``buf`` (a device tensor of a multiple of 16 bytes) once on the GPU
    with 16-byte loads: the plain read rate a decode GEMV is compared with.
    ``nontemporal`` picks the cache policy; ``workgroups`` 0 launches the
    one-shot grid, a positive count a persistent grid of that many
    workgroups."""
    dev = _check_dev(buf, sink)
    if sink is None:
        sink = torch.zeros(1, dtype=torch.int32, device=buf.device)
    nat.check(nat.lib().xrmm_stream_read_ex(_ptr(buf), buf.numel() * buf.element_size(), _ptr(sink),
                                            int(loads_per_lane), 1 if nontemporal else 0, int(workgroups),
                                            _stream(stream, dev)))
    return sink


def mfma_peak_operand_bytes():
    return int(nat.lib().xrmm_mfma_peak_operand_bytes())


def mfma_peak_flops(workgroups, waves, iters):
    return int(nat.lib().xrmm_mfma_peak_flops(int(workgroups), int(waves), int(iters)))


def mfma_peak(operands, clocks, *, workgroups, waves=4, accumulators=4, iters, sink=None, stream=None):
    """Back-to-back v_mfma_f32_32x32x16_f16 on ``operands`` (binary16,
    mfma_peak_operand_bytes() bytes) from ``workgroups`` workgroups of
    ``waves`` waves, ``16 * iters`` MFMAs per wave over ``accumulators``
    independent accumulators; ``clocks`` (int64, 4 per wave) receives each
    wave's shader-clock cycles, constant-rate counter at its loop's start and
    end, and workgroup index."""
    dev = _check_dev(operands, clocks, sink)
    if operands.numel() * operands.element_size() < mfma_peak_operand_bytes():
        raise nat.XrmmInvalid("mfma peak: operand buffer too small")
    if clocks.dtype != torch.int64 or clocks.numel() < 4 * workgroups * waves:
        raise nat.XrmmInvalid("mfma peak: clocks must be int64 with 4 * workgroups * waves elements")
    if sink is None:
        sink = torch.zeros(1, dtype=torch.float32, device=operands.device)
    nat.check(nat.lib().xrmm_mfma_peak(_ptr(operands), _ptr(sink), _ptr(clocks), int(workgroups), int(waves),
                                       int(accumulators), int(iters), _stream(stream, dev)))
    return clocks
