"""Request-level operator API: the Python form of ``xrgpu::operators::extended``.

Mirrors runtime/include/xrgpu/extended_operators.h:8-61 and the types of
runtime/include/xrgpu/operators.h:9-28:

* :class:`Tensor` owns little-endian contiguous host bytes (a NumPy array here)
  with a logical ``dtype`` and an optional ``storage_dtype``;
* :class:`Request` names the operation, its inputs by contract port name
  (``aT``, ``bT``, ``scalesT``, ...), ``attrs`` and ``args`` (args win);
  ``requested_outputs`` selects optional outputs and their storage dtype;
* :func:`plan` is metadata only (no device work);
* :meth:`Operator.prepare` uploads the inputs once, :meth:`Operator.run`
  launches and waits (bounded by ``Options.timeout_ns``),
  :meth:`Operator.read_outputs` returns fresh host tensors, :meth:`Operator.info`
  returns the JSON record, :meth:`Operator.close` releases the device memory.

Errors keep the reference's two classes: :class:`XrmmInvalid` (a ``ValueError``,
std::invalid_argument) and :class:`XrmmError` (a ``RuntimeError``,
std::runtime_error). Every call goes through libxrmm.so; nothing here computes.
"""
from __future__ import annotations

import ctypes
import json
from dataclasses import dataclass, field

import numpy as np

from . import _native as nat
from ._native import XrmmError, XrmmInvalid  # noqa: F401  (re-exported error classes)

MAX_RANK = 16
NAME_MAX = 32

# operators.h:9 DType order
DTYPES = ("float32", "float16", "int32", "uint32", "int16", "int8", "uint8", "int64", "bool", "unspecified")
_NP = {"float32": np.float32, "float16": np.float16, "int32": np.int32, "uint32": np.uint32,
       "int16": np.int16, "int8": np.int8, "uint8": np.uint8, "int64": np.int64, "bool": np.bool_}


def dtype_code(name: str) -> int:
    if name not in DTYPES:
        raise XrmmInvalid("Unknown dtype: " + str(name))
    return DTYPES.index(name)


def dtype_of(array) -> str:
    dt = np.asarray(array).dtype
    for name, t in _NP.items():
        if dt == np.dtype(t):
            return name
    raise XrmmInvalid(f"unsupported NumPy dtype {dt}")


class _CTensor(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("dtype", ctypes.c_int32), ("storage_dtype", ctypes.c_int32),
                ("rank", ctypes.c_int32), ("shape", ctypes.c_int64 * MAX_RANK), ("data", ctypes.c_void_p),
                ("nbytes", ctypes.c_uint64)]


class _CAttr(ctypes.Structure):
    _fields_ = [("key", ctypes.c_char_p), ("kind", ctypes.c_int32), ("i", ctypes.c_int64), ("f", ctypes.c_double),
                ("s", ctypes.c_char_p)]


class _CRequest(ctypes.Structure):
    _fields_ = [("operation", ctypes.c_char_p), ("inputs", ctypes.POINTER(_CTensor)), ("n_inputs", ctypes.c_int32),
                ("attrs", ctypes.POINTER(_CAttr)), ("n_attrs", ctypes.c_int32), ("args", ctypes.POINTER(_CAttr)),
                ("n_args", ctypes.c_int32), ("requested_outputs", ctypes.POINTER(_CTensor)),
                ("n_requested_outputs", ctypes.c_int32)]


class _COptions(ctypes.Structure):
    _fields_ = [("profiling", ctypes.c_int32), ("timeout_ns", ctypes.c_uint64), ("memory_limit_bytes", ctypes.c_uint64)]


class _CDesc(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * NAME_MAX), ("dtype", ctypes.c_int32), ("storage_dtype", ctypes.c_int32),
                ("rank", ctypes.c_int32), ("shape", ctypes.c_int64 * MAX_RANK), ("nbytes", ctypes.c_uint64)]


def _lifecycle_sigs(s):
    P = ctypes.POINTER
    s("xrmm_default_options", None, P(_COptions))
    s("xrmm_plan", ctypes.c_int, P(_CRequest), P(_CDesc), ctypes.c_int32, P(ctypes.c_int32))
    s("xrmm_prepare", ctypes.c_int, P(_CRequest), P(_COptions), P(ctypes.c_void_p))
    s("xrmm_run", ctypes.c_int, ctypes.c_void_p)
    s("xrmm_output_descs", ctypes.c_int, ctypes.c_void_p, P(_CDesc), ctypes.c_int32, P(ctypes.c_int32))
    s("xrmm_read_outputs", ctypes.c_int, ctypes.c_void_p, P(ctypes.c_void_p), P(ctypes.c_uint64), ctypes.c_int32)
    s("xrmm_info", ctypes.c_char_p, ctypes.c_void_p)
    s("xrmm_close", ctypes.c_int, ctypes.c_void_p)
    s("xrmm_destroy", None, ctypes.c_void_p)


_sigs_set = False


def _lib():
    """libxrmm.so with the lifecycle signatures declared."""
    global _sigs_set
    lib = nat.lib()
    if not _sigs_set:
        def s(name, res, *args):
            f = getattr(lib, name)
            f.restype = res
            f.argtypes = list(args)
        _lifecycle_sigs(s)
        _sigs_set = True
    return lib


@dataclass
class Tensor:
    """operators.h:16-23. ``data`` holds the storage bytes as a NumPy array
    (None for a requested output); ``shape``/``dtype`` default from it."""
    name: str
    data: np.ndarray | None = None
    shape: tuple | None = None
    dtype: str | None = None
    storage_dtype: str | None = None

    def __post_init__(self):
        if self.data is not None:
            self.data = np.ascontiguousarray(self.data)
            if self.shape is None:
                self.shape = tuple(self.data.shape)
            if self.dtype is None:
                self.dtype = dtype_of(self.data)
        if self.shape is None or self.dtype is None:
            raise XrmmInvalid(f"tensor {self.name}: shape and dtype required")
        self.shape = tuple(int(d) for d in self.shape)

    def array(self) -> np.ndarray:
        """The bytes viewed as the storage dtype, with the tensor's shape."""
        return self.data


@dataclass
class Request:
    """extended_operators.h:22-28."""
    operation: str
    inputs: list = field(default_factory=list)
    attrs: dict = field(default_factory=dict)
    args: dict = field(default_factory=dict)
    requested_outputs: list = field(default_factory=list)


@dataclass
class Options:
    """operators.h:24-28."""
    profiling: bool = False
    timeout_ns: int = 15_000_000_000
    memory_limit_bytes: int = 268_435_456


class _Marshal:
    """ctypes view of a Request; keeps every buffer alive while in use."""

    def __init__(self, req: Request):
        self.keep = []
        self.req = _CRequest()
        self.req.operation = self._s(req.operation)
        ins = [self._tensor(t, True) for t in req.inputs]
        outs = [self._tensor(t, False) for t in req.requested_outputs]
        self.inputs = (_CTensor * max(1, len(ins)))(*ins)
        self.outs = (_CTensor * max(1, len(outs)))(*outs)
        self.attrs = self._attrs(req.attrs)
        self.args = self._attrs(req.args)
        self.req.inputs, self.req.n_inputs = self.inputs, len(ins)
        self.req.requested_outputs, self.req.n_requested_outputs = self.outs, len(outs)
        self.req.attrs, self.req.n_attrs = self.attrs[0], self.attrs[1]
        self.req.args, self.req.n_args = self.args[0], self.args[1]

    def _s(self, text):
        enc = str(text).encode()
        self.keep.append(enc)  # the C side points into this buffer
        return enc

    def _tensor(self, t: Tensor, payload: bool) -> _CTensor:
        c = _CTensor()
        c.name = self._s(t.name)
        c.dtype = dtype_code(t.dtype)
        c.storage_dtype = dtype_code(t.storage_dtype) if t.storage_dtype else nat.UNSPECIFIED
        if len(t.shape) > MAX_RANK:
            raise XrmmInvalid("Rank outside the supported range: " + t.name)
        c.rank = len(t.shape)
        for i, d in enumerate(t.shape):
            c.shape[i] = d
        if payload and t.data is not None:
            arr = np.ascontiguousarray(t.data)
            self.keep.append(arr)
            c.data = arr.ctypes.data if arr.nbytes else None
            c.nbytes = arr.nbytes
        return c

    def _attrs(self, d: dict):
        items = []
        for k, v in d.items():
            a = _CAttr()
            a.key = self._s(k)
            if isinstance(v, (bool, np.bool_)):
                a.kind, a.i = 0, int(v)
            elif isinstance(v, (int, np.integer)):
                a.kind, a.i = 0, int(v)
            elif isinstance(v, (float, np.floating)):
                a.kind, a.f = 1, float(v)
            elif isinstance(v, str):
                a.kind, a.s = 2, self._s(v)
            else:
                raise XrmmInvalid("Unsupported native attribute encoding: " + str(k))
            items.append(a)
        arr = (_CAttr * max(1, len(items)))(*items)
        self.keep.append(arr)
        return arr, len(items)


def _desc_to_tensor(d: _CDesc) -> Tensor:
    shape = tuple(d.shape[i] for i in range(d.rank))
    return Tensor(name=d.name.decode(), shape=shape, dtype=DTYPES[d.dtype], storage_dtype=DTYPES[d.storage_dtype])


def plan(request: Request) -> list:
    """extended::plan: validated output descriptors, no device work."""
    m = _Marshal(request)
    descs = (_CDesc * 8)()
    n = ctypes.c_int32(0)
    nat.check(_lib().xrmm_plan(ctypes.byref(m.req), descs, 8, ctypes.byref(n)))
    return [_desc_to_tensor(descs[i]) for i in range(n.value)]


class Operator:
    """extended_operators.h:49-61 Operator. Not thread-safe (one stream)."""

    def __init__(self, handle, request: Request):
        self._h = ctypes.c_void_p(handle)
        self.request = request

    @classmethod
    def prepare(cls, package_directory, request: Request, options: Options | None = None) -> "Operator":
        """``package_directory`` is accepted for signature parity; the kernels
        are linked into libxrmm.so, so there is no shader package to read."""
        options = options or Options()
        m = _Marshal(request)
        o = _COptions(int(options.profiling), int(options.timeout_ns), int(options.memory_limit_bytes))
        h = ctypes.c_void_p()
        nat.check(_lib().xrmm_prepare(ctypes.byref(m.req), ctypes.byref(o), ctypes.byref(h)))
        return cls(h.value, request)

    def _live(self):
        if not self._h:
            raise XrmmError("Extended native operator is closed")
        return self._h

    def run(self) -> None:
        nat.check(_lib().xrmm_run(self._live()))

    def output_descriptors(self) -> list:
        descs = (_CDesc * 8)()
        n = ctypes.c_int32(0)
        nat.check(_lib().xrmm_output_descs(self._live(), descs, 8, ctypes.byref(n)))
        return [_desc_to_tensor(descs[i]) for i in range(n.value)]

    def read_outputs(self) -> list:
        descs = self.output_descriptors()
        arrays = [np.empty(t.shape, dtype=_NP[t.storage_dtype]) for t in descs]
        ptrs = (ctypes.c_void_p * max(1, len(arrays)))(*[a.ctypes.data if a.nbytes else None for a in arrays])
        sizes = (ctypes.c_uint64 * max(1, len(arrays)))(*[a.nbytes for a in arrays])
        nat.check(_lib().xrmm_read_outputs(self._live(), ptrs, sizes, len(arrays)))
        for t, a in zip(descs, arrays):
            t.data = a
        return descs

    def info(self) -> dict:
        return json.loads(_lib().xrmm_info(self._live()).decode())

    def close(self) -> None:
        if self._h:
            nat.check(_lib().xrmm_close(self._h))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h:
            try:
                _lib().xrmm_destroy(h)
            except Exception:
                pass
            self._h = ctypes.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()
