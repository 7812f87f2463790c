"""Host-side mirror of rew's eager surface over librew_mi355x.

Same names and meaning as the reference:

* ``DType``            -- src/rew/dtype.nim:10-30 (same enum order = ABI codes)
* ``Device``/``mi355x`` -- src/rew/device.nim:19-56 plus the new target
* ``Tensor``           -- src/rew/tensor.nim:42-52 (dtype, shape, device, handle)
* ``setEagerBackend`` / ``clearEagerBackend`` / ``dispatchEager``
                       -- src/rew/dispatch.nim:47-85 (per-thread backend slot,
                          ``NoEagerBackendError`` when none is installed)
* ``installEagerBackend`` -- src/rew/eager.nim:1769-1772, selecting the
                          mi355x backend for an mi355x device
* ``fromHost`` / ``toHost`` -- src/rew/eager.nim:344-377, 558-595

Every op executes inside the native library; this module only moves
handles and host buffers across the C ABI.
"""
from __future__ import annotations

import ctypes as C
import enum
import threading
import weakref
from typing import Callable, Iterable, Sequence

import numpy as np

from . import _lib


class EagerError(RuntimeError):
    """Backend failure (src/rew/eager.nim EagerError)."""


class NoEagerBackendError(RuntimeError):
    """Eager op without an installed backend (src/rew/dispatch.nim:35-37)."""


class TensorError(ValueError):
    """Op-level validation error (src/rew/tensor.nim TensorError)."""


class BufferReleasedError(EagerError):
    """Use of a handle after its last release (src/rew/buffer.nim:166-173)."""


class TensorModeError(TensorError):
    """A trace tensor and an eager tensor met inside an op (src/rew/tensor.nim:37-40)."""


class BufferDonatedError(RuntimeError):
    """Use of an input buffer donated to a jit call (src/rew/buffer.nim:38, 146-164)."""


class DType(enum.IntEnum):
    BOOL = 0
    INT8 = 1
    INT16 = 2
    INT32 = 3
    INT64 = 4
    UINT8 = 5
    UINT16 = 6
    UINT32 = 7
    UINT64 = 8
    FLOAT16 = 9
    BFLOAT16 = 10
    FLOAT32 = 11
    FLOAT64 = 12
    COMPLEX64 = 13
    COMPLEX128 = 14
    INT4 = 15
    UINT4 = 16
    NF4 = 17
    FLOAT8E4M3FN = 18
    FLOAT8E5M2 = 19

    @property
    def byte_size(self) -> int:
        return _BYTE_SIZE[self]

    @property
    def rew_name(self) -> str:
        """Canonical name rew sends in dtype attrs ("float32")."""
        return _NAMES[self]

    @property
    def enum_name(self) -> str:
        """Nim enum spelling ("dtFloat32")."""
        return _ENUM_NAMES[self]


_BYTE_SIZE = {DType.BOOL: 1, DType.INT8: 1, DType.INT16: 2, DType.INT32: 4, DType.INT64: 8,
              DType.UINT8: 1, DType.UINT16: 2, DType.UINT32: 4, DType.UINT64: 8,
              DType.FLOAT16: 2, DType.BFLOAT16: 2, DType.FLOAT32: 4, DType.FLOAT64: 8,
              DType.COMPLEX64: 8, DType.COMPLEX128: 16, DType.INT4: 1, DType.UINT4: 1,
              DType.NF4: 1, DType.FLOAT8E4M3FN: 1, DType.FLOAT8E5M2: 1}
_NAMES = {DType.BOOL: "bool", DType.INT8: "int8", DType.INT16: "int16", DType.INT32: "int32",
          DType.INT64: "int64", DType.UINT8: "uint8", DType.UINT16: "uint16",
          DType.UINT32: "uint32", DType.UINT64: "uint64", DType.FLOAT16: "float16",
          DType.BFLOAT16: "bfloat16", DType.FLOAT32: "float32", DType.FLOAT64: "float64",
          DType.COMPLEX64: "complex64", DType.COMPLEX128: "complex128", DType.INT4: "int4",
          DType.UINT4: "uint4", DType.NF4: "nf4", DType.FLOAT8E4M3FN: "float8_e4m3fn",
          DType.FLOAT8E5M2: "float8_e5m2"}
_ENUM_NAMES = {d: "dt" + {"bfloat16": "BFloat16", "float8_e4m3fn": "Float8E4M3Fn",
                           "float8_e5m2": "Float8E5M2", "nf4": "NF4"}.get(
                               _NAMES[d], _NAMES[d][0].upper() + _NAMES[d][1:])
               for d in DType}

# numpy storage type per dtype (bf16 travels as its uint16 bit pattern)
_NP = {DType.BOOL: np.bool_, DType.INT8: np.int8, DType.INT16: np.int16,
       DType.INT32: np.int32, DType.INT64: np.int64, DType.UINT8: np.uint8,
       DType.UINT16: np.uint16, DType.UINT32: np.uint32, DType.UINT64: np.uint64,
       DType.FLOAT16: np.float16, DType.BFLOAT16: np.uint16, DType.FLOAT32: np.float32,
       DType.FLOAT64: np.float64, DType.COMPLEX64: np.complex64,
       DType.COMPLEX128: np.complex128}

float32 = DType.FLOAT32
bfloat16 = DType.BFLOAT16
int32 = DType.INT32


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even f32 -> bf16 bit patterns (NaN stays quiet NaN)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7F800000) == 0x7F800000
    nan &= (u & 0x007FFFFF) != 0
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
    r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


# ---- devices -----------------------------------------------------------------------


class Device:
    """(target, ordinal); ``str(d)`` is rew's "target:ordinal" form."""

    __slots__ = ("target", "ordinal", "_hash")

    def __init__(self, target: str = "mi355x", ordinal: int = 0):
        if ordinal < 0:
            raise ValueError(f"initDevice: ordinal must be non-negative, got {ordinal}")
        self.target = target
        self.ordinal = ordinal
        self._hash = hash((target, ordinal))

    def __eq__(self, other):
        return self is other or (isinstance(other, Device) and (self.target, self.ordinal) == (
            other.target, other.ordinal))

    def __hash__(self):
        return self._hash

    def __str__(self):
        return f"{self.target}:{self.ordinal}"

    __repr__ = __str__


def mi355x(ordinal: int = 0) -> Device:
    """The native MI355X target (new next to rew's ``rocm()``, device.nim:46-48)."""
    return Device("mi355x", ordinal)


_default_device = threading.local()


def setDefaultDevice(d: Device) -> None:
    _default_device.value = d


def defaultDevice() -> Device:
    return getattr(_default_device, "value", None) or mi355x(0)


# ---- context + tensors -------------------------------------------------------------

_ctxs: dict[int, C.c_void_p] = {}


def _check(rc: int, what: str = "") -> None:
    if rc == 0:
        return
    msg = _lib.load().rew_mi355x_last_error().decode(errors="replace")
    if rc == 5:
        raise BufferReleasedError(msg)
    if rc == 1:
        raise TensorError(msg) if what == "validate" else EagerError(msg)
    raise EagerError(msg)


def context(d: Device | None = None) -> C.c_void_p:
    d = d or defaultDevice()
    if d.target != "mi355x":
        raise EagerError(f"device {d} is not served by the mi355x backend")
    ctx = _ctxs.get(d.ordinal)
    if ctx is None:
        lib = _lib.load()
        ctx = C.c_void_p()
        _check(lib.rew_mi355x_init(d.ordinal, C.byref(ctx)))
        _ctxs[d.ordinal] = ctx
    return ctx


class Tensor:
    """Value tensor owning one reference to a native tensor record."""

    __slots__ = ("handle", "dtype", "shape", "device", "__weakref__")

    def __init__(self, handle: int, dtype: DType, shape: Sequence[int], device: Device):
        self.handle = handle
        self.dtype = DType(dtype)
        self.shape = tuple(int(s) for s in shape)
        self.device = device

    @classmethod
    def _make(cls, handle: int, dtype: DType, shape: tuple, device: Device) -> "Tensor":
        """Fast constructor for already-normalised fields (the dispatch path)."""
        t = cls.__new__(cls)
        t.handle = handle
        t.dtype = dtype
        t.shape = shape
        t.device = device
        return t

    def __del__(self):
        h = getattr(self, "handle", None)
        if h and _lib._lib is not None:
            _lib._lib.rew_mi355x_release(h)
            self.handle = None

    @property
    def numElements(self) -> int:
        n = 1
        for s in self.shape:
            n *= s
        return n

    def __repr__(self):
        return f"Tensor({self.dtype.enum_name}, {list(self.shape)}, {self.device})"


# tensors whose buffers went to a jit call as donations, with the consumer
_donated: "weakref.WeakKeyDictionary[Tensor, str]" = weakref.WeakKeyDictionary()


def markDonated(t: Tensor, consumer: str) -> None:
    """Hands t's buffer to `consumer` (src/rew/buffer.nim:146-156): the
    native reference is dropped and later use raises BufferDonatedError."""
    _donated[t] = consumer
    h, t.handle = t.handle, None
    if h and _lib._lib is not None:
        _lib._lib.rew_mi355x_release(h)


def _raise_released(t: Tensor, what: str):
    """src/rew/buffer.nim:158-173 (requireLive); a trace tensor here is the
    mode error of requireEager (src/rew/tensor.nim:93-100)."""
    if hasattr(t, "traceId"):
        raise TensorModeError(f"{what}: expected an eager tensor, got a trace tensor")
    by = _donated.get(t)
    if by is not None:
        raise BufferDonatedError(
            f"{what}: buffer has been donated and may no longer be used (donated to: {by})")
    raise BufferReleasedError(f"{what}: tensor already released")


def _wrap(handle: int, d: Device) -> Tensor:
    lib = _lib.load()
    dt = C.c_int()
    rank = C.c_int()
    shape = (C.c_int64 * 8)()
    _check(lib.rew_mi355x_buf_meta(handle, C.byref(dt), C.byref(rank), shape))
    return Tensor(handle, DType(dt.value), [shape[i] for i in range(rank.value)], d)


def fromHost(data, dtype: DType | None = None, shape: Sequence[int] | None = None,
             device: Device | None = None) -> Tensor:
    """Copies host data to a new device tensor (eager.nim transferToDevice).

    ``data`` is a numpy array (or anything ``np.asarray`` accepts).  For
    ``dtype=bfloat16`` a float array is rounded (RNE) and a uint16 array is
    taken as raw bf16 bits.
    """
    d = device or defaultDevice()
    arr = np.asarray(data)
    if dtype is None:
        dtype = {np.dtype(np.float32): DType.FLOAT32, np.dtype(np.int32): DType.INT32,
                 np.dtype(np.bool_): DType.BOOL, np.dtype(np.uint32): DType.UINT32,
                 np.dtype(np.float16): DType.FLOAT16, np.dtype(np.int8): DType.INT8,
                 np.dtype(np.uint8): DType.UINT8, np.dtype(np.int16): DType.INT16,
                 np.dtype(np.uint16): DType.UINT16, np.dtype(np.int64): DType.INT64,
                 np.dtype(np.float64): DType.FLOAT64,
                 np.dtype(np.uint64): DType.UINT64,
                 np.dtype(np.complex64): DType.COMPLEX64,
                 np.dtype(np.complex128): DType.COMPLEX128}.get(arr.dtype)
        if dtype is None:
            raise TensorError(f"fromHost: unsupported host dtype {arr.dtype}")
    dtype = DType(dtype)
    shp = tuple(arr.shape) if shape is None else tuple(shape)  # (0-d stays 0-d below)
    if dtype == DType.BFLOAT16 and arr.dtype != np.uint16:
        arr = f32_to_bf16_bits(arr.astype(np.float32))
    else:
        arr = arr.astype(_NP[dtype], copy=False)
    arr = np.ascontiguousarray(arr)
    n = 1
    for s in shp:
        n *= s
    if n != arr.size:
        raise TensorError(f"fromHost: data length {arr.size} does not match shape {list(shp)}")
    lib = _lib.load()
    cshape = (C.c_int64 * max(1, len(shp)))(*shp)
    h = C.c_void_p()
    _check(lib.rew_mi355x_from_host(context(d), int(dtype), cshape, len(shp),
                                    arr.ctypes.data_as(C.c_void_p), arr.nbytes, C.byref(h)))
    return Tensor(h.value, dtype, shp, d)


def toHost(t: Tensor) -> np.ndarray:
    """Blocking device-to-host copy (flushes pending work).

    bf16 tensors come back as their uint16 bit pattern; use
    ``bf16_bits_to_f32`` to widen.
    """
    if t.handle is None:
        _raise_released(t, "toHost")
    out = np.empty(t.shape, dtype=_NP[t.dtype])
    _check(_lib.load().rew_mi355x_to_host(t.handle, out.ctypes.data_as(C.c_void_p),
                                           out.nbytes))
    return out


def empty(dtype: DType, shape: Sequence[int], device: Device | None = None) -> Tensor:
    """A new tensor with undefined contents (rew_mi355x_alloc), to be written
    on the device by a caller holding its address (``devicePtr``)."""
    d = device or defaultDevice()
    shp = tuple(int(s) for s in shape)
    cshape = (C.c_int64 * max(1, len(shp)))(*shp)
    h = C.c_void_p()
    _check(_lib.load().rew_mi355x_alloc(context(d), int(dtype), cshape, len(shp), C.byref(h)))
    return Tensor(h.value, DType(dtype), shp, d)


def devicePtr(t: Tensor) -> int:
    """Device address of t's storage (rew_mi355x_buf_device_ptr; flushes t's producer)."""
    if t.handle is None:
        _raise_released(t, "devicePtr")
    p = C.c_void_p()
    _check(_lib.load().rew_mi355x_buf_device_ptr(t.handle, C.byref(p)))
    return int(p.value or 0)


def _moe_args(x: Tensor, start: Tensor, topWeights: Tensor, topIndices: Tensor,
              experts: Sequence, expertIds: Sequence[int], routerWidth: int, out: Tensor):
    """Fills rew_mi355x_moe_args from backend tensors; returns (args, keepalive)."""
    T, H = x.shape
    ffn = experts[0].gateProj.weight.shape[1]
    n = len(experts)
    tables = []
    for attr, part in (("gateProj", "weight"), ("upProj", "weight"), ("gateProj", "bias"),
                       ("upProj", "bias"), ("downProj", "weight"), ("downProj", "bias")):
        tables.append((C.c_void_p * n)(*[devicePtr(getattr(getattr(e, attr), part))
                                        for e in experts]))
    ids = (C.c_int32 * n)(*[int(i) for i in expertIds])
    a = _lib.MoeArgs()
    a.x, a.x_row_stride = devicePtr(x), H
    a.start, a.start_row_stride = devicePtr(start), H
    a.top_ids, a.top_weights = devicePtr(topIndices), devicePtr(topWeights)
    a.tokens, a.hidden, a.ffn = T, H, ffn
    a.k, a.router_width, a.n_experts = topIndices.shape[1], int(routerWidth), n
    a.expert_ids = C.cast(ids, C.c_void_p)
    (a.gate_w, a.up_w, a.gate_b, a.up_b, a.down_w, a.down_b) = [C.cast(t, C.c_void_p)
                                                                for t in tables]
    a.out = devicePtr(out)
    return a, (tables, ids)


def moeRoutedFfn(x: Tensor, start: Tensor, topWeights: Tensor, topIndices: Tensor,
                 experts: Sequence, expertIds: Sequence[int], routerWidth: int) -> Tensor:
    """The routed experts of DeepSeekMoE.forward on the router's top-k
    (rew_mi355x_moe_routed_ffn): start + the chain of routed expert FFNs,
    each on its routed tokens only.  ``experts`` hold gateProj / upProj /
    downProj Linears over bf16 tensors."""
    out = empty(DType.BFLOAT16, x.shape, x.device)
    a, keep = _moe_args(x, start, topWeights, topIndices, experts, expertIds, routerWidth, out)
    _check(_lib.load().rew_mi355x_moe_routed_ffn(context(x.device), C.byref(a)))
    return out


def toHostF32(t: Tensor) -> np.ndarray:
    a = toHost(t)
    if t.dtype == DType.BFLOAT16:
        return bf16_bits_to_f32(a).reshape(t.shape)
    return a.astype(np.float32)


def flush(d: Device | None = None) -> None:
    """Launches every pending op of the device (asynchronous)."""
    _check(_lib.load().rew_mi355x_flush(context(d)))


def sync(d: Device | None = None) -> None:
    """Flushes and waits for the device."""
    _check(_lib.load().rew_mi355x_sync(context(d)))


MODE_DEFERRED = 0
MODE_OP_BY_OP = 1


def setMode(mode: int, d: Device | None = None) -> None:
    _check(_lib.load().rew_mi355x_set_mode(context(d), mode))


def stats(d: Device | None = None) -> dict:
    s = _lib.Stats()
    _check(_lib.load().rew_mi355x_get_stats(context(d), C.byref(s)))
    return {n: getattr(s, n) for n, _ in _lib.Stats._fields_}


def resetStats(d: Device | None = None) -> None:
    _check(_lib.load().rew_mi355x_reset_stats(context(d)))


def clearEagerCache(d: Device | None = None) -> None:
    """src/rew/eager.nim:1713-1715: drops the backend's cached state (here the
    device copies of small constants)."""
    _check(_lib.load().rew_mi355x_clear_cache(context(d)))


# ---- dispatcher (src/rew/dispatch.nim:47-85) ---------------------------------------

EagerBackend = Callable[[str, Sequence[Tensor], Sequence[tuple]], list]
_slot = threading.local()


def setEagerBackend(backend: EagerBackend) -> None:
    _slot.backend = backend


def clearEagerBackend() -> None:
    _slot.backend = None


def dispatchEager(op: str, operands: Sequence[Tensor] = (),
                  attrs: Iterable[tuple[str, str]] = ()) -> list:
    be = getattr(_slot, "backend", None)
    if be is None:
        raise NoEagerBackendError(
            f"eager op '{op}': no PJRT execution backend registered. call "
            "installEagerBackend() after selecting a PJRT device, or use trace "
            "mode (`withTrace`) for lowering only.")
    return be(op, operands, list(attrs))


_META = 2 + 8  # per output: dtype, rank, 8 dims (rew_mi355x_execute_ex)
_DTYPE_OF = {int(d): d for d in DType}
_enc_cache: dict = {}


def _enc(s) -> bytes:
    b = _enc_cache.get(s)
    if b is None:
        b = str(s).encode()
        if len(_enc_cache) < 65536:
            _enc_cache[s] = b
    return b


class _Scratch(threading.local):
    """Per-thread ctypes buffers reused by every dispatch."""

    def __init__(self):
        self.ops = (C.c_void_p * 16)()
        self.keys = (C.c_char_p * 16)()
        self.vals = (C.c_char_p * 16)()
        self.outs = (C.c_void_p * 4)()
        self.nout = C.c_int()
        self.meta = (C.c_int64 * (4 * _META))()


_scratch = _Scratch()


def executeMi355xOp(op: str, operands: Sequence[Tensor],
                    attrs: Sequence[tuple[str, str]]) -> list:
    """The mi355x EagerBackend (counterpart of executeEagerOp, eager.nim:1717-1767)."""
    if operands:
        d = operands[0].device
    else:
        d = defaultDevice()
        for k, v in attrs:
            if k == "device":
                tgt, _, o = v.partition(":")
                d = Device(tgt or "mi355x", int(o or 0))
    for t in operands:
        if t.device is not d and t.device != d:
            raise EagerError(f"eager '{op}': cross-device operands forbidden")
        if t.handle is None:
            _raise_released(t, f"eager '{op}'")
    lib = _lib.load()
    sc = _scratch
    n, na = len(operands), len(attrs)
    ops = sc.ops if n <= 16 else (C.c_void_p * n)()
    for i, t in enumerate(operands):
        ops[i] = t.handle
    keys = sc.keys if na <= 16 else (C.c_char_p * na)()
    vals = sc.vals if na <= 16 else (C.c_char_p * na)()
    for i, (k, v) in enumerate(attrs):
        keys[i] = _enc(k)
        vals[i] = _enc(v)
    rc = lib.rew_mi355x_execute_ex(context(d), _enc(op), ops, n, keys, vals, na, sc.outs, 4,
                                   C.byref(sc.nout), sc.meta)
    _check(rc)
    res = []
    meta = sc.meta
    for i in range(sc.nout.value):
        m = i * _META
        res.append(Tensor._make(sc.outs[i], _DTYPE_OF[meta[m]],
                                tuple(meta[m + 2:m + 2 + meta[m + 1]]), d))
    return res


def installEagerBackend(device: Device | None = None) -> None:
    """Installs the mi355x backend for this thread (idempotent)."""
    d = device or defaultDevice()
    if d.target != "mi355x":
        raise EagerError(f"installEagerBackend: {d} is not an mi355x device")
    context(d)
    setEagerBackend(executeMi355xOp)


def deviceCount() -> int:
    n = C.c_int()
    _check(_lib.load().rew_mi355x_device_count(C.byref(n)))
    return n.value


# ---- kernel timing hooks (rew_mi355x_profile_*) ----------------------------------------

def profileBegin(d: Device | None = None) -> None:
    """Starts bracketing every kernel launch with HIP events on the backend stream."""
    _check(_lib.load().rew_mi355x_profile_begin(context(d)))


def profileEnd(d: Device | None = None) -> list:
    """Stops profiling; returns [(kernel name, launches, total device ms)]."""
    lib = _lib.load()
    ctx = context(d)
    _check(lib.rew_mi355x_profile_end(ctx))
    out = []
    name = C.create_string_buffer(256)
    n = C.c_int64()
    ms = C.c_double()
    i = 0
    while lib.rew_mi355x_profile_entry(ctx, i, name, 256, C.byref(n), C.byref(ms)) == 0:
        out.append((name.value.decode(), int(n.value), float(ms.value)))
        i += 1
    return out
