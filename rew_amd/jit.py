"""Trace mode, ``jit`` and ``lazy`` over the mi355x backend.

Mirror of rew's runtime tracing and its jit execution path:

* ``withTrace`` / ``currentMode``  -- src/rew/dispatch.nim:86-119: inside a
  trace every op builds a StableHLO op instead of executing;
* the per-op trace lowering the ``{.rewOp.}`` procs do in trace mode
  (src/rew/ops/*.nim ``of dmTrace`` branches), written as the text rew's
  emitter prints (src/rew/stablehlo/text.nim) -- same mnemonics, forms and
  ``%v<id>`` numbering (arguments 1..n, then every value in creation order,
  region arguments before their region's ops);
* ``topK`` traced as rew traces it (src/rew/ops/sort.nim:53-85: a stable
  sort with a GE/LE comparator plus a slice, and a second sort of
  ``(x, iota)`` for the indices);
* ``jit`` / ``JitFunction`` -- src/rew/transform/jit.nim:1-229 (per-signature
  cache, ``text``, ``executableText`` with the entry renamed ``main``,
  ``call``);
* ``lazy`` / ``LazyFunction`` / ``lazyCall`` -- src/rew/transform/lazy.nim:17-52;
* ``executeJit`` / ``clearJitCache`` -- src/rew/eager.nim:1774-1847, backed by
  ``rew_mi355x_execute_jit`` (the native library parses the text, caches the
  translated module and runs it through its deferred graph).
"""
from __future__ import annotations

import ctypes as C
import operator
import struct
import threading
from contextlib import contextmanager
from typing import Callable, Sequence

import numpy as np

from . import _lib
from .eager import (DType, Device, EagerError, Tensor, TensorError, TensorModeError,
                    _check, _DTYPE_OF, _NP, _META, _raise_released, context,
                    f32_to_bf16_bits, markDonated)

# MLIR element types (src/rew/stablehlo/text.nim:20-46)
_ELEM = {DType.BOOL: "i1", DType.INT8: "i8", DType.INT16: "i16", DType.INT32: "i32",
         DType.INT64: "i64", DType.UINT8: "ui8", DType.UINT16: "ui16", DType.UINT32: "ui32",
         DType.UINT64: "ui64", DType.FLOAT16: "f16", DType.BFLOAT16: "bf16",
         DType.FLOAT32: "f32", DType.FLOAT64: "f64", DType.COMPLEX64: "complex<f32>",
         DType.COMPLEX128: "complex<f64>", DType.INT4: "i4", DType.UINT4: "ui4",
         DType.NF4: "i4", DType.FLOAT8E4M3FN: "f8E4M3FN", DType.FLOAT8E5M2: "f8E5M2"}

# eager op name -> StableHLO mnemonic (src/rew/stablehlo/text.nim:145-263)
_BINARY = {"add": "add", "sub": "subtract", "mul": "multiply", "divide": "divide",
           "maximum": "maximum", "minimum": "minimum", "power": "power",
           "remainder": "remainder", "atan2": "atan2", "bitwiseAnd": "and",
           "bitwiseOr": "or", "bitwiseXor": "xor", "shiftLeft": "shift_left",
           "shiftRightArithmetic": "shift_right_arithmetic",
           "shiftRightLogical": "shift_right_logical"}
_UNARY = {"neg": "negate", "abs": "abs", "exp": "exponential", "log": "log", "sqrt": "sqrt",
          "rsqrt": "rsqrt", "tanh": "tanh", "logistic": "logistic", "sine": "sine",
          "cosine": "cosine", "floor": "floor", "ceil": "ceil", "sign": "sign", "cbrt": "cbrt",
          "expm1": "exponential_minus_one", "log1p": "log_plus_one", "tan": "tan",
          "roundNearestAfz": "round_nearest_afz", "roundNearestEven": "round_nearest_even",
          "bitwiseNot": "not", "countLeadingZeros": "count_leading_zeros",
          "popcnt": "popcnt"}
_REDUCE = {"reduceSum": ("add", 0.0), "reduceMax": ("maximum", float("-inf")),
           "reduceMin": ("minimum", float("inf")), "reduceProd": ("multiply", 1.0)}


def _ty(dtype: DType, shape: Sequence[int]) -> str:
    """mlirTensorType (src/rew/stablehlo/text.nim:48-57)."""
    e = _ELEM[DType(dtype)]
    if not shape:
        return f"tensor<{e}>"
    return "tensor<" + "".join(f"{d}x" for d in shape) + e + ">"


def _list(xs) -> str:
    return "[" + ", ".join(str(int(x)) for x in xs) + "]"


def _ints(s: str) -> list[int]:
    """Parses the wire-format int lists the ops send ("[1,2]", "@[1, 2]")."""
    t = s.strip().lstrip("@").strip()
    body = t[1:-1].strip()
    return [int(x) for x in body.split(",")] if body else []


class TraceTensor(Tensor):
    """A trace-mode tensor: an SSA id in the active trace (src/rew/tensor.nim:112-127)."""

    __slots__ = ("traceId", "trace")

    def __init__(self, trace: "TraceContext", traceId: int, dtype: DType,
                 shape: Sequence[int], device: Device):
        self.handle = None
        self.dtype = DType(dtype)
        self.shape = tuple(int(s) for s in shape)
        self.device = device
        self.traceId = traceId
        self.trace = trace

    def __del__(self):
        pass

    def __repr__(self):
        return f"TraceTensor(%v{self.traceId}, {self.dtype.enum_name}, {list(self.shape)})"


class TraceContext:
    """One traced function being built (src/rew/dispatch.nim:86-103)."""

    def __init__(self, funcName: str, device: Device):
        self.funcName = funcName
        self.device = device
        self.moduleName = "trace_module"
        self.next_id = 1
        self.args: list[TraceTensor] = []
        self.lines: list[str] = []
        self.outputs: list[TraceTensor] | None = None

    def fresh(self) -> int:
        i = self.next_id
        self.next_id += 1
        return i

    def value(self, dtype, shape) -> TraceTensor:
        return TraceTensor(self, self.fresh(), dtype, shape, self.device)

    def text(self, entry: str | None = None) -> str:
        """emitText (src/rew/stablehlo/text.nim:1969-2025)."""
        if self.outputs is None:
            raise TensorError("trace: function has no return")
        args = ", ".join(f"%v{a.traceId}: {_ty(a.dtype, a.shape)}" for a in self.args)
        outs = [_ty(o.dtype, o.shape) for o in self.outputs]
        sig = ""
        if outs:
            sig = " -> " + (outs[0] if len(outs) == 1 else "(" + ", ".join(outs) + ")")
        ret = "    func.return"
        if self.outputs:
            ret += (" " + ", ".join(f"%v{o.traceId}" for o in self.outputs) + " : "
                    + ", ".join(outs))
        return (f"module @{self.moduleName} {{\n"
                f"  func.func @{entry or self.funcName}({args}){sig} {{\n"
                + "".join(line + "\n" for line in self.lines)
                + ret + "\n  }\n}\n")


_tls = threading.local()


def currentTrace() -> TraceContext | None:
    return getattr(_tls, "trace", None)


def currentMode() -> str:
    """"trace" inside withTrace, else "eager" (src/rew/dispatch.nim:52-58)."""
    return "trace" if getattr(_tls, "trace", None) is not None else "eager"


@contextmanager
def withTrace(funcName: str, device: Device):
    """src/rew/dispatch.nim:105-119."""
    ctx = TraceContext(funcName, device)
    prev = currentTrace()
    _tls.trace = ctx
    try:
        yield ctx
    finally:
        _tls.trace = prev


def traceInputs(ctx: TraceContext, dtypes: Sequence[DType],
                shapes: Sequence[Sequence[int]]) -> list[TraceTensor]:
    """src/rew/dispatch.nim:121-144: one argument per (dtype, shape)."""
    ctx.args = [ctx.value(dt, sh) for dt, sh in zip(dtypes, shapes)]
    return list(ctx.args)


def traceReturn(ctx: TraceContext, results: Sequence[Tensor]) -> None:
    """src/rew/dispatch.nim:155-172."""
    for t in results:
        _require_trace(ctx, t, "traceReturn")
    ctx.outputs = list(results)


def _require_trace(ctx: TraceContext, t: Tensor, op: str) -> None:
    """requireTrace (src/rew/tensor.nim:102-110)."""
    if not isinstance(t, TraceTensor) or t.trace is not ctx:
        raise TensorModeError(f"{op}: expected a trace tensor, got an eager tensor")


# ---- per-op trace lowering ---------------------------------------------------------

def _emit_constant(ctx: TraceContext, dtype: DType, shape: Sequence[int],
                   raw: bytes) -> TraceTensor:
    """builder.constant (src/rew/stablehlo/text.nim:354-373: dense raw bytes)."""
    r = ctx.value(dtype, shape)
    ctx.lines.append(f"    %v{r.traceId} = stablehlo.constant dense<\"0x{raw.hex().upper()}\"> : "
                     f"{_ty(dtype, shape)}")
    return r


def traceConstant(dtype: DType, shape: Sequence[int], data) -> TraceTensor:
    """The trace branch of rew's literals (src/rew/ops/literal.nim:56-77)."""
    ctx = currentTrace()
    dtype = DType(dtype)
    arr = np.asarray(data)
    if dtype == DType.BFLOAT16 and arr.dtype != np.uint16:
        arr = f32_to_bf16_bits(arr.astype(np.float32))
    else:
        arr = arr.astype(_NP[dtype], copy=False)
    n = 1
    for s in shape:
        n *= int(s)
    if arr.size != n:
        raise TensorError(f"constant: data length {arr.size} does not match shape {list(shape)}")
    return _emit_constant(ctx, dtype, shape, np.ascontiguousarray(arr).tobytes())


def _elementwise(ctx, mn, args, dtype, shape):
    r = ctx.value(dtype, shape)
    ctx.lines.append(f"    %v{r.traceId} = stablehlo.{mn} "
                     + ", ".join(f"%v{a.traceId}" for a in args) + f" : {_ty(dtype, shape)}")
    return r


def _typed(ctx, mn, a, extra, dtype, shape, quoted=False):
    """`%r = stablehlo.<mn> %a<extra> : (Tin) -> Tout` (or the quoted form)."""
    r = ctx.value(dtype, shape)
    if quoted:
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.{mn}\"(%v{a.traceId}) : "
                         f"({_ty(a.dtype, a.shape)}) -> {_ty(dtype, shape)}")
    else:
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.{mn} %v{a.traceId}{extra} : "
                         f"({_ty(a.dtype, a.shape)}) -> {_ty(dtype, shape)}")
    return r


def _sig(args, out):
    return "(" + ", ".join(_ty(a.dtype, a.shape) for a in args) + f") -> {out}"


def _reduce(ctx, op, x, dims):
    """reductionImpl (src/rew/ops/reduce.nim:93-117; text.nim:284-334)."""
    mn, init = _REDUCE[op]
    c = _emit_constant(ctx, x.dtype, [], struct.pack("<f", init))
    a, b = ctx.fresh(), ctx.fresh()
    body = ctx.fresh()
    rd = set(dims)
    shape = [d for i, d in enumerate(x.shape) if i not in rd]
    r = ctx.value(x.dtype, shape)
    s = _ty(x.dtype, [])
    ctx.lines += [
        f"    %v{r.traceId} = stablehlo.reduce(%v{x.traceId} init: %v{c.traceId}) across "
        f"dimensions = {_list(dims)} : ({_ty(x.dtype, x.shape)}, {s}) -> {_ty(x.dtype, shape)}",
        f"      reducer(%v{a}: {s}, %v{b}: {s}) {{",
        f"        %v{body} = stablehlo.{mn} %v{a}, %v{b} : {s}",
        f"        stablehlo.return %v{body} : {s}",
        "      }"]
    return r


def _sort(ctx, inputs, dim, stable, direction):
    """builder.sort with a one-compare comparator (src/rew/stablehlo/ops.nim:1438-1469;
    text.nim:1805-1866 generic form)."""
    region = []
    for t in inputs:
        region += [(ctx.fresh(), t.dtype), (ctx.fresh(), t.dtype)]
    cmp = ctx.fresh()
    res = [ctx.value(t.dtype, t.shape) for t in inputs]
    s0 = _ty(inputs[0].dtype, [])
    types = [_ty(t.dtype, t.shape) for t in inputs]
    rt = types[0] if len(types) == 1 else "(" + ", ".join(types) + ")"
    ctx.lines += [
        "    " + ", ".join(f"%v{r.traceId}" for r in res) + " = \"stablehlo.sort\"("
        + ", ".join(f"%v{t.traceId}" for t in inputs) + ") ({",
        "      ^bb0(" + ", ".join(f"%v{i}: {_ty(dt, [])}" for i, dt in region) + "):",
        f"        %v{cmp} = stablehlo.compare {direction}, %v{region[0][0]}, %v{region[1][0]} : "
        f"({s0}, {s0}) -> tensor<i1>",
        f"        stablehlo.return %v{cmp} : tensor<i1>",
        "    }) {dimension = " + str(dim) + " : i64, is_stable = "
        + ("true" if stable else "false") + "} : ("
        + ", ".join(types) + f") -> {rt}"]
    return res


def traceOp(op: str, operands: Sequence[Tensor], attrs: Sequence[tuple]) -> list:
    """Trace-mode lowering of one eager op name with its wire-format attrs."""
    ctx = currentTrace()
    for t in operands:
        _require_trace(ctx, t, op)
    a = dict(attrs)
    x = operands[0] if operands else None
    if op in _BINARY:
        return [_elementwise(ctx, _BINARY[op], operands, x.dtype, x.shape)]
    if op in _UNARY:
        return [_elementwise(ctx, _UNARY[op], operands, x.dtype, x.shape)]
    if op == "isFinite":
        return [_typed(ctx, "is_finite", x, "", DType.BOOL, x.shape, quoted=True)]
    if op == "astype":
        dt = _parse_dtype(a["dtype"])
        return [_typed(ctx, "convert", x, "", dt, x.shape, quoted=True)]
    if op == "reshape":
        return [_typed(ctx, "reshape", x, "", x.dtype, _ints(a["shape"]))]
    if op == "transpose":
        perm = _ints(a["permutation"])
        return [_typed(ctx, "transpose", x, f", dims = {_list(perm)}", x.dtype,
                       [x.shape[p] for p in perm])]
    if op == "reverse":
        dims = _ints(a["dimensions"])
        r = ctx.value(x.dtype, x.shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.reverse %v{x.traceId}, dims = "
                         f"{_list(dims)} : {_ty(x.dtype, x.shape)}")
        return [r]
    if op == "broadcastTo":
        return [_typed(ctx, "broadcast_in_dim", x, f", dims = {_list(_ints(a['broadcast_dimensions']))}",
                       x.dtype, _ints(a["output_shape"]))]
    if op == "slice":
        st, li = _ints(a["start_indices"]), _ints(a["limit_indices"])
        sd = _ints(a["strides"]) if "strides" in a else [1] * len(st)
        rng = ", ".join(f"{s}:{l}" + (f":{k}" if k != 1 else "") for s, l, k in zip(st, li, sd))
        shape = [(l - s + k - 1) // k for s, l, k in zip(st, li, sd)]
        r = ctx.value(x.dtype, shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.slice %v{x.traceId} [{rng}] : "
                         f"({_ty(x.dtype, x.shape)}) -> {_ty(x.dtype, shape)}")
        return [r]
    if op in ("pad", "dynamicSlice", "dynamicUpdateSlice"):
        # rew's generic forms (src/rew/stablehlo/text.nim:589-690)
        arr = lambda xs: "array<i64: " + ", ".join(str(int(v)) for v in xs) + ">"
        args = ", ".join(f"%v{t.traceId}" for t in operands)
        if op == "pad":
            lo, hi, it = (_ints(a[k]) for k in ("edge_padding_low", "edge_padding_high",
                                                "interior_padding"))
            shape = [d + l + h + max(d - 1, 0) * i for d, l, h, i in zip(x.shape, lo, hi, it)]
            attrs_s = (f" {{edge_padding_low = {arr(lo)}, edge_padding_high = {arr(hi)}, "
                       f"interior_padding = {arr(it)}}}")
            mn = "pad"
        elif op == "dynamicSlice":
            shape = _ints(a["slice_sizes"])
            attrs_s, mn = f" {{slice_sizes = {arr(shape)}}}", "dynamic_slice"
        else:
            shape, attrs_s, mn = list(x.shape), "", "dynamic_update_slice"
        r = ctx.value(x.dtype, shape)
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.{mn}\"({args}){attrs_s} : "
                         f"{_sig(list(operands), _ty(x.dtype, shape))}")
        return [r]
    if op in ("einsum", "unaryEinsum"):
        # emitEinsumAt (src/rew/stablehlo/text.nim:1696-1728)
        shape = _ints(a["output_shape"])
        r = ctx.value(x.dtype, shape)
        mn = "einsum" if op == "einsum" else "unary_einsum"
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.{mn}\"("
                         + ", ".join(f"%v{t.traceId}" for t in operands)
                         + f") {{einsum_config = \"{a['einsum_config']}\"}} : "
                         + _sig(list(operands), _ty(x.dtype, shape)))
        return [r]
    if op == "complex":
        # emitComplexAt (text.nim:826-838)
        dt = {DType.FLOAT32: DType.COMPLEX64, DType.FLOAT64: DType.COMPLEX128}[x.dtype]
        r = ctx.value(dt, x.shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.complex %v{x.traceId}, "
                         f"%v{operands[1].traceId} : {_ty(dt, x.shape)}")
        return [r]
    if op in ("real", "imag"):
        # emitTypeChangingUnaryAt (text.nim:390-406)
        dt = {DType.COMPLEX64: DType.FLOAT32, DType.COMPLEX128: DType.FLOAT64}.get(x.dtype, x.dtype)
        return [_typed(ctx, op, x, "", dt, x.shape, quoted=True)]
    if op == "fft":
        # emitFftAt (text.nim:1612-1638)
        fl = _ints(a["fft_length"])
        ty = a["fft_type"]
        shape = list(x.shape)
        cx = {DType.FLOAT32: DType.COMPLEX64, DType.FLOAT64: DType.COMPLEX128}
        rl = {DType.COMPLEX64: DType.FLOAT32, DType.COMPLEX128: DType.FLOAT64}
        dt = x.dtype
        if ty == "RFFT":
            shape[-1] = fl[-1] // 2 + 1
            dt = cx.get(x.dtype, x.dtype)
        elif ty == "IRFFT":
            shape[-1] = fl[-1]
            dt = rl.get(x.dtype, x.dtype)
        r = ctx.value(dt, shape)
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.fft\"(%v{x.traceId}) {{fft_type = "
                         f"#stablehlo<fft_type {ty}>, fft_length = [{', '.join(map(str, fl))}]}} : "
                         + _sig([x], _ty(dt, shape)))
        return [r]
    if op == "triangularSolve":
        # emitTriangularSolveAt (text.nim:1645-1695)
        b = operands[1]
        r = ctx.value(b.dtype, b.shape)
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.triangular_solve\"(%v{x.traceId}, "
                         f"%v{b.traceId}) {{left_side = {a['left_side']}, lower = {a['lower']}, "
                         f"unit_diagonal = {a['unit_diagonal']}, transpose_a = "
                         f"#stablehlo<transpose {a['transpose_a']}>}} : "
                         + _sig(list(operands), _ty(b.dtype, b.shape)))
        return [r]
    if op in ("dynamicPad", "realDynamicSlice"):
        # emitGenericVariadicAt (text.nim:780-801)
        shape = _ints(a["result_shape"])
        r = ctx.value(x.dtype, shape)
        mn = "dynamic_pad" if op == "dynamicPad" else "real_dynamic_slice"
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.{mn}\"("
                         + ", ".join(f"%v{t.traceId}" for t in operands) + ") : "
                         + _sig(list(operands), _ty(x.dtype, shape)))
        return [r]
    if op == "dynamicBroadcastInDim":
        # emitDynamicBroadcastInDimAt (text.nim:1575-1610)
        shape = _ints(a["result_shape"])
        r = ctx.value(x.dtype, shape)
        arr = lambda xs: "[" + ", ".join(str(int(v)) for v in xs) + "]"
        extra = ""
        for k, name in (("known_expanding_dimensions", "known_expanding_dimensions"),
                        ("known_nonexpanding_dimensions", "known_nonexpanding_dimensions")):
            if _ints(a.get(k, "[]")):
                extra += f", {name} = {arr(_ints(a[k]))}"
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.dynamic_broadcast_in_dim\"("
                         f"%v{x.traceId}, %v{operands[1].traceId}) {{broadcast_dimensions = "
                         f"{arr(_ints(a['broadcast_dimensions']))}{extra}}} : "
                         + _sig(list(operands), _ty(x.dtype, shape)))
        return [r]
    if op == "concat":
        d = int(a["dimension"])
        shape = list(x.shape)
        shape[d] = sum(t.shape[d] for t in operands)
        r = ctx.value(x.dtype, shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.concatenate "
                         + ", ".join(f"%v{t.traceId}" for t in operands)
                         + f", dim = {d} : {_sig(operands, _ty(x.dtype, shape))}")
        return [r]
    if op == "iota":
        dt = _parse_dtype(a["dtype"])
        shape = _ints(a["shape"])
        r = ctx.value(dt, shape)
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.iota\"() {{iota_dimension = "
                         f"{int(a['dimension'])} : i64}} : () -> {_ty(dt, shape)}")
        return [r]
    if op == "compare":
        r = ctx.value(DType.BOOL, x.shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.compare {a['comparison_direction']}, "
                         f"%v{x.traceId}, %v{operands[1].traceId} : "
                         f"{_sig(operands, _ty(DType.BOOL, x.shape))}")
        return [r]
    if op == "select":
        p, t = operands[0], operands[1]
        r = ctx.value(t.dtype, t.shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.select %v{p.traceId}, %v{t.traceId}, "
                         f"%v{operands[2].traceId} : {_ty(p.dtype, p.shape)}, "
                         f"{_ty(t.dtype, t.shape)}")
        return [r]
    if op == "clamp":
        v = operands[1]
        r = ctx.value(v.dtype, v.shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.clamp "
                         + ", ".join(f"%v{t.traceId}" for t in operands)
                         + f" : {_sig(operands, _ty(v.dtype, v.shape))}")
        return [r]
    if op in _REDUCE:
        return [_reduce(ctx, op, x, _ints(a["dims"]))]
    if op == "dotGeneral":
        b = operands[1]
        lb, rb = _ints(a["lhs_batching"]), _ints(a["rhs_batching"])
        lc, rc = _ints(a["lhs_contracting"]), _ints(a["rhs_contracting"])
        shape = ([x.shape[i] for i in lb]
                 + [d for i, d in enumerate(x.shape) if i not in lb and i not in lc]
                 + [d for i, d in enumerate(b.shape) if i not in rb and i not in rc])
        r = ctx.value(x.dtype, shape)
        ctx.lines.append(f"    %v{r.traceId} = stablehlo.dot_general %v{x.traceId}, "
                         f"%v{b.traceId}, batching_dims = {_list(lb)} x {_list(rb)}, "
                         f"contracting_dims = {_list(lc)} x {_list(rc)} : "
                         f"{_sig(operands, _ty(x.dtype, shape))}")
        return [r]
    if op == "dot":
        b = operands[1]
        shape = list(x.shape[:-1]) + list(b.shape[1:])
        r = ctx.value(x.dtype, shape)
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.dot\"(%v{x.traceId}, %v{b.traceId}) "
                         f": {_sig(operands, _ty(x.dtype, shape))}")
        return [r]
    if op == "torchIndexSelect":
        i = operands[1]
        d, bd = int(a["dim"]), int(a["batch_dims"])
        shape = list(x.shape[:d]) + list(i.shape[bd:]) + list(x.shape[d + 1:])
        r = ctx.value(x.dtype, shape)
        ctx.lines.append(f"    %v{r.traceId} = \"stablehlo.torch_index_select\"(%v{x.traceId}, "
                         f"%v{i.traceId}) {{dim = {d} : i64, batch_dims = {bd} : i64}} : "
                         f"{_sig(operands, _ty(x.dtype, shape))}")
        return [r]
    raise TensorError(f"{op}: no trace lowering in this mirror")


def _parse_dtype(s: str) -> DType:
    from .eager import _ENUM_NAMES, _NAMES
    s = s.strip()
    for d in DType:
        if s == _NAMES[d] or s == _ENUM_NAMES[d]:
            return d
    raise TensorError(f"unknown dtype attr '{s}'")


def traceSort(inputs: Sequence[Tensor], dim: int, stable: bool, direction: str) -> list:
    """sort's trace branch (src/rew/ops/sort.nim:18-31)."""
    ctx = currentTrace()
    for t in inputs:
        _require_trace(ctx, t, "sort")
    return _sort(ctx, list(inputs), dim, stable, direction)


def _region_body(ctx, dtype, op):
    """A two-argument scalar region returning op(a, b), or b for "replace"."""
    a, b = ctx.fresh(), ctx.fresh()
    s = _ty(dtype, [])
    head = f"      ^bb0(%v{a}: {s}, %v{b}: {s}):"
    if op == "replace":
        return [head, f"        stablehlo.return %v{b} : {s}"]
    c = ctx.fresh()
    return [head, f"        %v{c} = stablehlo.{op} %v{a}, %v{b} : {s}",
            f"        stablehlo.return %v{c} : {s}"]


def traceGather(operand, startIndices, dims, sliceSizes, resultShape, indicesAreSorted):
    """gather's trace branch (src/rew/ops/gather.nim:18-25; builder
    ops.nim:1387-1408, dims rendered as ops.nim:170-177)."""
    ctx = currentTrace()
    _require_trace(ctx, operand, "gather")
    _require_trace(ctx, startIndices, "gather")
    r = ctx.value(operand.dtype, resultShape)
    dn = (f"#stablehlo.gather<offset_dims = {_list(dims.offsetDims)}, collapsed_slice_dims = "
          f"{_list(dims.collapsedSliceDims)}, operand_batching_dims = "
          f"{_list(dims.operandBatchingDims)}, start_indices_batching_dims = "
          f"{_list(dims.startIndicesBatchingDims)}, start_index_map = "
          f"{_list(dims.startIndexMap)}, index_vector_dim = {int(dims.indexVectorDim)}>")
    ss = "array<i64: " + ", ".join(str(int(x)) for x in sliceSizes) + ">"
    ctx.lines.append(
        f"    %v{r.traceId} = \"stablehlo.gather\"(%v{operand.traceId}, %v{startIndices.traceId}) "
        f"{{dimension_numbers = {dn}, slice_sizes = {ss}, indices_are_sorted = "
        f"{'true' if indicesAreSorted else 'false'}}} : "
        f"{_sig([operand, startIndices], _ty(operand.dtype, resultShape))}")
    return r


def traceScatter(inputs, scatterIndices, updates, dims, op, indicesAreSorted, uniqueIndices):
    """scatter's trace branch (src/rew/ops/scatter.nim:20-37; builder
    ops.nim:1531-1569, dims rendered as ops.nim:179-188)."""
    ctx = currentTrace()
    for t in [*inputs, scatterIndices, *updates]:
        _require_trace(ctx, t, "scatter")
    if len(inputs) != 1:
        raise TensorError("scatter: the mirror traces one-input scatters only")
    body = _region_body(ctx, inputs[0].dtype, op)
    x = inputs[0]
    r = ctx.value(x.dtype, x.shape)
    dn = (f"#stablehlo.scatter<update_window_dims = {_list(dims.updateWindowDims)}, "
          f"inserted_window_dims = {_list(dims.insertedWindowDims)}, input_batching_dims = "
          f"{_list(dims.inputBatchingDims)}, scatter_indices_batching_dims = "
          f"{_list(dims.scatterIndicesBatchingDims)}, scatter_dims_to_operand_dims = "
          f"{_list(dims.scatterDimsToOperandDims)}, index_vector_dim = "
          f"{int(dims.indexVectorDim)}>")
    ops_ = [x, scatterIndices, updates[0]]
    ctx.lines += ([f"    %v{r.traceId} = \"stablehlo.scatter\"("
                   + ", ".join(f"%v{t.traceId}" for t in ops_) + ") ({"] + body
                  + ["    }) {scatter_dimension_numbers = " + dn + ", indices_are_sorted = "
                     + ("true" if indicesAreSorted else "false") + ", unique_indices = "
                     + ("true" if uniqueIndices else "false") + "} : "
                     + _sig(ops_, _ty(x.dtype, x.shape))])
    return [r]


def traceTopK(operand: Tensor, k: int, dim: int, largest: bool):
    """topK's trace branch (src/rew/ops/sort.nim:53-85)."""
    ctx = currentTrace()
    _require_trace(ctx, operand, "topK")
    direction = "GE" if largest else "LE"
    rank = len(operand.shape)
    (srt,) = _sort(ctx, [operand], dim, True, direction)
    starts = [0] * rank
    limits = [k if i == dim else operand.shape[i] for i in range(rank)]
    from . import ops as O
    values = O.slice_(srt, starts, limits, [1] * rank)
    idx = O.iota(DType.INT32, operand.shape, dim, operand.device)
    _, sidx = _sort(ctx, [operand, idx], dim, True, direction)
    indices = O.slice_(sidx, starts, limits, [1] * rank)
    return values, indices


# ---- jit (src/rew/transform/jit.nim) ----------------------------------------------

class JitError(RuntimeError):
    """src/rew/transform/jit.nim:74-76."""


JitFn = Callable[[Sequence[Tensor]], list]


def signatureOf(args: Sequence[Tensor]) -> str:
    """Cache key of one argument list (src/rew/transform/jit.nim:116-132):
    ``float32:[2,3]@mi355x:0#replicated|...``."""
    return "|".join(f"{a.dtype.rew_name}:[{','.join(str(d) for d in a.shape)}]@{a.device}"
                    "#replicated" for a in args)


# (dtype, shape, device) of a jit argument, and its native handle
_arg_sig = operator.attrgetter("dtype", "shape", "device")
_handle_of = operator.attrgetter("handle")


class JitCacheEntry:
    """Lowering of one input signature (src/rew/transform/jit.nim:51-63)."""

    __slots__ = ("trace", "text", "outDtypes", "outShapes", "signature", "_exec", "_exec_b")

    def __init__(self, trace: TraceContext, signature: str):
        self.trace = trace
        self.text = trace.text()
        self.outDtypes = [o.dtype for o in trace.outputs]
        self.outShapes = [list(o.shape) for o in trace.outputs]
        self.signature = signature
        self._exec = None
        self._exec_b = None

    def executableText(self) -> str:
        """The text with the entry function renamed ``main``
        (src/rew/transform/jit.nim:178-185)."""
        if self._exec is None:
            self._exec = self.trace.text(entry="main")
            self._exec_b = self._exec.encode()
        return self._exec


class JitFunction:
    """A traceable function with a per-signature cache
    (src/rew/transform/jit.nim:64-100)."""

    def __init__(self, fn: JitFn, funcName: str = "jit_fn", donateArgs: Sequence[int] = ()):
        self.fn = fn
        self.funcName = funcName
        self.donateArgs = [int(i) for i in donateArgs]
        self.cache: dict[str, JitCacheEntry] = {}
        self._fast: dict[tuple, JitCacheEntry] = {}
        # the last call's arguments and entry: the same tensor objects have
        # the same signature (dtype, shape and device never change), so a
        # call repeating them skips building the key.  Holds the last call's
        # inputs until the next call.
        self._last: tuple = ((), None)

    def _validate_donation(self, argCount: int) -> None:
        for idx in self.donateArgs:
            if idx < 0 or idx >= argCount:
                raise JitError(f"jit: donateArgs index {idx} out of range for {argCount} "
                               "input(s)")

    def _trace_once(self, args: Sequence[Tensor], sig: str) -> JitCacheEntry:
        """traceOnce (src/rew/transform/jit.nim:141-176)."""
        self._validate_donation(len(args))
        if not args:
            raise JitError("jit: at least one input required")
        dev = args[0].device
        for i, a in enumerate(args[1:], 1):
            if a.device != dev:
                raise JitError(f"jit: all inputs must share a device; arg 0 = {dev}, "
                               f"arg {i} = {a.device}")
        with withTrace(self.funcName, dev) as ctx:
            inputs = traceInputs(ctx, [a.dtype for a in args], [a.shape for a in args])
            outputs = list(self.fn(inputs))
            if not outputs:
                raise JitError("jit: function returned no outputs")
            traceReturn(ctx, outputs)
        return JitCacheEntry(ctx, sig)

    def compileFor(self, args: Sequence[Tensor]) -> JitCacheEntry:
        """The cache entry of this input signature, tracing on a miss."""
        prev, pe = self._last
        if pe is not None and len(prev) == len(args) and all(map(operator.is_, prev, args)):
            return pe
        fk = tuple(map(_arg_sig, args))
        e = self._fast.get(fk)
        if e is not None:
            self._last = (tuple(args), e)
            return e
        sig = signatureOf(args)
        e = self.cache.get(sig)
        if e is None:
            e = self._trace_once(args, sig)
            self.cache[sig] = e
        self._fast[fk] = e
        self._last = (tuple(args), e)
        return e

    def lower(self, args: Sequence[Tensor]) -> TraceContext:
        """The traced module of this signature (rew returns the ShModule)."""
        return self.compileFor(args).trace

    def text(self, args: Sequence[Tensor]) -> str:
        return self.compileFor(args).text

    def executableText(self, args: Sequence[Tensor]) -> str:
        return self.compileFor(args).executableText()

    def dumpHlo(self, args: Sequence[Tensor], path: str, executable: bool = False) -> str:
        """src/rew/transform/jit.nim:191-207."""
        import os
        d = os.path.dirname(path)
        if d:
            os.makedirs(d, exist_ok=True)
        with open(path, "w") as f:
            f.write(self.executableText(args) if executable else self.text(args))
        return path

    def cacheSize(self) -> int:
        return len(self.cache)

    def clearCache(self) -> None:
        self.cache.clear()
        self._fast.clear()
        self._last = ((), None)

    def call(self, args: Sequence[Tensor]) -> list:
        """Trace on a miss, then execute through the backend
        (src/rew/transform/jit.nim:209-229)."""
        e = self.compileFor(args)
        e.executableText()
        return _execute(self.funcName, e.signature, e._exec_b, args, e.outDtypes,
                        e.outShapes, self.donateArgs)


def jit(fn: JitFn, funcName: str = "jit_fn", donateArgs: Sequence[int] = ()) -> JitFunction:
    """src/rew/transform/jit.nim:80-100."""
    return JitFunction(fn, funcName, donateArgs)


# ---- lazy (src/rew/transform/lazy.nim) --------------------------------------------

class LazyFunction:
    """Cached lazy eager batch (src/rew/transform/lazy.nim:12-15)."""

    def __init__(self, compiled: JitFunction):
        self.compiled = compiled

    def call(self, args: Sequence[Tensor]) -> list:
        return self.compiled.call(args)

    def lower(self, args: Sequence[Tensor]) -> TraceContext:
        return self.compiled.lower(args)

    def text(self, args: Sequence[Tensor]) -> str:
        return self.compiled.text(args)

    def executableText(self, args: Sequence[Tensor]) -> str:
        return self.compiled.executableText(args)

    def cacheSize(self) -> int:
        return self.compiled.cacheSize()

    def clearCache(self) -> None:
        self.compiled.clearCache()


def lazy(fn: JitFn, funcName: str = "lazy_fn", donateArgs: Sequence[int] = ()) -> LazyFunction:
    """src/rew/transform/lazy.nim:17-27."""
    return LazyFunction(jit(fn, funcName, donateArgs))


def lazyCall(fn: JitFn, args: Sequence[Tensor], funcName: str = "lazy_fn",
             donateArgs: Sequence[int] = ()) -> list:
    """src/rew/transform/lazy.nim:49-52."""
    return lazy(fn, funcName, donateArgs).call(args)


# ---- execution (src/rew/eager.nim:1774-1847) --------------------------------------

def _execute(jitName: str, cacheKey: str, text: bytes, inputs: Sequence[Tensor],
             outDtypes: Sequence[DType], outShapes: Sequence[Sequence[int]],
             donateIdx: Sequence[int]) -> list:
    if not inputs:
        raise EagerError("executeJit: zero inputs")
    if len(outDtypes) != len(outShapes):
        raise EagerError("executeJit: outDtypes / outShapes length mismatch")
    d = inputs[0].device
    n = len(inputs)
    for t in inputs:
        if t.device is not d and t.device != d:
            raise EagerError(f"jit '{jitName}': cross-device inputs forbidden")
    handles = list(map(_handle_of, inputs))
    if None in handles:
        _raise_released(inputs[handles.index(None)], f"jit '{jitName}'")
    hs = (C.c_void_p * n)(*handles)
    for idx in donateIdx:
        if idx < 0 or idx >= n:
            raise EagerError(f"jit '{jitName}': donation index {idx} out of range")
    nd = len(donateIdx)
    don = (C.c_int * max(1, nd))(*donateIdx)
    m = max(1, len(outDtypes))
    outs = (C.c_void_p * m)()
    meta = (C.c_int64 * (m * _META))()
    nout = C.c_int()
    _check(_lib.load().rew_mi355x_execute_jit(
        context(d), jitName.encode(), cacheKey.encode(), text, len(text), hs, n, don, nd,
        outs, m, C.byref(nout), meta))
    res = []
    for i in range(nout.value):
        rank = meta[i * _META + 1]
        res.append(Tensor._make(outs[i], _DTYPE_OF[meta[i * _META]],
                                tuple(meta[i * _META + 2 + k] for k in range(rank)), d))
    if len(res) != len(outDtypes):
        raise EagerError(f"jit '{jitName}': backend returned {len(res)} output(s); trace "
                         f"expected {len(outDtypes)}")
    for i in donateIdx:
        markDonated(inputs[i], f"jit '{jitName}'")
    return res


def executeJit(jitName: str, cacheKey: str, moduleText: str, inputs: Sequence[Tensor],
               outDtypes: Sequence[DType], outShapes: Sequence[Sequence[int]],
               donateIdx: Sequence[int] = ()) -> list:
    """src/rew/eager.nim:1782-1847 over rew_mi355x_execute_jit."""
    return _execute(jitName, cacheKey, moduleText.encode(), inputs, outDtypes, outShapes,
                    donateIdx)


def clearJitCache() -> None:
    """src/rew/eager.nim:1776-1780: drops every context's translated modules."""
    from .eager import _ctxs
    for ctx in list(_ctxs.values()):
        _check(_lib.load().rew_mi355x_clear_jit_cache(ctx))
