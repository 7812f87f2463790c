"""Mirror of rew's eager ``{.rewOp.}`` procs used on the hot path.

Each function validates like the reference op, then calls ``dispatchEager``
with the same op name and the same stringly-typed attrs in the same wire
format, so the native backend sees exactly what rew would send it:

* ``joinInts`` lists "[a,b]" (src/rew/ops/linalg.nim:21-29, reduce.nim:87-92)
* Nim seq reprs "@[a, b]" for reshape/transpose/slice/iota shapes
  (src/rew/ops/shape.nim:41, 73; concat.nim:94-96; shape.nim:316-320)
* dtype names "float32" for astype (unary.nim:125), "dtInt32" for iota
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Sequence

import numpy as np

from . import jit as _jit
from .eager import (DType, Device, Tensor, TensorError, defaultDevice, dispatchEager,
                    fromHost)


def _join(xs: Sequence[int]) -> str:
    return "[" + ",".join(str(int(x)) for x in xs) + "]"


def _nimseq(xs: Sequence[int]) -> str:
    return "@[" + ", ".join(str(int(x)) for x in xs) + "]"


def _one(op, operands, attrs=()):
    if _jit._tls.__dict__.get("trace") is not None:   # trace mode: build the op
        return _jit.traceOp(op, operands, attrs)[0]
    outs = dispatchEager(op, operands, attrs)
    assert len(outs) == 1, f"{op}: eager backend returned wrong arity"
    return outs[0]


def _same(a: Tensor, b: Tensor, op: str):
    # src/rew/ops/arith.nim:21-28
    if a.device != b.device:
        raise TensorError(f"{op}: device mismatch")
    if a.dtype != b.dtype:
        raise TensorError(f"{op}: dtype mismatch ({a.dtype.enum_name} vs {b.dtype.enum_name})")
    if a.shape != b.shape:
        raise TensorError(f"{op}: shape mismatch")


# ---- literals (src/rew/ops/literal.nim:56-194) -------------------------------------

def constant(dtype: DType, shape: Sequence[int], data, device: Device | None = None) -> Tensor:
    if _jit.currentMode() == "trace":
        return _jit.traceConstant(dtype, shape, data)
    return fromHost(np.asarray(data), dtype=dtype, shape=shape, device=device)


def scalarF32(v: float, device: Device | None = None) -> Tensor:
    if _jit.currentMode() == "trace":
        return _jit.traceConstant(DType.FLOAT32, (), np.float32(v))
    return fromHost(np.array(v, dtype=np.float32), DType.FLOAT32, (), device)


def scalarI32(v: int, device: Device | None = None) -> Tensor:
    if _jit.currentMode() == "trace":
        return _jit.traceConstant(DType.INT32, (), np.int32(v))
    return fromHost(np.array(v, dtype=np.int32), DType.INT32, (), device)


def constantF32(shape: Sequence[int], data, device: Device | None = None) -> Tensor:
    a = np.asarray(data, dtype=np.float32)
    n = int(np.prod(shape)) if len(shape) else 1
    if a.size != n:
        raise TensorError(f"constantF32: data length {a.size} does not match shape product {n}")
    if _jit.currentMode() == "trace":
        return _jit.traceConstant(DType.FLOAT32, shape, a)
    return fromHost(a, DType.FLOAT32, shape, device)


def zeros(shape: Sequence[int], dtype: DType = DType.FLOAT32,
          device: Device | None = None) -> Tensor:
    """A zero scalar constant broadcast to `shape` (src/rew/ops/factory.nim:17-24)."""
    scalar = constant(dtype, [], np.zeros(1, np.float32), device)
    if len(shape) == 0:
        return scalar
    return broadcastTo(scalar, list(shape), [])


def zerosLike(t: Tensor, dtype: DType | None = None) -> Tensor:
    """src/rew/ops/factory.nim:26-28."""
    return zeros(t.shape, t.dtype if dtype is None else dtype, t.device)


# ---- elementwise (src/rew/ops/arith.nim, unary.nim) ---------------------------------

def _binary(name):
    def f(a: Tensor, b: Tensor) -> Tensor:
        _same(a, b, name)
        return _one(name, [a, b])
    f.__name__ = name
    return f


add = _binary("add")
sub = _binary("sub")
mul = _binary("mul")
divide = _binary("divide")
maximum = _binary("maximum")
minimum = _binary("minimum")
power = _binary("power")
remainder = _binary("remainder")
atan2 = _binary("atan2")
bitwiseAnd = _binary("bitwiseAnd")
bitwiseOr = _binary("bitwiseOr")
bitwiseXor = _binary("bitwiseXor")


def _unary(name):
    def f(a: Tensor) -> Tensor:
        return _one(name, [a])
    f.__name__ = name
    return f


neg = _unary("neg")
abs_ = _unary("abs")
exp = _unary("exp")
log = _unary("log")
sqrt = _unary("sqrt")
rsqrt = _unary("rsqrt")
tanh = _unary("tanh")
logistic = _unary("logistic")
sine = _unary("sine")
cosine = _unary("cosine")
floor = _unary("floor")
ceil = _unary("ceil")
sign = _unary("sign")
isFinite = _unary("isFinite")
cbrt = _unary("cbrt")
expm1 = _unary("expm1")
log1p = _unary("log1p")
tan = _unary("tan")
roundNearestAfz = _unary("roundNearestAfz")
roundNearestEven = _unary("roundNearestEven")
bitwiseNot = _unary("bitwiseNot")


def astype(a: Tensor, dtype: DType) -> Tensor:
    return _one("astype", [a], [("dtype", DType(dtype).rew_name)])


def clamp(lo: Tensor, x: Tensor, hi: Tensor) -> Tensor:
    return _one("clamp", [lo, x, hi])


# ---- shape ops (src/rew/ops/shape.nim, concat.nim, linalg.nim) ----------------------

def reshape(a: Tensor, newShape: Sequence[int]) -> Tensor:
    for d in newShape:
        if d <= 0:
            raise TensorError(f"reshape: shape contains non-positive dim {d}")
    n = 1
    for d in newShape:
        n *= d
    if n != a.numElements:
        raise TensorError(
            f"reshape: element count mismatch — operand has {a.numElements} elements, "
            f"target shape has {n}")
    return _one("reshape", [a], [("shape", _nimseq(newShape))])


def transpose(a: Tensor, permutation: Sequence[int]) -> Tensor:
    if len(permutation) != len(a.shape):
        raise TensorError(
            f"transpose: permutation length {len(permutation)} does not match operand rank "
            f"{len(a.shape)}")
    if sorted(permutation) != list(range(len(a.shape))):
        raise TensorError("transpose: invalid permutation")
    return _one("transpose", [a], [("permutation", _nimseq(permutation))])


def broadcastTo(t: Tensor, outputShape: Sequence[int],
                broadcastDimensions: Sequence[int]) -> Tensor:
    if len(broadcastDimensions) != len(t.shape):
        raise TensorError("broadcastTo: broadcastDimensions length must match operand rank")
    for i, od in enumerate(broadcastDimensions):
        if t.shape[i] != 1 and t.shape[i] != outputShape[od]:
            raise TensorError("broadcastTo: operand dim is not 1 and does not match")
    return _one("broadcastTo", [t], [("output_shape", _join(outputShape)),
                                     ("broadcast_dimensions", _join(broadcastDimensions))])


def slice_(t: Tensor, startIndices: Sequence[int], limitIndices: Sequence[int],
           strides: Sequence[int] = ()) -> Tensor:
    rank = len(t.shape)
    if len(startIndices) != rank or len(limitIndices) != rank:
        raise TensorError(f"slice: index arrays must match operand rank {rank}")
    st = list(strides) if len(strides) else [1] * rank
    for i in range(rank):
        if (startIndices[i] < 0 or limitIndices[i] > t.shape[i]
                or startIndices[i] >= limitIndices[i] or st[i] <= 0):
            raise TensorError(f"slice: invalid bounds at dim {i}")
    return _one("slice", [t], [("start_indices", _nimseq(startIndices)),
                               ("limit_indices", _nimseq(limitIndices)),
                               ("strides", _nimseq(st))])


def concat(tensors: Sequence[Tensor], dimension: int) -> Tensor:
    if not tensors:
        raise TensorError("concat: empty input list")
    return _one("concat", list(tensors), [("dimension", str(dimension))])


def iota(dtype: DType, shape: Sequence[int], dimension: int,
         device: Device | None = None) -> Tensor:
    if dtype == DType.BOOL:
        raise TensorError("iota: bool dtype is not supported")
    if dimension < 0 or dimension >= len(shape):
        raise TensorError(f"iota: dimension {dimension} out of range for rank {len(shape)}")
    d = device or defaultDevice()
    return _one("iota", [], [("dtype", DType(dtype).enum_name), ("shape", _nimseq(shape)),
                             ("dimension", str(dimension)), ("device", str(d))])


def unsqueeze(a: Tensor, dim: int) -> Tensor:
    s = list(a.shape)
    s.insert(dim, 1)
    return reshape(a, s)


def compare(lhs: Tensor, rhs: Tensor, direction: str) -> Tensor:
    if direction not in ("LT", "LE", "GT", "GE", "EQ", "NE"):
        raise TensorError(f"compare: invalid direction '{direction}'")
    return _one("compare", [lhs, rhs], [("comparison_direction", direction)])


def select(pred: Tensor, onTrue: Tensor, onFalse: Tensor) -> Tensor:
    if pred.dtype != DType.BOOL:
        raise TensorError(f"select: pred must be bool, got {pred.dtype.enum_name}")
    return _one("select", [pred, onTrue, onFalse])


# ---- reductions (src/rew/ops/reduce.nim:93-225) --------------------------------------

def _norm_dims(op: str, rank: int, dims: Sequence[int]) -> list[int]:
    out = []
    for d in dims:
        p = d + rank if d < 0 else d
        if p < 0 or p >= rank:
            raise TensorError(f"{op}: dim {d} out of range for rank {rank}")
        if p in out:
            raise TensorError(f"{op}: dim {d} repeated")
        out.append(p)
    return out


def _reduction(op: str, t: Tensor, dims: Sequence[int]) -> Tensor:
    rd = _norm_dims(op, len(t.shape), dims)
    if t.dtype != DType.FLOAT32:
        raise TensorError(f"{op}: v1 supports only float32 (got {t.dtype.enum_name})")
    return _one(op, [t], [("dims", _join(rd))])


def reduceSum(t: Tensor, dims: Sequence[int]) -> Tensor:
    return _reduction("reduceSum", t, dims)


def reduceMax(t: Tensor, dims: Sequence[int]) -> Tensor:
    return _reduction("reduceMax", t, dims)


def reduceMin(t: Tensor, dims: Sequence[int]) -> Tensor:
    return _reduction("reduceMin", t, dims)


def reduceProd(t: Tensor, dims: Sequence[int]) -> Tensor:
    return _reduction("reduceProd", t, dims)


def reduceMean(t: Tensor, dims: Sequence[int]) -> Tensor:
    # src/rew/ops/reduce.nim:132-150: reduceSum then divide by broadcast n.
    rd = _norm_dims("reduceMean", len(t.shape), dims)
    summed = reduceSum(t, rd)
    n = 1
    for d in rd:
        n *= t.shape[d]
    if n <= 0:
        raise TensorError(f"reduceMean: empty reduction (n = {n})")
    divisor = scalarF32(float(n), t.device)
    if len(summed.shape) == 0:
        return divide(summed, divisor)
    return divide(summed, broadcastTo(divisor, summed.shape, []))


def argmax(t: Tensor, dim: int) -> Tensor:
    """Index of the maximum along ``dim``; ties go to the smallest index.

    rew's composite (src/rew/ops/reduce.nim:202-225) raises at its int32
    ``reduceMin`` (fp32-only guard, reduce.nim:66-69); the backend runs the
    documented semantics as one native op instead, including the
    composite's NaN behaviour (a row containing NaN yields int32.high).
    """
    pos = dim + len(t.shape) if dim < 0 else dim
    if pos < 0 or pos >= len(t.shape):
        raise TensorError(f"argmax: dim {dim} out of range for rank {len(t.shape)}")
    if _jit.currentMode() == "trace":
        # rew's composite, which stops at the int32 reduceMin as rew's does
        m = reduceMax(t, [pos])
        mask = compare(t, broadcastTo(m, t.shape, [i for i in range(len(t.shape)) if i != pos]),
                       "EQ")
        ids = iota(DType.INT32, t.shape, pos, t.device)
        big = broadcastTo(scalarI32(2**31 - 1, t.device), t.shape, [])
        return reduceMin(select(mask, ids, big), [pos])
    return _one("argmax", [t], [("dimension", str(pos))])


def topK(operand: Tensor, k: int, dimension: int = -1, largest: bool = True):
    """(values, indices) of the k largest along the last dim, largest first,
    ties to the lower index (src/rew/ops/sort.nim:36-90 semantics; eager here,
    trace-only in the reference)."""
    if k <= 0:
        raise TensorError(f"topK: k must be positive, got {k}")
    rank = len(operand.shape)
    d = dimension + rank if dimension < 0 else dimension
    if k > operand.shape[d]:
        raise TensorError(f"topK: k {k} > dim size {operand.shape[d]}")
    if _jit.currentMode() == "trace":
        return _jit.traceTopK(operand, k, d, largest)
    outs = dispatchEager("topK", [operand], [("k", str(k)), ("dimension", str(d)),
                                             ("largest", "true" if largest else "false")])
    return outs[0], outs[1]


def sort(operand: Tensor, dimension: int = -1, isStable: bool = False,
         comparator: str = "LT", *others: Tensor):
    """Sorts along ``dimension`` (src/rew/ops/sort.nim:13-33).  rew takes the
    comparator as a builder callback; here it is the one compare direction
    such a callback emits on the operand pair ("LT"/"LE" ascending, "GT"/"GE"
    descending).  ``others`` are permuted along with ``operand`` (the
    multi-operand form of stablehlo.sort).  Trace-only in the reference; the
    backend also runs it eagerly (stable, NaN last)."""
    if comparator not in ("LT", "LE", "GT", "GE"):
        raise TensorError(f"sort: comparator must be LT, LE, GT or GE, got '{comparator}'")
    rank = len(operand.shape)
    d = dimension + rank if dimension < 0 else dimension
    if d < 0 or d >= rank:
        raise TensorError(f"sort: dimension {dimension} out of range for rank {rank}")
    ins = [operand, *others]
    if _jit.currentMode() == "trace":
        res = _jit.traceSort(ins, d, isStable, comparator)
    else:
        res = dispatchEager("sort", ins, [("dimension", str(d)),
                                          ("comparison_direction", comparator),
                                          ("is_stable", "true" if isStable else "false")])
    return res[0] if not others else res


@dataclass
class GatherDimensionNumbers:
    """src/rew/stablehlo/ops.nim:60-68."""
    offsetDims: Sequence[int]
    collapsedSliceDims: Sequence[int]
    startIndexMap: Sequence[int]
    indexVectorDim: int
    operandBatchingDims: Sequence[int] = ()
    startIndicesBatchingDims: Sequence[int] = ()


@dataclass
class ScatterDimensionNumbers:
    """src/rew/stablehlo/ops.nim:70-77."""
    updateWindowDims: Sequence[int]
    insertedWindowDims: Sequence[int]
    scatterDimsToOperandDims: Sequence[int]
    indexVectorDim: int
    inputBatchingDims: Sequence[int] = ()
    scatterIndicesBatchingDims: Sequence[int] = ()


def gather(operand: Tensor, startIndices: Tensor, dims: GatherDimensionNumbers,
           sliceSizes: Sequence[int], resultShape: Sequence[int],
           indicesAreSorted: bool = False) -> Tensor:
    """stablehlo.gather (src/rew/ops/gather.nim:10-28).  Trace-only in the
    reference; the backend also runs it eagerly (start indices clamped)."""
    if _jit.currentMode() == "trace":
        return _jit.traceGather(operand, startIndices, dims, sliceSizes, resultShape,
                                indicesAreSorted)
    out = _one("gather", [operand, startIndices], [
        ("offset_dims", _join(dims.offsetDims)),
        ("collapsed_slice_dims", _join(dims.collapsedSliceDims)),
        ("operand_batching_dims", _join(dims.operandBatchingDims)),
        ("start_indices_batching_dims", _join(dims.startIndicesBatchingDims)),
        ("start_index_map", _join(dims.startIndexMap)),
        ("index_vector_dim", str(dims.indexVectorDim)),
        ("slice_sizes", _join(sliceSizes))])
    if list(out.shape) != list(resultShape):
        raise TensorError(f"gather: resultShape {list(resultShape)} does not match the "
                          f"dimension numbers ({list(out.shape)})")
    return out


_UPDATES = ("replace", "add", "maximum", "minimum", "multiply")


def scatter(inputs: Sequence[Tensor], scatterIndices: Tensor, updates: Sequence[Tensor],
            dims: ScatterDimensionNumbers, updateComputation: str = "add",
            indicesAreSorted: bool = False, uniqueIndices: bool = False) -> list:
    """stablehlo.scatter (src/rew/ops/scatter.nim:10-39).  rew takes the update
    computation as a builder callback; here it names the one op such a
    callback emits on (current, update): "add", "maximum", "minimum",
    "multiply", or "replace" (the callback returns the update).  Updates of
    one element in several places combine in an unspecified order (atomics).
    Trace-only in the reference; the backend also runs one-input scatters
    eagerly."""
    if not inputs or len(inputs) != len(updates):
        raise TensorError("scatter: inputs and updates must have the same non-zero length")
    if updateComputation not in _UPDATES:
        raise TensorError(f"scatter: update computation must be one of {_UPDATES}")
    if _jit.currentMode() == "trace":
        return _jit.traceScatter(list(inputs), scatterIndices, list(updates), dims,
                                 updateComputation, indicesAreSorted, uniqueIndices)
    if len(inputs) != 1:
        raise TensorError("scatter: the backend runs one-input scatters only")
    return [_one("scatter", [inputs[0], scatterIndices, updates[0]], [
        ("update_window_dims", _join(dims.updateWindowDims)),
        ("inserted_window_dims", _join(dims.insertedWindowDims)),
        ("input_batching_dims", _join(dims.inputBatchingDims)),
        ("scatter_indices_batching_dims", _join(dims.scatterIndicesBatchingDims)),
        ("scatter_dims_to_operand_dims", _join(dims.scatterDimsToOperandDims)),
        ("index_vector_dim", str(dims.indexVectorDim)),
        ("update_computation", updateComputation)])]


def indexSelect(operand: Tensor, index: Tensor, dim: int = 0, batchDims: int = 0) -> Tensor:
    """src/rew/ops/gather.nim:55-81: torch_index_select in trace mode; the
    backend also runs it eagerly (as torchIndexSelect)."""
    if dim < 0 or dim >= len(operand.shape):
        raise TensorError(f"indexSelect: dim {dim} out of range for operand rank "
                          f"{len(operand.shape)}")
    return torchIndexSelect(operand, index, dim, batchDims)


# ---- linear algebra (src/rew/ops/linalg.nim:204-256, 432-461) -------------------------

def dotGeneral(a: Tensor, b: Tensor, lhsBatching: Sequence[int], rhsBatching: Sequence[int],
               lhsContracting: Sequence[int], rhsContracting: Sequence[int]) -> Tensor:
    if a.dtype != b.dtype:
        raise TensorError(
            f"dotGeneral: dtype mismatch ({a.dtype.enum_name} vs {b.dtype.enum_name})")
    return _one("dotGeneral", [a, b], [("lhs_batching", _join(lhsBatching)),
                                       ("rhs_batching", _join(rhsBatching)),
                                       ("lhs_contracting", _join(lhsContracting)),
                                       ("rhs_contracting", _join(rhsContracting))])


def matmul(a: Tensor, b: Tensor) -> Tensor:
    if len(a.shape) != 2 or len(b.shape) != 2:
        raise TensorError(
            f"matmul: expected rank-2 operands, got shapes {list(a.shape)} and {list(b.shape)}")
    if a.shape[1] != b.shape[0]:
        raise TensorError(f"matmul: inner dim mismatch — {list(a.shape)} * {list(b.shape)}")
    return dotGeneral(a, b, [], [], [1], [0])


def dot(a: Tensor, b: Tensor) -> Tensor:
    return _one("dot", [a, b])


def torchIndexSelect(operand: Tensor, index: Tensor, dim: int, batchDims: int) -> Tensor:
    if index.dtype not in (DType.INT8, DType.INT16, DType.INT32, DType.INT64, DType.UINT8,
                           DType.UINT16, DType.UINT32, DType.UINT64):
        raise TensorError("torchIndexSelect: index must be an integer tensor")
    return _one("torchIndexSelect", [operand, index], [("dim", str(dim)),
                                                        ("batch_dims", str(batchDims))])


# ---- shape, dynamic and linear-algebra ops outside the configs -------------------------
# src/rew/ops/shape.nim:108-475, ops/distributed.nim:11-35, ops/linalg.nim:177-202

_INT_DTYPES = {DType.INT4, DType.INT8, DType.INT16, DType.INT32, DType.INT64, DType.UINT4,
               DType.UINT8, DType.UINT16, DType.UINT32, DType.UINT64}


def getDimensionSize(a: Tensor, dimension: int) -> Tensor:
    if dimension < 0 or dimension >= len(a.shape):
        raise TensorError(f"getDimensionSize: dimension {dimension} out of range for rank "
                          f"{len(a.shape)}")
    return _one("getDimensionSize", [a], [("dimension", str(dimension))])


def pad(a: Tensor, paddingValue: Tensor, edgePaddingLow: Sequence[int],
        edgePaddingHigh: Sequence[int], interiorPadding: Sequence[int]) -> Tensor:
    if paddingValue.dtype != a.dtype or len(paddingValue.shape) != 0:
        raise TensorError(f"pad: paddingValue must be scalar with dtype {a.dtype.rew_name}")
    rank = len(a.shape)
    if not (len(edgePaddingLow) == len(edgePaddingHigh) == len(interiorPadding) == rank):
        raise TensorError(f"pad: padding arrays must match operand rank {rank}")
    for i, d in enumerate(a.shape):
        if interiorPadding[i] < 0:
            raise TensorError(f"pad: interior padding at dim {i} must be non-negative")
        if d + edgePaddingLow[i] + edgePaddingHigh[i] + max(d - 1, 0) * interiorPadding[i] < 0:
            raise TensorError(f"pad: result dimension {i} is negative")
    return _one("pad", [a, paddingValue], [("edge_padding_low", _nimseq(edgePaddingLow)),
                                           ("edge_padding_high", _nimseq(edgePaddingHigh)),
                                           ("interior_padding", _nimseq(interiorPadding))])


def _start_indices(a: Tensor, startIndices: Sequence[Tensor], op: str):
    if len(startIndices) != len(a.shape):
        raise TensorError(f"{op}: start index count {len(startIndices)} must match operand "
                          f"rank {len(a.shape)}")
    for i, idx in enumerate(startIndices):
        if idx.device != a.device:
            raise TensorError(f"{op}: device mismatch")
        if idx.dtype not in _INT_DTYPES or len(idx.shape) != 0:
            raise TensorError(f"{op}: start index #{i} must be an integer scalar")


def dynamicSlice(a: Tensor, startIndices: Sequence[Tensor], sliceSizes: Sequence[int]) -> Tensor:
    _start_indices(a, startIndices, "dynamicSlice")
    if len(sliceSizes) != len(a.shape):
        raise TensorError(f"dynamicSlice: sliceSizes length {len(sliceSizes)} must match "
                          f"operand rank {len(a.shape)}")
    for i, s in enumerate(sliceSizes):
        if s < 0 or s > a.shape[i]:
            raise TensorError(f"dynamicSlice: slice size {s} out of range for dim {i}")
    return _one("dynamicSlice", [a, *startIndices], [("slice_sizes", _nimseq(sliceSizes))])


def dynamicUpdateSlice(a: Tensor, update: Tensor, startIndices: Sequence[Tensor]) -> Tensor:
    if update.dtype != a.dtype:
        raise TensorError("dynamicUpdateSlice: update dtype must match operand dtype")
    if len(update.shape) != len(a.shape):
        raise TensorError("dynamicUpdateSlice: update rank must match operand rank")
    for i, (u, d) in enumerate(zip(update.shape, a.shape)):
        if u > d:
            raise TensorError(f"dynamicUpdateSlice: update dim {i} exceeds operand dim")
    _start_indices(a, startIndices, "dynamicUpdateSlice")
    return _one("dynamicUpdateSlice", [a, update, *startIndices])


def replicaId(device: Device | None = None) -> Tensor:
    return _one("replicaId", [], [("device", str(device or defaultDevice()))])


def partitionId(device: Device | None = None) -> Tensor:
    return _one("partitionId", [], [("device", str(device or defaultDevice()))])


def setDimensionSize(a: Tensor, size: Tensor, dimension: int) -> Tensor:
    if dimension < 0 or dimension >= len(a.shape):
        raise TensorError(f"setDimensionSize: dimension {dimension} out of range for rank "
                          f"{len(a.shape)}")
    if size.dtype not in _INT_DTYPES or len(size.shape) != 0:
        raise TensorError("setDimensionSize: size must be an integer scalar")
    return _one("setDimensionSize", [a, size], [("dimension", str(dimension))])


def dynamicReshape(a: Tensor, outputShape: Tensor, resultShape: Sequence[int]) -> Tensor:
    if outputShape.dtype not in _INT_DTYPES or tuple(outputShape.shape) != (len(resultShape),):
        raise TensorError(f"dynamicReshape: outputShape must be an integer vector of length "
                          f"{len(resultShape)}")
    if any(d < 0 for d in resultShape):
        raise TensorError("dynamicReshape: result shape contains negative dim")
    if int(np.prod(resultShape, dtype=np.int64)) != int(np.prod(a.shape, dtype=np.int64)):
        raise TensorError("dynamicReshape: result element count does not match operand")
    return _one("dynamicReshape", [a, outputShape], [("result_shape", _nimseq(resultShape))])


def dynamicIota(dtype: DType, outputShape: Tensor, resultShape: Sequence[int],
                dimension: int) -> Tensor:
    if dtype == DType.BOOL:
        raise TensorError("dynamicIota: bool dtype is not supported")
    if outputShape.dtype not in _INT_DTYPES or tuple(outputShape.shape) != (len(resultShape),):
        raise TensorError(f"dynamicIota: outputShape must be an integer vector of length "
                          f"{len(resultShape)}")
    if dimension < 0 or dimension >= len(resultShape):
        raise TensorError(f"dynamicIota: dimension {dimension} out of range for rank "
                          f"{len(resultShape)}")
    return _one("dynamicIota", [outputShape], [("dtype", DType(dtype).enum_name),
                                                ("result_shape", _nimseq(resultShape)),
                                                ("dimension", str(dimension))])


def cholesky(a: Tensor, lower: bool = True) -> Tensor:
    if a.dtype not in (DType.FLOAT16, DType.BFLOAT16, DType.FLOAT32, DType.FLOAT64):
        raise TensorError(f"cholesky: operand must be floating point, got {a.dtype.rew_name}")
    if len(a.shape) < 2:
        raise TensorError(f"cholesky: operand rank must be at least 2, got {len(a.shape)}")
    if a.shape[-1] != a.shape[-2]:
        raise TensorError(f"cholesky: innermost matrix dimensions must be square, got "
                          f"{list(a.shape)}")
    return _one("cholesky", [a], [("lower", "true" if lower else "false")])


# ---- batch norm (src/rew/ops/normalization.nim:40-205) ----------------------------------

def _bn_feature_index(operand: Tensor, featureIndex: int, op: str) -> list:
    if operand.dtype not in (DType.FLOAT16, DType.BFLOAT16, DType.FLOAT32, DType.FLOAT64):
        raise TensorError(f"{op}: operand must be floating point, got {operand.dtype.rew_name}")
    if featureIndex < 0 or featureIndex >= len(operand.shape):
        raise TensorError(f"{op}: featureIndex {featureIndex} out of range for rank "
                          f"{len(operand.shape)}")
    return [operand.shape[featureIndex]]


def _bn_feature(operand: Tensor, t: Tensor, name: str, fshape, op: str):
    if t.device != operand.device:
        raise TensorError(f"{op}: device mismatch")
    if t.dtype != operand.dtype:
        raise TensorError(f"{op}: {name} dtype {t.dtype.rew_name} differs from operand dtype "
                          f"{operand.dtype.rew_name}")
    if list(t.shape) != list(fshape):
        raise TensorError(f"{op}: {name} shape {list(t.shape)} must be {list(fshape)}")


def _bn_attrs(epsilon: float, featureIndex: int):
    return [("epsilon", repr(float(np.float32(epsilon)))), ("feature_index", str(featureIndex))]


def batchNormInference(operand: Tensor, scale: Tensor, offset: Tensor, mean: Tensor,
                       variance: Tensor, epsilon: float, featureIndex: int) -> Tensor:
    fs = _bn_feature_index(operand, featureIndex, "batchNormInference")
    for t, nm in ((scale, "scale"), (offset, "offset"), (mean, "mean"), (variance, "variance")):
        _bn_feature(operand, t, nm, fs, "batchNormInference")
    return _one("batchNormInference", [operand, scale, offset, mean, variance],
                _bn_attrs(epsilon, featureIndex))


def batchNormTraining(operand: Tensor, scale: Tensor, offset: Tensor, epsilon: float,
                      featureIndex: int):
    """(output, batchMean, batchVar)."""
    fs = _bn_feature_index(operand, featureIndex, "batchNormTraining")
    for t, nm in ((scale, "scale"), (offset, "offset")):
        _bn_feature(operand, t, nm, fs, "batchNormTraining")
    outs = dispatchEager("batchNormTraining", [operand, scale, offset],
                         _bn_attrs(epsilon, featureIndex))
    assert len(outs) == 3, "batchNormTraining: eager backend returned wrong arity"
    return tuple(outs)


def batchNormGrad(operand: Tensor, scale: Tensor, mean: Tensor, variance: Tensor,
                  gradOutput: Tensor, epsilon: float, featureIndex: int):
    """(gradOperand, gradScale, gradOffset)."""
    fs = _bn_feature_index(operand, featureIndex, "batchNormGrad")
    if gradOutput.dtype != operand.dtype or list(gradOutput.shape) != list(operand.shape):
        raise TensorError("batchNormGrad: gradOutput type must match operand type")
    for t, nm in ((scale, "scale"), (mean, "mean"), (variance, "variance")):
        _bn_feature(operand, t, nm, fs, "batchNormGrad")
    outs = dispatchEager("batchNormGrad", [operand, scale, mean, variance, gradOutput],
                         _bn_attrs(epsilon, featureIndex))
    assert len(outs) == 3, "batchNormGrad: eager backend returned wrong arity"
    return tuple(outs)


# ---- einsum and the shape-operand ops (src/rew/ops/linalg.nim, shape.nim) -----------

def _join_ints(xs: Sequence[int]) -> str:
    """joinInts (src/rew/ops/linalg.nim:21-29): "[a,b,c]"."""
    return "[" + ",".join(str(int(x)) for x in xs) + "]"


def einsum(a: Tensor, b: Tensor, config: str, outputShape: Sequence[int]) -> Tensor:
    """src/rew/ops/linalg.nim:378-403 (TensorFlow einsum grammar, explicit result shape)."""
    if a.device != b.device:
        raise TensorError("einsum: device mismatch")
    if a.dtype != b.dtype:
        raise TensorError(f"einsum: dtype mismatch ({a.dtype.rew_name} vs {b.dtype.rew_name})")
    if not config:
        raise TensorError("einsum: config must not be empty")
    return _one("einsum", [a, b], [("einsum_config", config),
                                   ("output_shape", _join_ints(outputShape))])


def unaryEinsum(a: Tensor, config: str, outputShape: Sequence[int]) -> Tensor:
    """src/rew/ops/linalg.nim:405-430."""
    if not config:
        raise TensorError("unaryEinsum: config must not be empty")
    return _one("unaryEinsum", [a], [("einsum_config", config),
                                     ("output_shape", _join_ints(outputShape))])


def dynamicBroadcastInDim(t: Tensor, outputDimensions: Tensor, resultShape: Sequence[int],
                          broadcastDimensions: Sequence[int],
                          knownExpandingDimensions: Sequence[int] = (),
                          knownNonexpandingDimensions: Sequence[int] = ()) -> Tensor:
    """src/rew/ops/linalg.nim:288-326."""
    if outputDimensions.dtype not in _INT_DTYPES or \
            tuple(outputDimensions.shape) != (len(resultShape),):
        raise TensorError("dynamicBroadcastInDim: outputDimensions must be an integer vector "
                          f"of length {len(resultShape)}")
    return _one("dynamicBroadcastInDim", [t, outputDimensions],
                [("result_shape", _join_ints(resultShape)),
                 ("broadcast_dimensions", _join_ints(broadcastDimensions)),
                 ("known_expanding_dimensions", _join_ints(knownExpandingDimensions)),
                 ("known_nonexpanding_dimensions", _join_ints(knownNonexpandingDimensions))])


def dynamicPad(a: Tensor, paddingValue: Tensor, edgePaddingLow: Tensor,
               edgePaddingHigh: Tensor, interiorPadding: Tensor,
               resultShape: Sequence[int]) -> Tensor:
    """src/rew/ops/shape.nim:395-441."""
    if paddingValue.dtype != a.dtype or len(paddingValue.shape) != 0:
        raise TensorError(f"dynamicPad: paddingValue must be scalar with dtype {a.dtype.rew_name}")
    for name, t in (("edgePaddingLow", edgePaddingLow), ("edgePaddingHigh", edgePaddingHigh),
                    ("interiorPadding", interiorPadding)):
        if t.dtype not in _INT_DTYPES or tuple(t.shape) != (len(a.shape),):
            raise TensorError(f"dynamicPad: {name} must be an integer vector of length "
                              f"{len(a.shape)}")
    return _one("dynamicPad", [a, paddingValue, edgePaddingLow, edgePaddingHigh, interiorPadding],
                [("result_shape", _nimseq(resultShape))])


def realDynamicSlice(a: Tensor, startIndices: Tensor, limitIndices: Tensor, strides: Tensor,
                     resultShape: Sequence[int]) -> Tensor:
    """src/rew/ops/shape.nim:477-517."""
    for name, t in (("startIndices", startIndices), ("limitIndices", limitIndices),
                    ("strides", strides)):
        if t.dtype not in _INT_DTYPES or tuple(t.shape) != (len(a.shape),):
            raise TensorError(f"realDynamicSlice: {name} must be an integer vector of length "
                              f"{len(a.shape)}")
    return _one("realDynamicSlice", [a, startIndices, limitIndices, strides],
                [("result_shape", _nimseq(resultShape))])


def triangularSolve(a: Tensor, b: Tensor, leftSide: bool = True, lower: bool = True,
                    unitDiagonal: bool = False, transposeA: str = "NO_TRANSPOSE") -> Tensor:
    """src/rew/ops/linalg.nim:350-376 (transposeA: NO_TRANSPOSE, TRANSPOSE or ADJOINT)."""
    if a.device != b.device:
        raise TensorError("triangularSolve: device mismatch")
    return _one("triangularSolve", [a, b],
                [("left_side", "true" if leftSide else "false"),
                 ("lower", "true" if lower else "false"),
                 ("unit_diagonal", "true" if unitDiagonal else "false"),
                 ("transpose_a", transposeA)])


# ---- complex parts and the Fourier transform ----------------------------------------

def complex(real: Tensor, imag: Tensor) -> Tensor:  # noqa: A001 (rew's name)
    """src/rew/ops/arith.nim:86-106: float32 / float64 parts -> complex64 / complex128."""
    if real.dtype not in (DType.FLOAT32, DType.FLOAT64):
        raise TensorError(f"complex: operands must be float32 or float64, got {real.dtype.rew_name}")
    return _one("complex", [real, imag])


def real(a: Tensor) -> Tensor:
    """src/rew/ops/unary.nim:184-202."""
    return _one("real", [a])


def imag(a: Tensor) -> Tensor:
    """src/rew/ops/unary.nim:204-224."""
    return _one("imag", [a])


def fft(a: Tensor, fftType: str, fftLength: Sequence[int]) -> Tensor:
    """src/rew/ops/linalg.nim:328-348 (fftType FFT, IFFT, RFFT or IRFFT)."""
    return _one("fft", [a], [("fft_type", fftType), ("fft_length", _join_ints(fftLength))])
