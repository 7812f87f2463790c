"""In-graph control flow: cond, condN, whileLoop, fori, caseOp.

Mirrors src/rew/transform/control.nim: valid in trace mode only (inside
`jit` / `lazy`), each combinator traces its branch or loop functions once
into the regions of a `stablehlo.if`, `stablehlo.while` or `stablehlo.case`
op, printed as rew's emitter prints them (src/rew/stablehlo/text.nim:
emitIf 984-1020, emitWhile 1074-1130, the generic quoted form with
emitRegionList 1805-1868 for case, and emitStablehloReturn 267-282 for the
region terminators).  The mi355x library runs those regions on the host
side of the call, reading each predicate back from the device
(rew_mi355x_execute_jit).
"""
from __future__ import annotations

from typing import Callable, Sequence

from . import jit as _jit
from . import ops as _ops
from .eager import DType, Tensor


class CondError(RuntimeError):
    """Misuse of a control combinator (control.nim:44-46): wrong dtype /
    shape, mode, or mismatched branch outputs."""


def _require_trace_mode(op: str) -> _jit.TraceContext:
    ctx = _jit.currentTrace()
    if ctx is None:
        raise CondError(f"{op}: only valid in trace mode (open a `withTrace`/`jit` block)")
    return ctx


def _require_trace(ctx, t: Tensor, op: str) -> None:
    if not isinstance(t, _jit.TraceTensor) or t.trace is not ctx:
        raise CondError(f"{op}: expected a trace tensor, got an eager tensor")


def _ty(t: Tensor) -> str:
    return _jit._ty(t.dtype, t.shape)


def _ret(values: Sequence[Tensor]) -> str:
    """stablehlo.return %a, %b : T, T (text.nim:267-282)."""
    return ("stablehlo.return " + ", ".join(f"%v{v.traceId}" for v in values) + " : "
            + ", ".join(_ty(v) for v in values))


def _region(ctx, fn: Callable, *args):
    """Runs fn(*args) with the trace's op lines collected apart; returns
    (lines, fn's result)."""
    saved = ctx.lines
    ctx.lines = []
    try:
        out = fn(*args)
        lines = ctx.lines
    finally:
        ctx.lines = saved
    return lines, out


def _indent(lines: Sequence[str], by: str) -> list[str]:
    return [by + ln for ln in lines]


def _results_ref(res: Sequence[Tensor]) -> str:
    """`%vN` or `%vN:K` for an op whose results take the ids N .. N + K - 1
    (text.nim:995-1001)."""
    head = f"%v{res[0].traceId}"
    return head if len(res) == 1 else f"{head}:{len(res)}"


def _check_outs(op: str, branch: str, outs, ctx, expected=None):
    if not isinstance(outs, (list, tuple)):
        raise CondError(f"{op}: {branch} must return a sequence of tensors")
    if len(outs) == 0:
        raise CondError(f"{op}: {branch} returned no values")
    for i, t in enumerate(outs):
        if not isinstance(t, _jit.TraceTensor) or t.trace is not ctx:
            raise CondError(f"{op}: {branch} result #{i} is not a trace tensor")
    if expected is not None:
        if len(outs) != len(expected):
            raise CondError(f"{op}: {branch} returned {len(outs)} value(s), "
                            f"expected {len(expected)}")
        for i, (t, e) in enumerate(zip(outs, expected)):
            if t.dtype != e.dtype or tuple(t.shape) != tuple(e.shape):
                raise CondError(f"{op}: {branch} result #{i} type mismatch — expected "
                                f"{e.dtype.enum_name}{list(e.shape)}, got "
                                f"{t.dtype.enum_name}{list(t.shape)}")


def condN(pred: Tensor, thenFn: Callable[[], Sequence[Tensor]],
          elseFn: Callable[[], Sequence[Tensor]]) -> list:
    """Multi-output if / else (control.nim:48-101; builder ifOp,
    src/rew/stablehlo/ops.nim:2060-2095)."""
    ctx = _require_trace_mode("cond")
    _require_trace(ctx, pred, "cond")
    if pred.dtype != DType.BOOL or len(pred.shape) != 0:
        raise CondError(f"cond: predicate must be a 0-rank bool tensor, got dtype="
                        f"{pred.dtype.enum_name} shape={list(pred.shape)}")
    then_lines, then_outs = _region(ctx, thenFn)
    _check_outs("cond", "then-branch", then_outs, ctx)
    else_lines, else_outs = _region(ctx, elseFn)
    _check_outs("cond", "else-branch", else_outs, ctx, then_outs)
    res = [ctx.value(t.dtype, t.shape) for t in then_outs]
    ctx.lines += ([f"    {_results_ref(res)} = \"stablehlo.if\"(%v{pred.traceId}) ({{"]
                  + _indent(then_lines, "  ") + ["      " + _ret(then_outs), "    }, {"]
                  + _indent(else_lines, "  ") + ["      " + _ret(else_outs)]
                  + ["    }) : (tensor<i1>) -> (" + ", ".join(_ty(t) for t in res) + ")"])
    return res


def cond(pred: Tensor, thenFn: Callable[[], Tensor], elseFn: Callable[[], Tensor]) -> Tensor:
    """Single-output if / else (control.nim:103-111)."""
    return condN(pred, lambda: [thenFn()], lambda: [elseFn()])[0]


def whileLoop(init: Sequence[Tensor], condFn: Callable[[Sequence[Tensor]], Tensor],
              bodyFn: Callable[[Sequence[Tensor]], Sequence[Tensor]]) -> list:
    """stablehlo.while over the carry `init` (control.nim:115-190; builder
    whileOp, src/rew/stablehlo/ops.nim:2150-2200)."""
    ctx = _require_trace_mode("whileLoop")
    if len(init) == 0:
        raise CondError("whileLoop: must carry at least one value")
    for t in init:
        _require_trace(ctx, t, "whileLoop")
    cargs = [ctx.value(t.dtype, t.shape) for t in init]
    cond_lines, pred = _region(ctx, condFn, cargs)
    if (not isinstance(pred, _jit.TraceTensor) or pred.dtype != DType.BOOL
            or len(pred.shape) != 0):
        raise CondError("whileLoop: condFn must return a 0-rank bool trace tensor")
    bargs = [ctx.value(t.dtype, t.shape) for t in init]
    body_lines, nxt = _region(ctx, bodyFn, bargs)
    _check_outs("whileLoop", "body", nxt, ctx, init)
    res = [ctx.value(t.dtype, t.shape) for t in init]
    types = ", ".join(_ty(t) for t in init)
    ctx.lines += ([f"    {_results_ref(res)} = \"stablehlo.while\"("
                   + ", ".join(f"%v{t.traceId}" for t in init) + ") ({",
                   "      ^cond(" + ", ".join(f"%v{a.traceId}: {_ty(a)}" for a in cargs) + "):"]
                  + _indent(cond_lines, "    ") + ["        " + _ret([pred]), "    }, {",
                   "      ^body(" + ", ".join(f"%v{a.traceId}: {_ty(a)}" for a in bargs) + "):"]
                  + _indent(body_lines, "    ") + ["        " + _ret(nxt)]
                  + [f"    }}) : ({types}) -> ({types})"])
    return res


def fori(low: int, high: int, init: Sequence[Tensor],
         body: Callable[[Tensor, Sequence[Tensor]], Sequence[Tensor]]) -> list:
    """Integer-counter loop over [low, high) (control.nim:194-227): an int32
    counter carried first, compared LT with `high`."""
    _require_trace_mode("fori")
    counter0 = _ops.scalarI32(low)
    upper = _ops.scalarI32(high)
    one = _ops.scalarI32(1)

    def body_fn(carry):
        i = carry[0]
        user = list(carry[1:])
        nxt = body(i, user)
        if len(nxt) != len(user):
            raise CondError(f"fori: body returned {len(nxt)} value(s), expected {len(user)}")
        return [_ops.add(i, one)] + list(nxt)

    outs = whileLoop([counter0] + list(init), lambda c: _ops.compare(c[0], upper, "LT"),
                     body_fn)
    return outs[1:]


def caseOp(index: Tensor, branches: Sequence[Callable[[], Sequence[Tensor]]]) -> list:
    """stablehlo.case on a 0-rank int32 index (control.nim:229-283; builder
    caseOp, src/rew/stablehlo/ops.nim:1504-1529).  An index outside
    [0, len(branches)) runs the last branch."""
    ctx = _require_trace_mode("caseOp")
    _require_trace(ctx, index, "caseOp")
    if index.dtype != DType.INT32 or len(index.shape) != 0:
        raise CondError(f"caseOp: index must be a 0-rank int32 tensor, got "
                        f"{index.dtype.enum_name} shape {list(index.shape)}")
    if len(branches) == 0:
        raise CondError("caseOp: at least one branch is required")
    regions = []
    first = None
    for bi, br in enumerate(branches):
        lines, outs = _region(ctx, br)
        _check_outs("caseOp", f"branch #{bi}", outs, ctx, first)
        if first is None:
            first = list(outs)
        regions.append((lines, outs))
    res = [ctx.value(t.dtype, t.shape) for t in first]
    out_ty = (_ty(res[0]) if len(res) == 1
              else "(" + ", ".join(_ty(t) for t in res) + ")")
    text = [", ".join(f"%v{r.traceId}" for r in res)
            + f" = \"stablehlo.case\"(%v{index.traceId}) ("]
    for k, (lines, outs) in enumerate(regions):
        text[-1] += "{" if k == 0 else ", {"
        text += ["      ^bb0:"] + _indent(lines, "    ") + ["        " + _ret(outs), "    }"]
    text[-1] += f") : (tensor<i32>) -> {out_ty}"
    ctx.lines += ["    " + text[0]] + text[1:]
    return res


def scan(init: Sequence[Tensor], xs: Sequence[Tensor],
         body: Callable[[Sequence[Tensor], Sequence[Tensor]], tuple]) -> tuple:
    """Sequential scan over the leading axis of `xs` (control.nim:290-420):
    the body is traced once on slice 0 for its output types (those ops stay
    in the trace, unused), then a whileLoop carries (counter, carry...,
    ys accumulators...), slicing x[counter] with dynamicSlice and writing
    each y into its accumulator with dynamicUpdateSlice.  Returns
    (carry, ys).  As in rew, the update's start list has one entry per
    dimension of y (the counter, then zeros), which fits scalar ys."""
    _require_trace_mode("scan")
    if len(xs) == 0:
        raise CondError("scan: at least one xs tensor required")
    ctx = _jit.currentTrace()
    n = xs[0].shape[0]
    for x in xs:
        _require_trace(ctx, x, "scan")
        if x.shape[0] != n:
            raise CondError("scan: all xs must have the same leading dim size")
    for t in init:
        _require_trace(ctx, t, "scan")
    start_zeros = [_ops.scalarI32(0) for _ in xs[0].shape]
    sizes = [1] + list(xs[0].shape[1:])

    def squeeze0(t):
        return _ops.reshape(t, list(t.shape[1:]))
    x0 = [squeeze0(_ops.dynamicSlice(x, start_zeros, sizes)) for x in xs]
    dummy_carry, dummy_y = body(list(init), x0)
    if len(dummy_carry) != len(init):
        raise CondError(f"scan: body returned {len(dummy_carry)} carry value(s), "
                        f"expected {len(init)}")
    counter0, n_val, one = _ops.scalarI32(0), _ops.scalarI32(n), _ops.scalarI32(1)
    nc, ny = len(init), len(dummy_y)
    full = [counter0] + list(init)
    for t in dummy_y:
        shp = [n] + list(t.shape)
        if t.dtype == DType.FLOAT32:
            full.append(_ops.broadcastTo(_ops.scalarF32(0.0), shp, []))
        elif t.dtype == DType.INT32:
            full.append(_ops.broadcastTo(_ops.scalarI32(0), shp, []))
        else:
            full.append(_ops.astype(_ops.broadcastTo(_ops.scalarF32(0.0), shp, []), t.dtype))

    def body_fn(args):
        counter = args[0]
        carry = list(args[1:1 + nc])
        xsl = []
        for x in xs:
            starts = [counter] + [_ops.scalarI32(0) for _ in range(1, len(x.shape))]
            xsl.append(squeeze0(_ops.dynamicSlice(x, starts, sizes)))
        new_carry, ys_out = body(carry, xsl)
        if len(new_carry) != nc:
            raise CondError(f"scan: body returned {len(new_carry)} carry value(s), expected {nc}")
        if len(ys_out) != ny:
            raise CondError(f"scan: body returned {len(ys_out)} y value(s), expected {ny}")
        res = [_ops.add(counter, one)] + list(new_carry)
        for yi, y in enumerate(ys_out):
            starts = [counter] + [_ops.scalarI32(0) for _ in range(1, len(y.shape))]
            res.append(_ops.dynamicUpdateSlice(args[1 + nc + yi], _ops.unsqueeze(y, 0), starts))
        return res

    outs = whileLoop(full, lambda a: _ops.compare(a[0], n_val, "LT"), body_fn)
    return list(outs[1:1 + nc]), list(outs[1 + nc:])
