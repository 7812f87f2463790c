"""CPU checks of the control combinators' trace (rew_amd.control, mirroring
src/rew/transform/control.nim): the region structure and text forms rew's
emitter prints (tests/tcond.nim, tests/twhile.nim) and the misuse errors.
Nothing here touches a device."""
import pytest

from rew_amd import control as K
from rew_amd import jit as J
from rew_amd import ops as O
from rew_amd.eager import DType, Tensor, mi355x

D = mi355x(0)


def ph(dt, shape):
    return Tensor._make(None, DType(dt), tuple(shape), D)


def traced(fn, args):
    with J.withTrace("main", D) as ctx:
        ins = J.traceInputs(ctx, [a.dtype for a in args], [a.shape for a in args])
        J.traceReturn(ctx, fn(ins))
    return ctx.text()


def test_cond_lowers_to_stablehlo_if():
    # tcond.nim:9-22
    def f(a):
        p = O.compare(a[0], a[1], "GT")
        return [K.cond(p, lambda: O.add(a[0], a[0]), lambda: O.mul(a[0], a[0]))]
    text = traced(f, [ph(DType.FLOAT32, []), ph(DType.FLOAT32, [])])
    assert '"stablehlo.if"(%v3) ({' in text
    assert "stablehlo.return %v4 : tensor<f32>" in text
    assert "stablehlo.return %v5 : tensor<f32>" in text
    assert "}) : (tensor<i1>) -> (tensor<f32>)" in text
    # the branch ops sit inside the regions
    assert text.index('"stablehlo.if"') < text.index("stablehlo.add") < text.index("}, {")


def test_while_loop_lowers_to_stablehlo_while():
    # twhile.nim:28-47
    def f(a):
        zero, limit = O.scalarI32(0), O.scalarI32(3)
        outs = K.whileLoop([zero, a[0]], lambda c: O.compare(c[0], limit, "LT"),
                           lambda c: [O.add(c[0], O.scalarI32(1)), O.add(c[1], a[0])])
        assert len(outs) == 2 and outs[0].dtype == DType.INT32 and outs[1].shape == (2,)
        return outs
    text = traced(f, [ph(DType.FLOAT32, [2])])
    assert '"stablehlo.while"(%v2, %v1) ({' in text
    assert "^cond(%v4: tensor<i32>, %v5: tensor<2xf32>):" in text
    assert "^body(%v7: tensor<i32>, %v8: tensor<2xf32>):" in text
    assert "stablehlo.compare" in text
    assert ":2 = \"stablehlo.while\"" in text
    assert "}) : (tensor<i32>, tensor<2xf32>) -> (tensor<i32>, tensor<2xf32>)" in text


def test_fori_threads_carry():
    # twhile.nim:49-64
    def f(a):
        def body(i, carry):
            assert i.dtype == DType.INT32 and i.shape == ()
            return [O.add(carry[0], a[0])]
        outs = K.fori(0, 4, [a[0]], body)
        assert len(outs) == 1 and outs[0].shape == (3,)
        return outs
    assert '"stablehlo.while"' in traced(f, [ph(DType.FLOAT32, [3])])


def test_case_generic_form():
    def f(a):
        i = O.scalarI32(1)
        return K.caseOp(i, [lambda: [a[0]], lambda: [O.neg(a[0])]])
    text = traced(f, [ph(DType.FLOAT32, [4])])
    assert '= "stablehlo.case"(%v2) ({' in text
    assert text.count("^bb0:") == 2
    assert "}) : (tensor<i32>) -> tensor<4xf32>" in text


def test_misuse_raises():
    # twhile.nim:66-76, tcond.nim (mode, predicate and branch checks)
    with pytest.raises(K.CondError):
        K.cond(ph(DType.BOOL, []), lambda: None, lambda: None)  # eager mode

    def bad_body(a):
        return K.whileLoop([a[0]], lambda c: O.compare(c[0], c[0], "LT"),
                           lambda c: [O.add(c[0], c[0]), c[0]])
    with pytest.raises(K.CondError):
        traced(bad_body, [ph(DType.FLOAT32, [2])])

    def bad_pred(a):
        return [K.cond(a[0], lambda: a[0], lambda: a[0])]
    with pytest.raises(K.CondError):
        traced(bad_pred, [ph(DType.FLOAT32, [])])

    def mismatch(a):
        return [K.cond(O.compare(a[0], a[0], "EQ"), lambda: a[0],
                       lambda: O.astype(a[0], DType.INT32))]
    with pytest.raises(K.CondError):
        traced(mismatch, [ph(DType.FLOAT32, [])])

    def bad_index(a):
        return K.caseOp(O.scalarF32(0.0), [lambda: [a[0]]])
    with pytest.raises(K.CondError):
        traced(bad_index, [ph(DType.FLOAT32, [])])
