"""CPU checks of the trace/jit/lazy mirror: the StableHLO text it emits
against the exact strings and substrings of rew's emitter tests
(tests/tstablehlo_text.nim), and the JitFunction cache, signature and
validation behaviour of tests/tjit.nim.  Nothing here touches a device:
traced functions only build text."""
import os
import tempfile

import pytest

from rew_amd import jit as J
from rew_amd import nn
from rew_amd import ops as O
from rew_amd.eager import DType, Tensor, TensorError, TensorModeError, mi355x

D = mi355x(0)


def ph(dt, shape):
    """A placeholder argument: only dtype, shape and device matter to a trace."""
    return Tensor._make(None, DType(dt), tuple(shape), D)


def traced(fn, args, module="trace_module", func="main"):
    with J.withTrace(func, D) as ctx:
        ctx.moduleName = module
        ins = J.traceInputs(ctx, [a.dtype for a in args], [a.shape for a in args])
        J.traceReturn(ctx, fn(ins))
    return ctx.text()


# ---- tests/tstablehlo_text.nim -------------------------------------------------------

def test_emit_minimal_passthrough():
    # tstablehlo_text.nim:15-30
    assert traced(lambda a: [a[0]], [ph(DType.FLOAT32, [])], module="m") == (
        "module @m {\n"
        "  func.func @main(%v1: tensor<f32>) -> tensor<f32> {\n"
        "    func.return %v1 : tensor<f32>\n"
        "  }\n"
        "}\n")


def test_emit_add_two_vectors():
    # tstablehlo_text.nim:32-49
    t = traced(lambda a: [O.add(a[0], a[1])], [ph(DType.FLOAT32, [3])] * 2, module="addmod")
    assert t == (
        "module @addmod {\n"
        "  func.func @main(%v1: tensor<3xf32>, %v2: tensor<3xf32>) -> tensor<3xf32> {\n"
        "    %v3 = stablehlo.add %v1, %v2 : tensor<3xf32>\n"
        "    func.return %v3 : tensor<3xf32>\n"
        "  }\n"
        "}\n")


def test_emit_constant_then_neg():
    # tstablehlo_text.nim:51-65 (a traced function always has an argument
    # here; the constant and the negate keep their forms and numbering)
    def f(a):
        return [O.neg(O.constant(DType.FLOAT32, [], [1.0]))]
    t = traced(f, [ph(DType.FLOAT32, [])])
    assert 'stablehlo.constant dense<"0x0000803F"> : tensor<f32>' in t
    assert "stablehlo.negate %v2 : tensor<f32>" in t
    assert "func.return %v3 : tensor<f32>" in t


def test_emit_mul_then_sub_higher_rank():
    # tstablehlo_text.nim:67-80
    t = traced(lambda a: [O.sub(O.mul(a[0], a[1]), a[2])], [ph(DType.INT32, [2, 3])] * 3)
    assert "tensor<2x3xi32>" in t
    assert "stablehlo.multiply %v1, %v2 : tensor<2x3xi32>" in t
    assert "stablehlo.subtract %v4, %v3 : tensor<2x3xi32>" in t


@pytest.mark.parametrize("dt,name", [
    (DType.BOOL, "i1"), (DType.INT8, "i8"), (DType.UINT8, "ui8"), (DType.INT16, "i16"),
    (DType.UINT16, "ui16"), (DType.FLOAT16, "f16"), (DType.BFLOAT16, "bf16"),
    (DType.INT32, "i32"), (DType.UINT32, "ui32"), (DType.FLOAT32, "f32"),
    (DType.INT64, "i64"), (DType.UINT64, "ui64"), (DType.FLOAT64, "f64"),
    (DType.COMPLEX64, "complex<f32>"), (DType.COMPLEX128, "complex<f64>")])
def test_emit_dtype_spellings(dt, name):
    # tstablehlo_text.nim:82-111
    assert J._ty(dt, []) == f"tensor<{name}>"


def test_reduce_form_and_numbering():
    # text.nim:284-334; reduce.nim:93-117: init constant, region arguments,
    # body, then the result
    t = traced(lambda a: [O.reduceSum(a[0], [1])], [ph(DType.FLOAT32, [4, 3])])
    assert t.splitlines()[2:8] == [
        '    %v2 = stablehlo.constant dense<"0x00000000"> : tensor<f32>',
        "    %v6 = stablehlo.reduce(%v1 init: %v2) across dimensions = [1] : "
        "(tensor<4x3xf32>, tensor<f32>) -> tensor<4xf32>",
        "      reducer(%v3: tensor<f32>, %v4: tensor<f32>) {",
        "        %v5 = stablehlo.add %v3, %v4 : tensor<f32>",
        "        stablehlo.return %v5 : tensor<f32>",
        "      }"]


def test_topk_traces_as_sort_slice_iota_sort_slice():
    # sort.nim:53-85: values from sort(x) GE + slice, ids from sort(x, iota)
    t = traced(lambda a: list(O.topK(a[0], 2, 1, True)), [ph(DType.FLOAT32, [4, 8])])
    lines = [ln.strip() for ln in t.splitlines()]
    sorts = [ln for ln in lines if '"stablehlo.sort"' in ln]
    assert len(sorts) == 2
    assert sorts[0].startswith('%v5 = "stablehlo.sort"(%v1) ({')
    assert sorts[1].startswith('%v13, %v14 = "stablehlo.sort"(%v1, %v7) ({')
    assert "%v4 = stablehlo.compare GE, %v2, %v3 : (tensor<f32>, tensor<f32>) -> tensor<i1>" in lines
    assert ("}) {dimension = 1 : i64, is_stable = true} : (tensor<4x8xf32>, tensor<4x8xi32>) "
            "-> (tensor<4x8xf32>, tensor<4x8xi32>)") in lines
    assert "%v6 = stablehlo.slice %v5 [0:4, 0:2] : (tensor<4x8xf32>) -> tensor<4x2xf32>" in lines
    assert "%v7 = \"stablehlo.iota\"() {iota_dimension = 1 : i64} : () -> tensor<4x8xi32>" in lines
    assert "%v15 = stablehlo.slice %v14 [0:4, 0:2] : (tensor<4x8xi32>) -> tensor<4x2xi32>" in lines
    assert "func.return %v6, %v15 : tensor<4x2xf32>, tensor<4x2xi32>" in lines


def test_argmax_trace_stops_at_the_int32_reduce_min():
    # reduce.nim:202-225 with the fp32-only guard of reductionImpl (:66-69)
    with pytest.raises(TensorError, match="reduceMin: v1 supports only float32"):
        traced(lambda a: [O.argmax(a[0], 1)], [ph(DType.FLOAT32, [4, 3])])


def test_eager_tensor_in_trace_is_a_mode_error():
    # tensor.nim:102-110, 177-186: a closed-over eager tensor
    eager = ph(DType.FLOAT32, [3])
    with pytest.raises(TensorModeError, match="expected a trace tensor"):
        traced(lambda a: [O.add(a[0], eager)], [ph(DType.FLOAT32, [3])])


def test_slice_and_misc_forms():
    def f(a):
        return [O.slice_(a[0], [0, 1], [2, 3], [1, 2]), O.transpose(a[0], [1, 0]),
                O.broadcastTo(a[1], [4, 3], [1]), O.astype(a[0], DType.BFLOAT16),
                O.select(O.compare(a[0], a[0], "GT"), a[0], a[0]),
                O.concat([a[0], a[0]], 0), O.clamp(a[2], a[0], a[2]),
                O.torchIndexSelect(a[0], a[3], 0, 0), O.isFinite(a[0])]
    t = traced(f, [ph(DType.FLOAT32, [4, 3]), ph(DType.FLOAT32, [3]), ph(DType.FLOAT32, []),
                   ph(DType.INT32, [5])])
    for s in ["stablehlo.slice %v1 [0:2, 1:3:2] : (tensor<4x3xf32>) -> tensor<2x1xf32>",
              "stablehlo.transpose %v1, dims = [1, 0] : (tensor<4x3xf32>) -> tensor<3x4xf32>",
              "stablehlo.broadcast_in_dim %v2, dims = [1] : (tensor<3xf32>) -> tensor<4x3xf32>",
              '"stablehlo.convert"(%v1) : (tensor<4x3xf32>) -> tensor<4x3xbf16>',
              "stablehlo.compare GT, %v1, %v1 : (tensor<4x3xf32>, tensor<4x3xf32>) -> "
              "tensor<4x3xi1>",
              "stablehlo.select %v9, %v1, %v1 : tensor<4x3xi1>, tensor<4x3xf32>",
              "stablehlo.concatenate %v1, %v1, dim = 0 : (tensor<4x3xf32>, tensor<4x3xf32>) -> "
              "tensor<8x3xf32>",
              "stablehlo.clamp %v3, %v1, %v3 : (tensor<f32>, tensor<4x3xf32>, tensor<f32>) -> "
              "tensor<4x3xf32>",
              '"stablehlo.torch_index_select"(%v1, %v4) {dim = 0 : i64, batch_dims = 0 : i64} : '
              "(tensor<4x3xf32>, tensor<5xi32>) -> tensor<5x3xf32>",
              '"stablehlo.is_finite"(%v1) : (tensor<4x3xf32>) -> tensor<4x3xi1>']:
        assert s in t, s


# ---- tests/tjit.nim ------------------------------------------------------------------

def test_jit_lower_caches():
    j = J.jit(lambda a: [O.add(a[0], a[1])], "addPair")
    a, b = ph(DType.FLOAT32, [2, 3]), ph(DType.FLOAT32, [2, 3])
    assert j.cacheSize() == 0
    j.lower([a, b])
    assert j.cacheSize() == 1
    j.lower([a, b])
    assert j.cacheSize() == 1
    assert "stablehlo.add" in j.text([a, b])
    assert "func.func @addPair(" in j.text([a, b])


def test_lazy_lower_caches():
    def f(a):
        y = O.add(a[0], a[1])
        return [O.mul(y, y)]
    lz = J.lazy(f, "lazySquare")
    a, b = ph(DType.FLOAT32, [2, 3]), ph(DType.FLOAT32, [2, 3])
    assert lz.cacheSize() == 0
    t1 = lz.text([a, b])
    assert lz.cacheSize() == 1
    assert lz.text([a, b]) == t1
    assert "stablehlo.add" in t1 and "stablehlo.multiply" in t1


def test_jit_text_and_dump_helpers():
    j = J.jit(lambda a: [O.neg(a[0])], "dumpPair")
    x = ph(DType.FLOAT32, [2])
    assert "stablehlo.negate" in j.text([x])
    assert "@main" in j.executableText([x])
    with tempfile.TemporaryDirectory() as d:
        p = j.dumpHlo([x], os.path.join(d, "sub", "rew_jit_dump.mlir"))
        assert "stablehlo.negate" in open(p).read()


def test_jit_signature_specialisation_and_string():
    j = J.jit(lambda a: [O.mul(a[0], a[0])])
    small, big = ph(DType.FLOAT32, [2]), ph(DType.FLOAT32, [4])
    j.lower([small])
    j.lower([big])
    assert j.cacheSize() == 2
    j.lower([small])
    assert j.cacheSize() == 2
    s = J.signatureOf([ph(DType.FLOAT32, [2, 3]), ph(DType.FLOAT32, [3])])
    assert "float32:[2,3]" in s and "float32:[3]" in s
    assert "@mi355x:0" in s and "#replicated" in s


def test_jit_donate_validates_and_zero_inputs_rejected():
    with pytest.raises(J.JitError):
        J.jit(lambda a: [a[0]], donateArgs=[3]).lower([ph(DType.FLOAT32, [2])])
    with pytest.raises(J.JitError):
        J.jit(lambda a: []).lower([])


def test_jit_call_requires_eager_inputs():
    # tjit.nim:109-118: tracing succeeds and is cached, execution rejects
    # trace tensors
    j = J.jit(lambda a: [a[0]])
    with J.withTrace("outer", D) as ctx:
        (x,) = J.traceInputs(ctx, [DType.FLOAT32], [[2]])
    with pytest.raises(TensorModeError):
        j.call([x])
    assert j.cacheSize() == 1


def test_jit_clear_cache():
    j = J.jit(lambda a: [a[0]])
    j.lower([ph(DType.FLOAT32, [2])])
    assert j.cacheSize() == 1
    j.clearCache()
    assert j.cacheSize() == 0


def test_moe_traces_with_parameters_as_arguments():
    T, H, I, E_, S, k = 16, 32, 16, 4, 1, 2
    args = [ph(DType.BFLOAT16, [T, H]), ph(DType.FLOAT32, [H, E_]), ph(DType.FLOAT32, [E_])]
    for _ in range(S + E_):
        for fi, fo in [(H, I), (H, I), (I, H)]:
            args += [ph(DType.BFLOAT16, [fi, fo]), ph(DType.BFLOAT16, [fo])]
    t = J.jit(lambda a: [nn.moeFromParams(a[1:], S, E_, k).forward(a[0])], "moe").text(args)
    assert t.count('"stablehlo.sort"') == 2
    assert t.count("stablehlo.dot_general") == 1 + 3 * (S + E_)
    assert t.rstrip().endswith("}")


def test_emit_pad_and_dynamic_slices():
    """The generic forms of rew's emitter (src/rew/stablehlo/text.nim:589-690,
    arrays rendered by renderI64Array, text.nim:123-130)."""
    def fn(a):
        return [O.pad(a[0], a[1], [1, 0], [0, 2], [1, 0]),
                O.dynamicSlice(a[0], [a[2], a[2]], [1, 2]),
                O.dynamicUpdateSlice(a[0], a[3], [a[2], a[2]])]
    text = traced(fn, [ph(DType.FLOAT32, [2, 3]), ph(DType.FLOAT32, []),
                       ph(DType.INT32, []), ph(DType.FLOAT32, [1, 1])])
    assert ('"stablehlo.pad"(%v1, %v2) {edge_padding_low = array<i64: 1, 0>, '
            'edge_padding_high = array<i64: 0, 2>, interior_padding = array<i64: 1, 0>} : '
            '(tensor<2x3xf32>, tensor<f32>) -> tensor<4x5xf32>') in text
    assert ('"stablehlo.dynamic_slice"(%v1, %v3, %v3) {slice_sizes = array<i64: 1, 2>} : '
            '(tensor<2x3xf32>, tensor<i32>, tensor<i32>) -> tensor<1x2xf32>') in text
    assert ('"stablehlo.dynamic_update_slice"(%v1, %v4, %v3, %v3) : (tensor<2x3xf32>, '
            'tensor<1x1xf32>, tensor<i32>, tensor<i32>) -> tensor<2x3xf32>') in text
