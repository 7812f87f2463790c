"""GPU checks of jit/lazy execution through rew_mi355x_execute_jit.

The cases follow rew's tests/tjit_execute.nim:78-302 (eager vs jit on the
same inputs) for the ops this backend implements, plus:

* the row sort (stablehlo.sort; src/rew/ops/sort.nim:13-33) against numpy's
  stable argsort (NaN last, -0 == +0), along the last dim and along dim 0,
  ascending and descending, with a carried operand;
* rew's traced topK (sort + slice, src/rew/ops/sort.nim:53-85) equal to the
  eager topK bit for bit and served by the one topK kernel;
* DeepSeekMoE.forward under lazy (its only executable form in rew, since
  topK is trace-only) equal to the eager forward bit for bit, through the
  routed kernels;
* module cache, donation, input checking and unsupported-op errors.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import jit as J
from rew_amd import nn
from rew_amd import ops as O
from rew_amd.eager import DType

from test_gpu_moe import build_moe


def f32(x):
    return E.fromHost(np.asarray(x, np.float32))


def close(got, want, tol=1e-4):
    # tjit_execute.nim:72-75
    got, want = np.asarray(got), np.asarray(want)
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=0, atol=tol)


def test_add_pair_twice_one_module(gpu):
    # tjit_execute.nim:84-97
    E.resetStats()
    j = J.jit(lambda a: [O.add(a[0], a[1])], "addPair")
    a, b = f32([1, 2, 3, 4]), f32([10, 20, 30, 40])
    outs = j.call([a, b])
    assert len(outs) == 1 and outs[0].shape == (4,)
    assert E.toHost(outs[0]).tolist() == [11, 22, 33, 44]
    assert E.toHost(j.call([a, b])[0]).tolist() == [11, 22, 33, 44]
    assert j.cacheSize() == 1
    s = E.stats()
    assert s["jit_module_compiles"] == 1 and s["jit_module_hits"] == 1


def test_lazy_batch_execute(gpu):
    # tjit_execute.nim:99-112
    def f(a):
        y = O.add(a[0], a[1])
        return [O.mul(y, y)]
    lz = J.lazy(f, "lazyBatchExecute")
    outs = lz.call([f32([1, 2, 3, 4]), f32([10, 20, 30, 40])])
    close(E.toHost(outs[0]), [121, 484, 1089, 1936])
    assert lz.cacheSize() == 1


def test_unary_eager_vs_jit(gpu):
    # tjit_execute.nim:114-125
    def f(a):
        x = a[0]
        return [O.cbrt(x), O.ceil(x), O.expm1(x), O.floor(x), O.log1p(x), O.logistic(x),
                O.tan(x), O.sign(x), O.roundNearestAfz(x), O.roundNearestEven(x)]
    x = f32([0.25, 0.5, 1.0, 1.5])
    eager = f([x])
    got = J.jit(f, "openxlaUnary").call([x])
    assert len(got) == len(eager)
    for g, e in zip(got, eager):
        close(E.toHost(g), E.toHost(e))


def test_binary_eager_vs_jit(gpu):
    # tjit_execute.nim:127-138
    f = lambda a: [O.atan2(a[0], a[1]), O.power(a[0], a[1]), O.remainder(a[0], a[1])]
    a, b = f32([1.5, 2.0, 2.5, 3.0]), f32([2.0, 3.0, 2.0, 2.0])
    for g, e in zip(J.jit(f, "openxlaBinary").call([a, b]), f([a, b])):
        close(E.toHost(g), E.toHost(e))


def test_clamp_scalar_bounds_eager_vs_jit(gpu):
    # tjit_execute.nim:140-151
    f = lambda a: [O.clamp(a[1], a[0], a[2])]
    ins = [f32([1, 2, 3, 4]), O.scalarF32(1.5), O.scalarF32(3.5)]
    got = J.jit(f, "clampScalarBounds").call(ins)
    assert got[0].shape == (4,)
    close(E.toHost(got[0]), E.toHost(f(ins)[0]))


def test_dot_eager_vs_jit(gpu):
    # tjit_execute.nim:277-285 (exact equality)
    f = lambda a: [O.dot(O.reshape(a[0], [2, 2]), O.reshape(a[1], [2, 2]))]
    a, b = f32([1, 2, 3, 4]), f32([10, 20, 30, 40])
    assert E.toHost(J.jit(f, "dot").call([a, b])[0]).tolist() == E.toHost(f([a, b])[0]).tolist()


def test_bitwise_eager_vs_jit(gpu):
    # tjit_execute.nim:287-302
    f = lambda a: [O.bitwiseAnd(a[0], a[1]), O.bitwiseOr(a[0], a[1]), O.bitwiseXor(a[0], a[1]),
                   O.bitwiseNot(a[0])]
    x = E.fromHost(np.array([0x0F, 0xF0, 0xAA, 0x55], np.uint32))
    y = E.fromHost(np.array([0xFF, 0x0F, 0x0F, 0xF0], np.uint32))
    for g, e in zip(J.jit(f, "openxlaBitwise").call([x, y]), f([x, y])):
        assert E.toHost(g).tolist() == E.toHost(e).tolist()


def _np_sort(x, axis, descending):
    """Stable order: NaN last, -0 == +0 (the comparator's equivalence)."""
    key = np.where(x == 0, 0, x).astype(np.float64) if x.dtype.kind == "f" else x.astype(np.int64)
    if descending:
        key = -key
    return np.argsort(key, axis=axis, kind="stable")


@pytest.mark.parametrize("rows,cols,axis", [(5, 7, 1), (3, 64, 1), (2, 300, 1), (4, 4100, 1),
                                            (37, 6, 0)])
@pytest.mark.parametrize("direction", ["LT", "GE"])
def test_sort_against_stable_argsort(gpu, rows, cols, axis, direction):
    rs = np.random.default_rng(rows * 131 + cols)
    x = rs.integers(-4, 5, size=(rows, cols)).astype(np.float32)   # many ties
    x[rs.random(x.shape) < 0.05] = np.nan
    x[rs.random(x.shape) < 0.05] = -0.0
    ids = np.broadcast_to(np.arange(x.shape[axis], dtype=np.int32).reshape(
        (-1, 1) if axis == 0 else (1, -1)), x.shape).copy()
    f = lambda a: list(O.sort(a[0], axis, True, direction, a[1]))
    vals, idx = J.jit(f, f"sort{axis}{direction}").call([E.fromHost(x), E.fromHost(ids)])
    order = _np_sort(x, axis, direction in ("GT", "GE"))
    np.testing.assert_array_equal(E.toHost(idx), np.take_along_axis(ids, order, axis))
    np.testing.assert_array_equal(E.toHost(vals).view(np.uint32),
                                  np.take_along_axis(x, order, axis).view(np.uint32))
    if axis == x.ndim - 1:   # the eager extension op (last dim) gives the same bits
        ev, ei = O.sort(E.fromHost(x), axis, True, direction, E.fromHost(ids))
        np.testing.assert_array_equal(E.toHost(ei), E.toHost(idx))


@pytest.mark.parametrize("dt", [DType.BFLOAT16, DType.INT32])
def test_sort_key_dtypes(gpu, dt):
    rs = np.random.default_rng(7)
    x = rs.integers(-1000, 1000, size=(9, 333)).astype(np.float32)
    t = E.fromHost(x, dt) if dt == DType.BFLOAT16 else E.fromHost(x.astype(np.int32))
    got = E.toHost(O.sort(t, -1, True, "GT"))
    ref = (E.bf16_bits_to_f32(E.f32_to_bf16_bits(x)).reshape(x.shape) if dt == DType.BFLOAT16
           else x.astype(np.int32))
    want = np.take_along_axis(ref, _np_sort(ref, 1, True), 1)
    if dt == DType.BFLOAT16:
        got = E.bf16_bits_to_f32(got)
    np.testing.assert_array_equal(got, want)


def test_traced_topk_equals_eager_topk(gpu):
    rs = np.random.default_rng(3)
    p = rs.random((513, 64)).astype(np.float32)
    p[5, 10] = p[5, 20]   # an exact tie: lower index first
    xt = E.fromHost(p)
    j = J.jit(lambda a: list(O.topK(nn.softmax(a[0], 1), 6, 1, True)), "topk")
    E.profileBegin()
    tv, ti = j.call([xt])
    tv, ti = E.toHost(tv), E.toHost(ti)
    names = [n for n, _, _ in E.profileEnd()]
    assert any(n.startswith("topk{") for n in names), names
    assert not any(n.startswith("sort{") for n in names), names
    ev, ei = O.topK(nn.softmax(xt, 1), 6, 1, True)
    np.testing.assert_array_equal(ti, E.toHost(ei))
    np.testing.assert_array_equal(tv.view(np.uint32), E.toHost(ev).view(np.uint32))


def test_moe_lazy_equals_eager(gpu, oracle):
    T, H, I, E_, k, S = 256, 256, 128, 16, 4, 2
    moe, host = build_moe(oracle, T, H, I, E_, k, S, 0x5EED0505)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    params = nn.moeParams(moe)
    lz = J.lazy(lambda a: [nn.moeFromParams(a[1:], S, E_, k).forward(a[0])], "deepseekMoE")
    E.profileBegin()
    got = E.toHost(lz.call([xt] + params)[0])
    names = [n for n, _, _ in E.profileEnd()]
    assert any(n.startswith("moe_gemm_swiglu") for n in names), names
    # the traced topK (sort + slice) became one topK node, which the router
    # launch takes in along with the router's Linear and softmax
    assert any(n.startswith("moe_router{") for n in names), names
    assert not any(n.startswith("sort{") for n in names), names
    want = E.toHost(moe.forward(xt))
    np.testing.assert_array_equal(got, want)
    again = E.toHost(lz.call([xt] + params)[0])
    np.testing.assert_array_equal(again, want)
    assert lz.cacheSize() == 1


def test_reduce_with_a_non_identity_init(gpu):
    text = """module @trace_module {
  func.func @main(%v1: tensor<4x3xf32>) -> tensor<4xf32> {
    %v2 = stablehlo.constant dense<"0x00002041"> : tensor<f32>
    %v6 = stablehlo.reduce(%v1 init: %v2) across dimensions = [1] : (tensor<4x3xf32>, tensor<f32>) -> tensor<4xf32>
      reducer(%v3: tensor<f32>, %v4: tensor<f32>) {
        %v5 = stablehlo.add %v3, %v4 : tensor<f32>
        stablehlo.return %v5 : tensor<f32>
      }
    func.return %v6 : tensor<4xf32>
  }
}
"""
    x = np.arange(12, dtype=np.float32).reshape(4, 3)
    (r,) = J.executeJit("reduceInit", "k", text, [E.fromHost(x)], [DType.FLOAT32], [[4]])
    np.testing.assert_array_equal(E.toHost(r), x.sum(1) + 10.0)


def test_splat_constants_exact(gpu):
    """Splat constants as MLIR prints them: integers beyond 2^53 and at the
    ends of their type's range are taken exactly, and an unquoted hex splat is
    the element's bit pattern (dense<0xFF800000> is -inf in f32).  An integer
    splat out of its type's range is an error, not a wrapped value."""
    text = """module @m {
  func.func @main(%v1: tensor<2xf32>) -> (tensor<3xi64>, tensor<3xi64>, tensor<2xui64>, tensor<2xf32>) {
    %v2 = stablehlo.constant dense<9007199254740993> : tensor<3xi64>
    %v3 = stablehlo.constant dense<-9223372036854775808> : tensor<3xi64>
    %v4 = stablehlo.constant dense<18446744073709551615> : tensor<2xui64>
    %v5 = stablehlo.constant dense<0xFF800000> : tensor<2xf32>
    %v6 = stablehlo.add %v1, %v5 : tensor<2xf32>
    func.return %v2, %v3, %v4, %v6 : tensor<3xi64>, tensor<3xi64>, tensor<2xui64>, tensor<2xf32>
  }
}
"""
    outs = J.executeJit("splats", "k", text, [E.fromHost(np.ones(2, np.float32))],
                        [DType.INT64, DType.INT64, DType.UINT64, DType.FLOAT32],
                        [[3], [3], [2], [2]])
    r5, r7, r9, r11 = (E.toHost(t) for t in outs)
    np.testing.assert_array_equal(r5, [9007199254740993] * 3)
    np.testing.assert_array_equal(r7, [np.iinfo(np.int64).min] * 3)
    np.testing.assert_array_equal(r9, [np.iinfo(np.uint64).max] * 2)
    assert np.all(np.isneginf(r11))
    bad = """module @m {
  func.func @main(%v1: tensor<2xui8>) -> tensor<2xui8> {
    %v2 = stablehlo.constant dense<300> : tensor<2xui8>
    %v3 = stablehlo.add %v1, %v2 : tensor<2xui8>
    func.return %v3 : tensor<2xui8>
  }
}
"""
    with pytest.raises(E.EagerError, match="integer constant 300 is out of range"):
        J.executeJit("badsplat", "k", bad, [E.fromHost(np.zeros(2, np.uint8))],
                     [DType.UINT8], [[2]])


def test_donated_input_is_rejected_afterwards(gpu):
    j = J.jit(lambda a: [O.add(a[0], a[0])], "donate", donateArgs=[0])
    x = f32([1, 2])
    y = j.call([x])[0]
    assert E.toHost(y).tolist() == [2, 4]
    with pytest.raises(E.BufferDonatedError, match="donated to: jit 'donate'"):
        E.toHost(x)


def test_input_mismatch_and_unsupported_op(gpu):
    text = J.jit(lambda a: [O.neg(a[0])], "neg").executableText([f32([1, 2])])
    with pytest.raises(E.EagerError, match="input 0 is dtFloat32\\[3\\], the module expects"):
        J.executeJit("neg", "k", text, [f32([1, 2, 3])], [DType.FLOAT32], [[3]])
    bad = """module @m {
  func.func @main(%v1: tensor<2xf32>) -> tensor<2xf32> {
    %v2 = stablehlo.convolution %v1 : tensor<2xf32>
    func.return %v2 : tensor<2xf32>
  }
}
"""
    with pytest.raises(E.EagerError, match="line 3: stablehlo.convolution: op not supported"):
        J.executeJit("conv", "k", bad, [f32([1, 2])], [DType.FLOAT32], [[2]])


GATHER_CASES = [
    # (x shape, idx, dims kwargs for the oracle) -- index_select rows, points,
    # clamped windows, batching dims
    ((6, 5), np.array([[3], [0], [5], [5], [1], [-2], [9]], np.int32),
     dict(offset_dims=[1], collapsed=[0], start_index_map=[0], ivd=1, slice_sizes=[1, 5])),
    ((5, 7), np.array([[0, 0], [4, 6], [2, 3], [1, 5]], np.int32),
     dict(offset_dims=[], collapsed=[0, 1], start_index_map=[0, 1], ivd=1, slice_sizes=[1, 1])),
    ((5, 7), np.array([[0, 0], [4, 6], [2, 3], [1, 5]], np.int64),
     dict(offset_dims=[1, 2], collapsed=[], start_index_map=[0, 1], ivd=1, slice_sizes=[2, 3])),
    ((3, 6, 4), np.random.default_rng(3).integers(0, 6, size=(3, 5)).astype(np.int32),
     dict(offset_dims=[2], collapsed=[1], start_index_map=[1], ivd=2, slice_sizes=[1, 1, 4],
          operand_batching=[0], start_batching=[0])),
]


def _gdims(kw):
    return O.GatherDimensionNumbers(kw["offset_dims"], kw["collapsed"], kw["start_index_map"],
                                    kw["ivd"], kw.get("operand_batching", ()),
                                    kw.get("start_batching", ()))


@pytest.mark.parametrize("case", range(len(GATHER_CASES)))
def test_gather_eager_and_jit_against_oracle(gpu, oracle, case):
    shape, idx, kw = GATHER_CASES[case]
    x = np.random.default_rng(case).standard_normal(shape).astype(np.float32)
    want = oracle.gather(x, idx, **kw)
    dims, ss = _gdims(kw), kw["slice_sizes"]
    xt, it = E.fromHost(x), E.fromHost(idx)
    eager = O.gather(xt, it, dims, ss, want.shape)
    np.testing.assert_array_equal(E.toHost(eager), want)
    (jitted,) = J.jit(lambda a: [O.gather(a[0], a[1], dims, ss, want.shape)],
                      f"gather{case}").call([xt, it])
    np.testing.assert_array_equal(E.toHost(jitted), want)


@pytest.mark.parametrize("op", ["add", "maximum", "minimum", "multiply", "replace"])
@pytest.mark.parametrize("dt", [DType.FLOAT32, DType.INT32, DType.BFLOAT16])
def test_scatter_eager_and_jit_against_oracle(gpu, oracle, op, dt):
    rs = np.random.default_rng(11)
    x = rs.integers(-4, 5, size=(6, 3)).astype(np.float32)
    upd = rs.integers(-4, 5, size=(7, 3)).astype(np.float32)
    if op == "replace":   # unique in-range indices: the result is order-free
        idx = np.array([[1], [4], [0], [9], [-1], [5], [2]], np.int32)
    else:                 # duplicates and two out-of-range rows (skipped)
        idx = np.array([[1], [4], [1], [9], [4], [-1], [4]], np.int32)
    dims = O.ScatterDimensionNumbers([1], [0], [0], 1)
    want = oracle.scatter(x, idx, upd, update_window_dims=[1], inserted=[0],
                          scatter_dims_to_operand=[0], ivd=1, op=op)
    np_dt = {DType.FLOAT32: np.float32, DType.INT32: np.int32}.get(dt)
    mk = (lambda a: E.fromHost(a.astype(np_dt))) if np_dt else (lambda a: E.fromHost(a, dt))
    rd = (lambda t: E.toHost(t).astype(np.float32)) if np_dt else (lambda t: E.toHostF32(t))
    xt, it, ut = mk(x), E.fromHost(idx), mk(upd)
    (eager,) = O.scatter([xt], it, [ut], dims, op)
    np.testing.assert_array_equal(rd(eager), want)   # small integers: every order is exact
    (jitted,) = J.jit(lambda a: O.scatter([a[0]], a[1], [a[2]], dims, op),
                      f"scatter_{op}_{int(dt)}").call([xt, it, ut])
    np.testing.assert_array_equal(rd(jitted), want)


def test_pad_and_dynamic_slices_eager_and_jit(gpu, oracle):
    """stablehlo.pad / dynamic_slice / dynamic_update_slice in rew's generic
    text form (src/rew/stablehlo/text.nim:589-690) equal the eager ops and
    the oracle bit for bit, the start indices passed as module inputs."""
    rs = np.random.default_rng(31)
    x = rs.standard_normal((6, 9)).astype(np.float32)
    u = rs.standard_normal((2, 4)).astype(np.float32)
    xt, ut, vt = E.fromHost(x), E.fromHost(u), E.fromHost(np.float32(-2.0))
    s0, s1 = E.fromHost(np.int32(5)), E.fromHost(np.int32(-3))   # both clamp

    def fn(a):
        p = O.pad(a[0], a[2], [1, -1], [2, 0], [1, 2])
        d = O.dynamicSlice(a[0], [a[3], a[4]], [3, 4])
        w = O.dynamicUpdateSlice(a[0], a[1], [a[3], a[4]])
        return [p, d, w]

    eager = [E.toHost(t) for t in fn([xt, ut, vt, s0, s1])]
    jitted = [E.toHost(t) for t in J.jit(fn, "pad_dslice").call([xt, ut, vt, s0, s1])]
    want = [oracle.pad(x, np.float32(-2.0), [1, -1], [2, 0], [1, 2]),
            oracle.dynamic_slice(x, [5, -3], [3, 4]),
            oracle.dynamic_update_slice(x, u, [5, -3])]
    for e, j, w in zip(eager, jitted, want):
        np.testing.assert_array_equal(e, w)
        np.testing.assert_array_equal(j, w)
