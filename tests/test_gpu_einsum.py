"""GPU checks of einsum / unaryEinsum (src/rew/ops/linalg.nim:378-430) and the
shape-operand ops dynamicPad, realDynamicSlice and dynamicBroadcastInDim
(src/rew/ops/shape.nim:395-517, linalg.nim:288-326), which the library
records as primitive nodes (reduceSum, dotGeneral, transpose; pad, slice,
broadcastTo).  einsum is checked against numpy.einsum in float64 (fp32
tolerance 1e-5 normwise); the index ops bit for bit against numpy."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import ops as O
from rew_amd.eager import DType, EagerError


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


CASES = [
    ("ab,bc->ac", (5, 7), (7, 3)),
    ("bij,bjk->bik", (2, 4, 6), (2, 6, 3)),
    ("ab,bc->ca", (4, 5), (5, 6)),
    ("a,b->ab", (3,), (4,)),
    ("ab,ab->", (6, 5), (6, 5)),
    ("abc,cd->ad", (3, 4, 5), (5, 2)),
    ("ij,kj->ik", (8, 16), (3, 16)),
    ("bhqd,bhkd->bhqk", (2, 3, 5, 8), (2, 3, 7, 8)),
    ("ab,ab->ab", (3, 4), (3, 4)),      # batch only: the elementwise product
    ("ab,b->a", (5, 6), (6,)),          # matrix-vector
    ("i,i->", (7,), (7,)),              # inner product
    ("ab,c->cab", (2, 3), (4,)),        # outer product, reordered
]


@pytest.mark.parametrize("cfg,sa,sb", CASES)
def test_einsum_against_numpy(gpu, cfg, sa, sb):
    a, b = rnd(sa, 1), rnd(sb, 2)
    want = np.einsum(cfg, a.astype(np.float64), b.astype(np.float64))
    got = E.toHost(O.einsum(E.fromHost(a), E.fromHost(b), cfg, list(want.shape)))
    assert got.shape == want.shape
    err = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert err <= 1e-5, (cfg, err)


@pytest.mark.parametrize("cfg,sa", [("abc->cab", (2, 3, 4)), ("abc->b", (3, 4, 5)),
                                    ("ab->", (4, 6)), ("ab->ab", (2, 3))])
def test_unary_einsum_against_numpy(gpu, cfg, sa):
    a = rnd(sa, 3)
    want = np.einsum(cfg, a.astype(np.float64))
    got = E.toHost(O.unaryEinsum(E.fromHost(a), cfg, list(want.shape)))
    assert got.shape == want.shape
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


def test_einsum_errors(gpu):
    a, b = E.fromHost(rnd((3, 3), 4)), E.fromHost(rnd((3, 3), 5))
    with pytest.raises(EagerError, match="repeated"):
        O.einsum(a, b, "aa,ab->b", [3])       # a diagonal: not supported
    with pytest.raises(EagerError, match="->"):
        O.einsum(a, b, "ab,bc", [3, 3])
    with pytest.raises(EagerError, match="output_shape"):
        O.einsum(a, b, "ab,bc->ac", [3, 4])


def test_dynamic_broadcast_pad_slice(gpu):
    x = np.arange(12, dtype=np.float32).reshape(3, 4)
    i32 = lambda v: E.fromHost(np.asarray(v, np.int32))
    # dynamicBroadcastInDim: [3,4] -> [2,3,4] along dims (1, 2)
    got = E.toHost(O.dynamicBroadcastInDim(E.fromHost(x), i32([2, 3, 4]), [2, 3, 4], [1, 2]))
    assert got.tolist() == np.broadcast_to(x, (2, 3, 4)).tolist()
    # dynamicPad with low (1, 0), high (0, 2), interior (1, 1)
    pv = E.fromHost(np.float32(-1.0))
    got = E.toHost(O.dynamicPad(E.fromHost(x), pv, i32([1, 0]), i32([0, 2]), i32([1, 1]),
                                [6, 9]))
    want = np.full((6, 9), -1.0, np.float32)
    want[1::2, 0:7:2] = x
    assert got.tolist() == want.tolist()
    # realDynamicSlice rows 1..3 step 1, cols 0..4 step 2 (int64 bounds)
    i64 = lambda v: E.fromHost(np.asarray(v, np.int64))
    got = E.toHost(O.realDynamicSlice(E.fromHost(x), i64([1, 0]), i64([3, 4]), i64([1, 2]),
                                      [2, 2]))
    assert got.tolist() == x[1:3, 0:4:2].tolist()
    with pytest.raises(EagerError, match="result_shape"):
        O.realDynamicSlice(E.fromHost(x), i64([0, 0]), i64([3, 4]), i64([1, 1]), [2, 2])


@pytest.mark.parametrize("left", [True, False])
@pytest.mark.parametrize("lower", [True, False])
@pytest.mark.parametrize("trans", ["NO_TRANSPOSE", "TRANSPOSE", "ADJOINT"])
@pytest.mark.parametrize("unit", [False, True])
def test_triangular_solve_against_numpy(gpu, left, lower, trans, unit):
    # stablehlo.triangular_solve (src/rew/ops/linalg.nim:350-376): the
    # referenced triangle only (the other one holds junk), batched
    rng = np.random.default_rng(7)
    n, m, bt = 12, 5, 3
    a = rng.standard_normal((bt, n, n)).astype(np.float32)
    a[:, np.arange(n), np.arange(n)] += 4.0 * np.sign(a[:, np.arange(n), np.arange(n)]) + 0.5
    b = rng.standard_normal((bt, n, m) if left else (bt, m, n)).astype(np.float32)
    t = np.tril(a) if lower else np.triu(a)
    if unit:
        t = t.copy()
        t[:, np.arange(n), np.arange(n)] = 1.0
    op = t if trans == "NO_TRANSPOSE" else np.swapaxes(t, 1, 2)
    op64 = op.astype(np.float64)
    want = (np.linalg.solve(op64, b.astype(np.float64)) if left
            else np.swapaxes(np.linalg.solve(np.swapaxes(op64, 1, 2),
                                             np.swapaxes(b.astype(np.float64), 1, 2)), 1, 2))
    got = E.toHost(O.triangularSolve(E.fromHost(a), E.fromHost(b), left, lower, unit, trans))
    assert got.shape == b.shape
    err = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert err <= 1e-5, err


def test_triangular_solve_errors(gpu):
    a = E.fromHost(np.eye(4, dtype=np.float32))
    with pytest.raises(EagerError, match="does not fit"):
        O.triangularSolve(a, E.fromHost(np.ones((3, 2), np.float32)))
    with pytest.raises(EagerError, match="transpose_a"):
        O.triangularSolve(a, E.fromHost(np.ones((4, 2), np.float32)), transposeA="CONJ")


def test_ops_under_jit_equal_eager(gpu):
    # the same ops traced by jit (stablehlo.einsum / unary_einsum /
    # triangular_solve / dynamic_pad / real_dynamic_slice /
    # dynamic_broadcast_in_dim in rew's text forms) give the eager results
    from rew_amd import jit as J
    rng = np.random.default_rng(11)
    a = rng.standard_normal((4, 6)).astype(np.float32)
    b = rng.standard_normal((6, 3)).astype(np.float32)
    t = np.tril(rng.standard_normal((6, 6)).astype(np.float32)) + 4 * np.eye(6, dtype=np.float32)
    i32 = lambda v: E.fromHost(np.asarray(v, np.int32))

    def f(x):
        e = O.einsum(x[0], x[1], "ab,bc->ca", [3, 4])
        u = O.unaryEinsum(x[0], "ab->b", [6])
        s = O.triangularSolve(x[2], x[1], True, True, False, "TRANSPOSE")
        p = O.dynamicPad(x[0], x[3], x[4], x[4], x[5], [6, 11])
        r = O.realDynamicSlice(x[0], x[5], x[6], x[7], [4, 3])
        g = O.dynamicBroadcastInDim(x[1], x[8], [2, 6, 3], [1, 2])
        return [e, u, s, p, r, g]
    ins = [E.fromHost(a), E.fromHost(b), E.fromHost(t), E.fromHost(np.float32(0.5)),
           i32([1, 0]), i32([0, 1]), i32([4, 6]), i32([1, 2]), i32([2, 6, 3])]
    text = J.jit(f, "opsJit").text(ins)
    for mn in ("stablehlo.einsum", "stablehlo.unary_einsum", "stablehlo.triangular_solve",
               "stablehlo.dynamic_pad", "stablehlo.real_dynamic_slice",
               "stablehlo.dynamic_broadcast_in_dim"):
        assert mn in text, mn
    got = [E.toHost(o) for o in J.jit(f, "opsJit").call(ins)]
    want = [E.toHost(o) for o in f(ins)]
    for g_, w_ in zip(got, want):
        assert g_.shape == w_.shape and g_.tolist() == w_.tolist()


def test_largest_triangular_solve_and_edge_transforms(gpu):
    # the 64 x 64 limit, a length-1 FFT, an einsum over an empty batch
    rng = np.random.default_rng(9)
    a = np.tril(rng.standard_normal((64, 64))).astype(np.float64) + 8 * np.eye(64)
    b = rng.standard_normal((64, 3))
    got = E.toHost(O.triangularSolve(E.fromHost(a), E.fromHost(b)))
    np.testing.assert_allclose(got, np.linalg.solve(a, b), rtol=1e-10, atol=1e-12)
    with pytest.raises(EagerError, match="above 64"):
        O.triangularSolve(E.fromHost(np.eye(65)), E.fromHost(np.ones((65, 1))))
    z = (rng.standard_normal((4, 1)) + 1j * rng.standard_normal((4, 1))).astype(np.complex64)
    assert E.toHost(O.fft(E.fromHost(z), "FFT", [1])).tolist() == z.tolist()
    e = E.toHost(O.einsum(E.fromHost(np.zeros((0, 2, 3), np.float32)),
                          E.fromHost(np.zeros((0, 3, 4), np.float32)), "bij,bjk->bik", [0, 2, 4]))
    assert e.shape == (0, 2, 4)
