"""GPU checks of jit modules with control flow (stablehlo.while / if / case,
traced by rew_amd.control as rew's src/rew/transform/control.nim traces
them) run through rew_mi355x_execute_jit: the library runs the regions on
the host side of the call and reads each predicate back from the device.
Results are checked against numpy restatements of the same loops."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import control as K
from rew_amd import eager as E
from rew_amd import jit as J
from rew_amd import ops as O
from rew_amd.eager import DType


def f32(x):
    return E.fromHost(np.asarray(x, np.float32))


def test_fori_accumulates(gpu):
    # twhile.nim:49-64 executed: carry + x, four times
    j = J.jit(lambda a: K.fori(0, 4, [a[0]], lambda i, c: [O.add(c[0], a[0])]), "foriAcc")
    x = np.array([1.5, -2.0, 3.25], np.float32)
    out = E.toHost(j.call([f32(x)])[0])
    want = x.copy()
    for _ in range(4):
        want = want + x
    assert out.tolist() == want.tolist()
    # a second call reuses the module and runs the loop again
    assert E.toHost(j.call([f32(2 * x)])[0]).tolist() == (5 * 2 * x).tolist()


def test_while_data_dependent_trip_count(gpu):
    # doubles v until its sum passes the limit; the counter is carried too
    def f(a):
        limit = O.scalarF32(100.0)
        outs = K.whileLoop(
            [O.scalarI32(0), a[0]],
            lambda c: O.compare(O.reduceSum(c[1], [0]), limit, "LT"),
            lambda c: [O.add(c[0], O.scalarI32(1)), O.add(c[1], c[1])])
        return outs
    j = J.jit(f, "whileDouble")
    for x in ([1, 2, 3], [60, 50, 1], [0.5, 0.25, 0.25]):
        x = np.asarray(x, np.float32)
        n, v = j.call([f32(x)])
        k, w = 0, x.copy()
        while w.sum() < 100:
            k, w = k + 1, w + w
        assert int(E.toHost(n)) == k and E.toHost(v).tolist() == w.tolist()


def test_cond_picks_branch_from_data(gpu):
    def f(a):
        p = O.compare(O.reduceSum(a[0], [0]), O.scalarF32(0.0), "GT")
        return K.condN(p, lambda: [O.mul(a[0], a[0]), O.exp(a[0])],
                       lambda: [O.neg(a[0]), a[0]])
    j = J.jit(f, "condPick")
    pos = np.array([1.0, 2.0, -0.5], np.float32)
    neg = -pos
    y0, y1 = j.call([f32(pos)])
    assert E.toHost(y0).tolist() == (pos * pos).tolist()
    ref = E.toHost(O.exp(f32(pos)))  # the eager op of the same kernel family
    np.testing.assert_allclose(E.toHost(y1), ref, rtol=1e-6, atol=0)
    z0, z1 = j.call([f32(neg)])
    assert E.toHost(z0).tolist() == pos.tolist() and E.toHost(z1).tolist() == neg.tolist()


def test_case_index_and_out_of_range_runs_last(gpu):
    def f(a):
        idx = O.astype(O.reduceSum(a[1], [0]), DType.INT32)
        return K.caseOp(idx, [lambda: [O.add(a[0], a[0])], lambda: [O.neg(a[0])],
                              lambda: [O.mul(a[0], a[0])]])
    j = J.jit(f, "caseIdx")
    x = np.array([1.0, -3.0, 0.5, 2.0], np.float32)
    for k, want in ((0, x + x), (1, -x), (2, x * x), (7, x * x), (-1, x * x)):
        out = j.call([f32(x), f32([float(k)])])[0]
        assert E.toHost(out).tolist() == want.tolist(), k


def test_cond_nested_in_loop_under_lazy(gpu):
    # collatz-style step on a counter vector, lazy form (rew's lazy of a loop)
    def f(a):
        def body(c):
            v = c[0]
            even = O.compare(O.reduceSum(v, [0]), O.scalarF32(10.0), "GT")
            half, three, one = (O.constant(DType.FLOAT32, [2], [c, c]) for c in (0.5, 3.0, 1.0))
            nv = K.cond(even, lambda: O.mul(v, half), lambda: O.add(O.mul(v, three), one))
            return [nv, O.add(c[1], O.scalarI32(1))]
        return K.whileLoop([a[0], O.scalarI32(0)],
                           lambda c: O.compare(c[1], O.scalarI32(6), "LT"), body)
    lz = J.lazy(f, "lazyNested")
    x = np.array([1.0, 2.0], np.float32)
    v, n = lz.call([f32(x)])
    w = x.copy()
    for _ in range(6):
        w = w * np.float32(0.5) if w.sum() > 10 else w * np.float32(3.0) + np.float32(1.0)
    assert int(E.toHost(n)) == 6 and E.toHost(v).tolist() == w.tolist()


def test_edge_cases_zero_trip_single_branch_nested_loops(gpu):
    # a loop whose predicate is false at once returns its initial carry;
    # a one-branch case runs it whatever the index; loops nest
    def f(a):
        z = K.whileLoop([a[0]], lambda c: O.compare(O.reduceSum(c[0], [0]),
                                                    O.scalarF32(-1e9), "LT"),
                        lambda c: [O.neg(c[0])])
        s = K.caseOp(O.scalarI32(5), [lambda: [O.add(a[0], a[0])]])
        outer = K.fori(0, 3, [a[0]], lambda i, c: K.fori(0, 2, [c[0]],
                                                         lambda j, d: [O.add(d[0], a[0])]))
        return [z[0], s[0], outer[0]]
    x = np.array([1.0, -2.0, 0.5], np.float32)
    z, s, o = J.jit(f, "edgeLoops").call([f32(x)])
    assert E.toHost(z).tolist() == x.tolist()
    assert E.toHost(s).tolist() == (x + x).tolist()
    assert E.toHost(o).tolist() == (x * 7).tolist()


def test_scan_running_sum(gpu):
    # control.nim scan: carry the running sum of the rows of xs, emit each
    # row's dot with w as a scalar y
    def f(a):
        def body(carry, x):
            s = O.add(carry[0], x[0])
            y = O.reduceSum(O.mul(x[0], a[1]), [0])
            return [s], [y]
        carry, ys = K.scan([a[2]], [a[0]], body)
        return [carry[0], ys[0]]
    xs = np.random.default_rng(3).standard_normal((5, 4)).astype(np.float32)
    w = np.array([1.0, -1.0, 0.5, 2.0], np.float32)
    c0 = np.zeros(4, np.float32)
    carry, ys = J.jit(f, "scanSum").call([f32(xs), f32(w), f32(c0)])
    want_c = c0.copy()
    for r in xs:
        want_c = want_c + r
    assert E.toHost(carry).tolist() == want_c.tolist()
    got = E.toHost(ys)
    assert got.shape == (5,)
    np.testing.assert_allclose(got, (xs * w).sum(1), rtol=1e-5, atol=1e-6)
