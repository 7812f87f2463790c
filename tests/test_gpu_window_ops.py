"""GPU parity of the eager ops of rew's table outside the configs
(src/rew/eager.nim:838-850): pad, dynamicSlice, dynamicUpdateSlice,
getDimensionSize, replicaId / partitionId, setDimensionSize, dynamicReshape,
dynamicIota and cholesky, through the C ABI against the oracle.

Tolerances: every layout op and constant is bit-exact (any dtype);
cholesky is within 1e-5 relative (f32) or 1e-12 (f64) of the float64
oracle, normwise per matrix.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import ops as O
from rew_amd.eager import DType


def dev(a, dt=None):
    return E.fromHost(np.asarray(a), dt)


def host(t):
    return E.toHost(t)


def scalar(v, dt=np.int32):
    return dev(np.array(v, dt))


@pytest.fixture(params=[E.MODE_DEFERRED, E.MODE_OP_BY_OP], ids=["deferred", "op_by_op"])
def mode(request, gpu):
    E.setMode(request.param)
    yield request.param
    E.setMode(E.MODE_DEFERRED)


def test_known_answers(mode):
    """tests/teager_dispatch.nim:465-531."""
    spd = dev(np.array([[4, 2], [2, 3]], np.float32))
    dim = O.getDimensionSize(spd, 0)
    assert dim.dtype == DType.INT32 and tuple(dim.shape) == ()
    assert int(host(dim)) == 2
    padded = O.pad(spd, dev(np.float32(0)), [1, 1], [1, 1], [0, 0])
    assert tuple(padded.shape) == (4, 4)
    np.testing.assert_array_equal(host(padded).ravel(),
                                  [0, 0, 0, 0, 0, 4, 2, 0, 0, 2, 3, 0, 0, 0, 0, 0])
    chol = host(O.cholesky(spd))
    np.testing.assert_allclose(chol.ravel(), [2, 0, 1, np.sqrt(np.float32(2))], rtol=1e-6)

    x = dev(np.array([[1, 2], [3, 4]], np.float32))
    s0, s1 = scalar(0), scalar(1)
    sl = O.dynamicSlice(x, [s0, s1], [2, 1])
    assert tuple(sl.shape) == (2, 1)
    np.testing.assert_array_equal(host(sl).ravel(), [2, 4])
    up = O.dynamicUpdateSlice(x, dev(np.array([[9]], np.float32)), [s0, s1])
    np.testing.assert_array_equal(host(up).ravel(), [1, 9, 3, 4])

    rid, pid = O.replicaId(), O.partitionId()
    assert rid.dtype == DType.UINT32 and pid.dtype == DType.UINT32
    assert int(host(rid)) == 0 and int(host(pid)) == 0

    sized = O.setDimensionSize(x, scalar(2), 0)
    assert tuple(sized.shape) == (2, 2)
    np.testing.assert_array_equal(host(sized), host(x))
    resh = O.dynamicReshape(x, dev(np.array([4], np.int32)), [4])
    np.testing.assert_array_equal(host(resh), [1, 2, 3, 4])
    dio = O.dynamicIota(DType.INT32, dev(np.array([2, 3], np.int32)), [2, 3], 1)
    np.testing.assert_array_equal(host(dio).ravel(), [0, 1, 2, 0, 1, 2])


@pytest.mark.parametrize("dt", [np.float32, np.int8, np.int64, "bf16"])
def test_pad_any_dtype(mode, oracle, dt):
    """Edge padding (negative edges crop) and interior padding, rank 3,
    bit-exact against the oracle."""
    rs = np.random.default_rng(11)
    raw = rs.integers(-100, 100, (5, 6, 7))
    if dt == "bf16":
        xh = raw.astype(np.float32)
        x, v = dev(xh, DType.BFLOAT16), dev(np.float32(-3.5), DType.BFLOAT16)
        want = oracle.pad(xh, np.float32(-3.5), [2, -1, 0], [-2, 3, 1], [1, 0, 2])
        got = E.toHostF32(O.pad(x, v, [2, -1, 0], [-2, 3, 1], [1, 0, 2]))
    else:
        xh = raw.astype(dt)
        x, v = dev(xh), dev(np.array(-3, dt))
        want = oracle.pad(xh, dt(-3), [2, -1, 0], [-2, 3, 1], [1, 0, 2])
        got = host(O.pad(x, v, [2, -1, 0], [-2, 3, 1], [1, 0, 2]))
    np.testing.assert_array_equal(got, want)


def test_pad_inside_a_fused_graph(gpu, oracle):
    """pad between elementwise producers and consumers in one deferred flush:
    relu(pad(x + x) * 2) against the oracle."""
    rs = np.random.default_rng(12)
    xh = rs.standard_normal((33, 65)).astype(np.float32)
    x = dev(xh)
    y = O.pad(O.add(x, x), dev(np.float32(-1)), [1, 0], [0, 2], [1, 1])
    z = O.maximum(O.mul(y, O.broadcastTo(dev(np.float32(2)), list(y.shape), [])),
                  O.broadcastTo(dev(np.float32(0)), list(y.shape), []))
    want = np.maximum(oracle.pad(xh + xh, np.float32(-1), [1, 0], [0, 2], [1, 1]) * 2, 0)
    np.testing.assert_array_equal(host(z), want)


@pytest.mark.parametrize("idx_dt", [np.int32, np.int64, np.uint32, np.uint64, np.int8])
def test_dynamic_slice_clamps(mode, oracle, idx_dt):
    """Starts outside [0, dim - size] clamp (negative, past the end, a uint64
    above INT64_MAX), any integer start dtype, bit-exact."""
    rs = np.random.default_rng(13)
    xh = rs.standard_normal((9, 10, 11)).astype(np.float32)
    x = dev(xh)
    signed = np.issubdtype(idx_dt, np.signedinteger)
    cases = [([2, 3, 4], [3, 4, 5]), ([100, 0, 7], [4, 10, 1]), ([0, 0, 0], [9, 10, 11]),
             ([5, 9, 10], [0, 2, 3])]
    if signed:
        cases.append(([-5, 2, -1], [2, 2, 2]))
    if idx_dt == np.uint64:
        cases.append(([2**64 - 1, 1, 2**63], [2, 2, 2]))
    for starts, sizes in cases:
        st = [dev(np.array(s, dtype=idx_dt)) for s in starts]
        got = host(O.dynamicSlice(x, st, sizes))
        want = oracle.dynamic_slice(xh, [min(s, 2**62) for s in starts], sizes)
        np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("dt", [np.float32, np.int16, "bf16"])
def test_dynamic_update_slice(mode, oracle, dt):
    rs = np.random.default_rng(14)
    raw = rs.integers(-1000, 1000, (8, 12))
    uraw = rs.integers(-1000, 1000, (3, 5))
    for starts in ([2, 4], [-3, 10], [7, 7], [0, 0]):
        st = [dev(np.array(s, np.int32)) for s in starts]
        if dt == "bf16":
            xh = oracle.round_bf16(raw.astype(np.float32))   # bf16-exact values
            uh = oracle.round_bf16(uraw.astype(np.float32))
            got = E.toHostF32(O.dynamicUpdateSlice(dev(xh, DType.BFLOAT16),
                                                   dev(uh, DType.BFLOAT16), st))
        else:
            xh, uh = raw.astype(dt), uraw.astype(dt)
            got = host(O.dynamicUpdateSlice(dev(xh), dev(uh), st))
        np.testing.assert_array_equal(got, oracle.dynamic_update_slice(xh, uh, starts))


@pytest.mark.parametrize("dt,n,lower", [(np.float32, 5, True), (np.float32, 64, False),
                                        (np.float64, 33, True), (np.float64, 1, False)])
def test_cholesky_batches(mode, oracle, dt, n, lower):
    rs = np.random.default_rng(15 + n)
    m = rs.standard_normal((3, 2, n, n))
    spd = m @ m.transpose(0, 1, 3, 2) + n * np.eye(n)
    xh = spd.astype(dt)
    if lower:
        xh = xh + np.triu(np.full((n, n), 1e3, dt), 1)   # the other triangle is not read
    else:
        xh = xh + np.tril(np.full((n, n), 1e3, dt), -1)
    got = host(O.cholesky(dev(xh), lower))
    want = oracle.cholesky(xh, lower)
    tol = 1e-5 if dt == np.float32 else 1e-12
    err = np.abs(got - want).reshape(6, -1).max(axis=1)
    assert np.all(err <= tol * np.abs(want).reshape(6, -1).max(axis=1)), err
    tri = np.tril(np.ones((n, n))) if lower else np.triu(np.ones((n, n)))
    assert np.all(got[..., tri == 0] == 0)


def test_validation_errors(gpu):
    x = dev(np.zeros((2, 3), np.float32))
    with pytest.raises(E.TensorError, match="paddingValue"):
        O.pad(x, dev(np.int32(0)), [0, 0], [0, 0], [0, 0])
    with pytest.raises(E.TensorError, match="start index count"):
        O.dynamicSlice(x, [scalar(0)], [1, 1])
    with pytest.raises(E.TensorError, match="out of range"):
        O.dynamicSlice(x, [scalar(0), scalar(0)], [3, 1])
    with pytest.raises(E.TensorError, match="square"):
        O.cholesky(x)
    # the backend's own checks (bypassing the mirror) raise EagerError
    with pytest.raises(E.EagerError, match="interior padding"):
        E.dispatchEager("pad", [x, dev(np.float32(0))],
                        [("edge_padding_low", "[0,0]"), ("edge_padding_high", "[0,0]"),
                         ("interior_padding", "[-1,0]")])
    with pytest.raises(E.EagerError, match="not implemented natively"):
        E.dispatchEager("conv2d", [x], [])


def test_batch_norm_known_answers(mode):
    """tests/teager_dispatch.nim:426-463."""
    a = dev(np.array([1, 2, 3, 4], np.float32))
    one, zero = dev(np.ones(4, np.float32)), dev(np.zeros(4, np.float32))
    r = O.batchNormInference(a, one, zero, one, one, 0.0, 0)
    assert r.dtype == DType.FLOAT32
    np.testing.assert_array_equal(host(r), [0, 1, 2, 3])
    x = dev(np.array([[1, 2], [3, 4]], np.float32))
    o2, z2 = dev(np.ones(2, np.float32)), dev(np.zeros(2, np.float32))
    y, m, v = O.batchNormTraining(x, o2, z2, 0.0, 1)
    assert tuple(y.shape) == (2, 2) and tuple(m.shape) == (2,) and tuple(v.shape) == (2,)
    np.testing.assert_allclose(host(y).ravel(), [-1, -1, 1, 1], rtol=1e-6)
    np.testing.assert_array_equal(host(m), [2, 3])
    np.testing.assert_array_equal(host(v), [1, 1])
    g = dev(np.full((2, 2), 0.1, np.float32))
    dx, ds, do = O.batchNormGrad(x, o2, dev(np.array([2, 3], np.float32)), o2, g, 0.0, 1)
    np.testing.assert_allclose(host(dx).ravel(), 0, atol=1e-7)
    np.testing.assert_allclose(host(ds), 0, atol=1e-7)
    np.testing.assert_allclose(host(do), [0.2, 0.2], rtol=1e-6)


@pytest.mark.parametrize("dt", [np.float32, np.float64])
def test_batch_norm_empty_batch(mode, dt):
    """An empty batch ([0, C], feature dim 1) still gives the [C] outputs:
    batchNormTraining's mean and variance are 0 / 0 = NaN, batchNormGrad's
    gradient sums over no elements are 0, and the [0, C] results are empty."""
    C = 5
    x = np.zeros((0, C), dt)
    sc, of = np.ones(C, dt), np.zeros(C, dt)
    y, m, v = O.batchNormTraining(dev(x), dev(sc), dev(of), 1e-3, 1)
    assert host(y).shape == (0, C)
    assert np.all(np.isnan(host(m))) and np.all(np.isnan(host(v)))
    dx, ds, do = O.batchNormGrad(dev(x), dev(sc), dev(np.zeros(C, dt)), dev(np.ones(C, dt)),
                                 dev(x), 1e-3, 1)
    assert host(dx).shape == (0, C)
    np.testing.assert_array_equal(host(ds), 0)
    np.testing.assert_array_equal(host(do), 0)


@pytest.mark.parametrize("dt,shape,fi", [(np.float32, (8, 16, 33), 1), (np.float64, (5, 7), 0),
                                         (np.float32, (4, 3, 2, 64), 3)])
def test_batch_norm_against_oracle(mode, oracle, dt, shape, fi):
    """All three forms against the float64 oracle: within 1e-5 (f32) or
    1e-12 (f64) relative, normwise per output."""
    rs = np.random.default_rng(22 + fi)
    C = shape[fi]
    x = (rs.standard_normal(shape) * 3 + 1).astype(dt)
    sc, of = rs.standard_normal(C).astype(dt), rs.standard_normal(C).astype(dt)
    mu, va = rs.standard_normal(C).astype(dt), (rs.random(C) + 0.5).astype(dt)
    dy = rs.standard_normal(shape).astype(dt)
    eps = 1e-3
    tol = 1e-5 if dt == np.float32 else 1e-12

    def check(got, want):
        got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
        assert np.abs(got - want).max() <= tol * max(np.abs(want).max(), 1.0)

    check(host(O.batchNormInference(dev(x), dev(sc), dev(of), dev(mu), dev(va), eps, fi)),
          oracle.batch_norm_inference(x, sc, of, mu, va, np.float32(eps), fi))
    got = O.batchNormTraining(dev(x), dev(sc), dev(of), eps, fi)
    for g, w in zip(got, oracle.batch_norm_training(x, sc, of, np.float32(eps), fi)):
        check(host(g), w)
    got = O.batchNormGrad(dev(x), dev(sc), dev(mu), dev(va), dev(dy), eps, fi)
    for g, w in zip(got, oracle.batch_norm_grad(x, sc, mu, va, dy, np.float32(eps), fi)):
        check(host(g), w)
