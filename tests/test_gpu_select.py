"""GPU parity of the index-producing ops: argmax (src/rew/ops/reduce.nim:202-225
semantics) and topK (src/rew/ops/sort.nim:36-90 semantics), bit-exact against
the oracle, plus the MNIST-shaped MLP inference path (config C1) ending in
argmax.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import nn, rng
from rew_amd import ops as O


def dev(a, dt=None):
    return E.fromHost(np.asarray(a), dt)


@pytest.mark.parametrize("shape,dim", [((128, 10), 1), ((33, 1000), 1), ((7, 5, 300), 2),
                                       ((64, 9), 0), ((4, 130, 6), 1), ((1, 1), 1)])
def test_argmax_matches_oracle(gpu, oracle, shape, dim):
    x = oracle.normal_f32(oracle.init_key(sum(shape) + dim), int(np.prod(shape))).reshape(shape)
    got = E.toHost(O.argmax(dev(x), dim))
    xm = np.moveaxis(x, dim, -1)
    want = oracle.argmax_rows(xm.reshape(-1, xm.shape[-1])).reshape(xm.shape[:-1])
    np.testing.assert_array_equal(got, want)


def test_argmax_ties_nan_and_signed_zero(gpu, oracle):
    x = np.array([[1, 3, 3, 2], [np.nan, 1, 2, 3], [-1, -1, -1, -1], [-0.0, 0.0, -0.0, -1],
                  [-np.inf, -np.inf, -np.inf, -np.inf], [2, np.inf, np.inf, np.nan]], np.float32)
    got = E.toHost(O.argmax(dev(x), 1))
    np.testing.assert_array_equal(got, oracle.argmax_rows(x))
    np.testing.assert_array_equal(got, [1, 2147483647, 0, 0, 0, 2147483647])
    # ties planted across lanes of a long row: lowest index wins
    y = np.zeros((3, 4096), np.float32)
    y[0, [100, 7, 4000]] = 5.0
    y[1, [4095, 64, 65]] = 1.0
    y[2, :] = 1.0
    np.testing.assert_array_equal(E.toHost(O.argmax(dev(y), 1)), [7, 64, 0])


@pytest.mark.parametrize("rows,cols,k", [(8192, 64, 6), (50, 64, 1), (17, 100, 7),
                                         (5, 4096, 64), (3, 64, 64), (2, 1, 1)])
def test_topk_matches_oracle(gpu, oracle, rows, cols, k):
    x = oracle.normal_f32(oracle.init_key(rows * cols + k), rows * cols).reshape(rows, cols)
    v, i = O.topK(dev(x), k, -1, True)
    wv, wi = oracle.topk_rows(x, k)
    np.testing.assert_array_equal(E.toHost(i), wi)
    np.testing.assert_array_equal(E.toHost(v).view(np.uint32), wv.view(np.uint32))


def test_topk_ties_nan_and_smallest(gpu, oracle):
    x = np.array([[0.1, 0.5, 0.5, 0.2, 0.9, np.nan, 0.5, -1.0]], np.float32)
    v, i = O.topK(dev(x), 5, -1, True)
    np.testing.assert_array_equal(E.toHost(i), [[4, 1, 2, 6, 3]])
    # NaN ranks after every number, so the 8th pick is the NaN
    v8, i8 = O.topK(dev(x), 8, -1, True)
    np.testing.assert_array_equal(E.toHost(i8), [[4, 1, 2, 6, 3, 0, 7, 5]])
    # smallest first (LE comparator): ties to the lower index, NaN last
    vs, is_ = O.topK(dev(x), 8, -1, False)
    np.testing.assert_array_equal(E.toHost(is_), [[7, 0, 3, 1, 2, 6, 4, 5]])
    np.testing.assert_array_equal(E.toHost(vs)[0, :7], x[0, [7, 0, 3, 1, 2, 6, 4]])
    # many equal keys spread over lanes and slots
    y = np.ones((4, 1000), np.float32)
    y[:, 500] = 2.0
    _, iy = O.topK(dev(y), 10, -1, True)
    np.testing.assert_array_equal(E.toHost(iy), np.tile([500, 0, 1, 2, 3, 4, 5, 6, 7, 8], (4, 1)))


def test_topk_rejects_out_of_range(gpu):
    with pytest.raises(E.EagerError):
        O.topK(dev(np.zeros((2, 5000), np.float32)), 4, -1, True)
    with pytest.raises(E.TensorError):
        O.topK(dev(np.zeros((2, 8), np.float32)), 9, -1, True)


@pytest.mark.parametrize("M,K,N1,N2,fused", [(128, 784, 128, 10, True), (130, 100, 64, 7, True),
                                             (33, 100, 128, 70, False)])
def test_mlp_forward_two_launches(gpu, oracle, M, K, N1, N2, fused):
    """rew's MLP forward -- Linear, relu, Linear, softmax, argmax
    (nn/linear.nim:43-49, nn/activation.nim:21-77, ops/reduce.nim:202-225) --
    with nothing but the ids read back runs as two launches, eager and under
    lazy: the first Linear with the relu in its epilogue, then the last
    Linear, the softmax and the argmax in one kernel (within its limits:
    hidden <= 1024, classes <= 64).  The ids equal the unfused kernels' (the
    same fma chains, softmax and argmax order) bit for bit, a row holding NaN
    gives INT32_MAX, and outside the limits the head falls back to the
    unfused kernels."""
    from rew_amd import jit as J
    rs = np.random.default_rng(M + K)
    x = rs.random((M, K), dtype=np.float32)
    x[5, 3] = np.nan
    w1 = rng.xavierUniformF32(rng.initKey(K), K, N1).reshape(K, N1)
    w2 = rng.xavierUniformF32(rng.initKey(N1), N1, N2).reshape(N1, N2)
    b1 = rs.normal(0, 0.1, N1).astype(np.float32)
    b2 = rs.normal(0, 0.1, N2).astype(np.float32)
    xt, l1, l2 = dev(x), nn.Linear(dev(w1), dev(b1)), nn.Linear(dev(w2), dev(b2))

    def head():
        return O.argmax(nn.softmax(l2.forward(nn.relu(l1.forward(xt))), 1), 1)

    E.profileBegin()
    ids = E.toHost(head())
    names = [n for n, _, _ in E.profileEnd()]
    lz = J.lazy(lambda a: [nn.softmax(nn.Linear(a[3], a[4]).forward(
        nn.relu(nn.Linear(a[1], a[2]).forward(a[0]))), 1)], "mlpHead")
    E.profileBegin()
    ids_lazy = E.toHost(O.argmax(lz.call([xt, l1.weight, l1.bias, l2.weight, l2.bias])[0], 1))
    names_lazy = [n for n, _, _ in E.profileEnd()]
    if fused:
        assert names == [f"gemm_f32_small+bias+relu[1,{M},{N1},{K}]",
                         f"class_head{{{M}x{N1}x{N2}}}"], names
        assert names_lazy == names, names_lazy
    else:
        assert not any(n.startswith("class_head") for n in names + names_lazy), names
    # the unfused kernels: every intermediate held, so each is materialized
    h_t = nn.relu(l1.forward(xt))
    z_t = l2.forward(h_t)
    p_t = nn.softmax(z_t, 1)
    ref = E.toHost(O.argmax(p_t, 1))
    np.testing.assert_array_equal(ids, ref)
    np.testing.assert_array_equal(ids_lazy, ref)
    assert ids[5] == np.iinfo(np.int32).max
    want = oracle.argmax_rows(E.toHost(p_t))
    np.testing.assert_array_equal(ids, want)


def test_mnist_mlp_inference(gpu, oracle):
    """Config C1: x [128,784] ~ U[0,1); Linear 784->128 + relu, Linear 128->10,
    softmax, argmax; Glorot-uniform weights (nn/init.nim:93-97), zero biases."""
    keys = rng.split(rng.initKey(0x5EED0001), 3)
    x = rng.uniformF32(keys[0], 128 * 784, 0.0, 1.0).reshape(128, 784)
    w1 = rng.xavierUniformF32(keys[1], 784, 128).reshape(784, 128)
    w2 = rng.xavierUniformF32(keys[2], 128, 10).reshape(128, 10)
    b1, b2 = np.zeros(128, np.float32), np.zeros(10, np.float32)
    l1 = nn.Linear(dev(w1), dev(b1))
    l2 = nn.Linear(dev(w2), dev(b2))
    h_t = nn.relu(l1.forward(dev(x)))
    logits_t = l2.forward(h_t)
    probs_t = nn.softmax(logits_t, 1)
    ids = E.toHost(O.argmax(probs_t, 1))
    probs, logits, hid = E.toHost(probs_t), E.toHost(logits_t), E.toHost(h_t)
    h = np.maximum(oracle.linear(x, w1, b1, False), 0)
    want_z = oracle.linear(h, w2, b2, False)
    want_p = oracle.softmax_rows(want_z)
    want_ids = oracle.argmax_rows(want_p)
    # fp32 contractions: the accumulation order is the backend's, so each
    # dot product is held to the normwise bound |d| <= 1e-5 * sum_k |a_k b_k|
    bound_h = 1e-5 * (np.abs(x) @ np.abs(w1))
    assert np.all(np.abs(hid - h) <= bound_h + 1e-30)
    bound_z = 1e-5 * (np.abs(h) @ np.abs(w2))
    assert np.all(np.abs(logits - want_z) <= bound_z + 1e-30)
    # softmax: |dp_i| <= p_i * (|dz_i| + sum_j p_j |dz_j|) <= 2 p_i max|dz|
    dz = float(np.max(np.abs(logits - want_z)))
    assert np.all(np.abs(probs - want_p) <= want_p * (2 * dz + 1e-6) + 1e-12)
    # argmax is bit-exact except at near-ties the fp32 GEMM order can flip
    srt = np.sort(want_p, axis=1)
    near_tie = (srt[:, -1] - srt[:, -2]) <= 4 * dz * srt[:, -1]
    mism = ids != want_ids
    assert not np.any(mism & ~near_tie), f"argmax differs off near-ties: rows {np.where(mism)}"
    assert np.array_equal(ids[~near_tie], want_ids[~near_tie])
