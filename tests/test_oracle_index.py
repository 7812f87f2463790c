"""Pins of the oracle's gather / scatter / sort restatements
(oracle/oracle.py) against independent numpy routines: np.take,
fancy indexing, np.take_along_axis, np.add.at / np.maximum.at /
np.minimum.at, explicit slicing, and Python's stable sorted()."""
import numpy as np
import pytest


def test_gather_as_index_select(oracle):
    rs = np.random.default_rng(1)
    x = rs.standard_normal((6, 5)).astype(np.float32)
    idx = np.array([3, 0, 5, 5, 1, -2, 9], np.int32)   # out-of-range starts clamp
    got = oracle.gather(x, idx[:, None], offset_dims=[1], collapsed=[0], start_index_map=[0],
                        ivd=1, slice_sizes=[1, 5])
    np.testing.assert_array_equal(got, np.take(x, np.clip(idx, 0, 5), axis=0))
    # index_vector_dim == rank: scalar indices
    got2 = oracle.gather(x, idx, offset_dims=[1], collapsed=[0], start_index_map=[0], ivd=1,
                         slice_sizes=[1, 5])
    np.testing.assert_array_equal(got2, got)


def test_gather_points_and_windows(oracle):
    rs = np.random.default_rng(2)
    x = rs.standard_normal((5, 7)).astype(np.float32)
    pts = np.array([[0, 0], [4, 6], [2, 3], [1, 5]], np.int32)
    got = oracle.gather(x, pts, offset_dims=[], collapsed=[0, 1], start_index_map=[0, 1],
                        ivd=1, slice_sizes=[1, 1])
    np.testing.assert_array_equal(got, x[pts[:, 0], pts[:, 1]])
    # 2x3 windows, starts clamped so the window stays inside
    win = oracle.gather(x, pts, offset_dims=[1, 2], collapsed=[], start_index_map=[0, 1],
                        ivd=1, slice_sizes=[2, 3])
    for i, (r, c) in enumerate(pts):
        r, c = min(r, 5 - 2), min(c, 7 - 3)
        np.testing.assert_array_equal(win[i], x[r:r + 2, c:c + 3])


def test_gather_with_batching_dims(oracle):
    rs = np.random.default_rng(3)
    x = rs.standard_normal((3, 6, 4)).astype(np.float32)
    idx = rs.integers(0, 6, size=(3, 5)).astype(np.int32)
    got = oracle.gather(x, idx, offset_dims=[2], collapsed=[1], start_index_map=[1], ivd=2,
                        slice_sizes=[1, 1, 4], operand_batching=[0], start_batching=[0])
    np.testing.assert_array_equal(got, np.take_along_axis(x, idx[:, :, None], axis=1))


@pytest.mark.parametrize("op,ref", [("add", np.add), ("maximum", np.maximum),
                                    ("minimum", np.minimum)])
def test_scatter_matches_ufunc_at(oracle, op, ref):
    rs = np.random.default_rng(4)
    x = rs.integers(-5, 5, size=(6, 3)).astype(np.float32)
    idx = np.array([1, 4, 1, 0, 4, 4], np.int32)       # duplicates
    upd = rs.integers(-5, 5, size=(6, 3)).astype(np.float32)
    got = oracle.scatter(x, idx[:, None], upd, update_window_dims=[1], inserted=[0],
                         scatter_dims_to_operand=[0], ivd=1, op=op)
    want = x.copy()
    ref.at(want, idx, upd)
    np.testing.assert_array_equal(got, want)


def test_scatter_replace_and_out_of_bounds_skip(oracle):
    x = np.zeros((4, 2), np.float32)
    idx = np.array([2, 7, -1, 0], np.int32)             # 7 and -1 fall outside: skipped
    upd = np.arange(8, dtype=np.float32).reshape(4, 2) + 1
    got = oracle.scatter(x, idx[:, None], upd, update_window_dims=[1], inserted=[0],
                         scatter_dims_to_operand=[0], ivd=1, op="replace")
    want = np.zeros((4, 2), np.float32)
    want[2], want[0] = upd[0], upd[3]
    np.testing.assert_array_equal(got, want)


def test_sort_order_is_stable_nan_last(oracle):
    x = np.array([2.0, np.nan, -0.0, 1.0, 0.0, 2.0, -3.0, np.nan], np.float32)
    for desc in (False, True):
        got = oracle.sort_order(x, 0, desc)
        key = [(1, 0.0) if np.isnan(v) else (0, (-1 if desc else 1) * float(v) + 0.0)
               for v in x]
        want = sorted(range(len(x)), key=lambda i: key[i])
        assert list(got) == want


# ---- pad / dynamicSlice / dynamicUpdateSlice / cholesky --------------------------------

def test_pad_known_answer(oracle):
    """tests/teager_dispatch.nim:477-483: a 2x2 padded by one on every edge."""
    x = np.array([[4, 2], [2, 3]], np.float32)
    got = oracle.pad(x, 0.0, [1, 1], [1, 1], [0, 0])
    np.testing.assert_array_equal(got.ravel(), [0, 0, 0, 0, 0, 4, 2, 0, 0, 2, 3, 0, 0, 0, 0, 0])


def test_pad_against_numpy(oracle):
    """Non-negative edges without interior padding are np.pad with a constant;
    interior padding is the zero-stuffed array (x placed at every
    (interior + 1)-th position) padded the same way; negative edges crop the
    padded array."""
    rs = np.random.default_rng(5)
    x = rs.integers(-50, 50, (3, 4, 2)).astype(np.int32)
    lo, hi = [1, 0, 2], [0, 3, 1]
    np.testing.assert_array_equal(oracle.pad(x, -7, lo, hi, [0, 0, 0]),
                                  np.pad(x, list(zip(lo, hi)), constant_values=-7))
    it = [2, 0, 1]
    stuffed = np.full([d + (d - 1) * i for d, i in zip(x.shape, it)], -7, np.int32)
    stuffed[::3, :, ::2] = x
    np.testing.assert_array_equal(oracle.pad(x, -7, lo, hi, it),
                                  np.pad(stuffed, list(zip(lo, hi)), constant_values=-7))
    full = oracle.pad(x, -7, [2, 2, 2], [2, 2, 2], it)
    np.testing.assert_array_equal(oracle.pad(x, -7, [-1, 2, 0], [2, -2, -1], it),
                                  full[3:, :-4, 2:-3])


def test_dynamic_slice_and_update_known_answers(oracle):
    """tests/teager_dispatch.nim:496-503, and the StableHLO spec examples of
    clamped starts (start (-1, 3) on a 4x4 operand)."""
    a = np.array([[1, 2], [3, 4]], np.float32)
    np.testing.assert_array_equal(oracle.dynamic_slice(a, [0, 1], [2, 1]).ravel(), [2, 4])
    np.testing.assert_array_equal(
        oracle.dynamic_update_slice(a, np.array([[9]], np.float32), [0, 1]).ravel(), [1, 9, 3, 4])
    op = np.array([[0, 0, 1, 1], [0, 0, 1, 1], [0, 0, 0, 0], [0, 0, 0, 0]], np.int64)
    np.testing.assert_array_equal(oracle.dynamic_slice(op, [-1, 3], [2, 2]), [[1, 1], [1, 1]])
    op2 = np.array([[1, 1, 0, 0], [1, 1, 0, 0], [1, 1, 1, 1], [1, 1, 1, 1]], np.int64)
    np.testing.assert_array_equal(
        oracle.dynamic_update_slice(op2, np.ones((2, 2), np.int64), [-1, 3]), np.ones((4, 4)))


def test_cholesky_pins(oracle):
    """tests/teager_dispatch.nim:466-470 ([[4,2],[2,3]] -> [2,0,1,sqrt 2]),
    np.linalg.cholesky on random SPD batches, the upper form as the
    transpose, and L L^T == A."""
    got = oracle.cholesky(np.array([[4, 2], [2, 3]], np.float32))
    np.testing.assert_allclose(got.ravel(), [2, 0, 1, np.sqrt(2)], rtol=1e-15)
    rs = np.random.default_rng(9)
    m = rs.standard_normal((3, 7, 7))
    spd = m @ m.transpose(0, 2, 1) + 7 * np.eye(7)
    L = oracle.cholesky(spd, True)
    np.testing.assert_allclose(L, np.linalg.cholesky(spd), rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(L @ L.transpose(0, 2, 1), spd, rtol=1e-12)
    np.testing.assert_allclose(oracle.cholesky(spd, False), L.transpose(0, 2, 1), rtol=1e-12)
    # only the referenced triangle is read
    junk = spd + np.triu(np.full((7, 7), 1e3), 1)
    np.testing.assert_allclose(oracle.cholesky(junk, True), L, rtol=1e-12)


def test_batch_norm_pins(oracle):
    """tests/teager_dispatch.nim:426-463 known answers; training output with unit
    scale and zero offset has per-feature mean 0 and variance var / (var + eps);
    the grad equals central finite differences of sum(dy * training output)
    (mean and variance recomputed from the perturbed input)."""
    a = np.array([1, 2, 3, 4], np.float64)
    one, zero = np.ones(4), np.zeros(4)
    np.testing.assert_array_equal(oracle.batch_norm_inference(a, one, zero, one, one, 0.0, 0),
                                  [0, 1, 2, 3])
    y, m, v = oracle.batch_norm_training(a.reshape(2, 2), np.ones(2), np.zeros(2), 0.0, 1)
    np.testing.assert_allclose(y.ravel(), [-1, -1, 1, 1])
    np.testing.assert_array_equal(m, [2, 3])
    np.testing.assert_array_equal(v, [1, 1])
    dx, ds, do = oracle.batch_norm_grad(a.reshape(2, 2), np.ones(2), np.array([2., 3.]),
                                        np.ones(2), np.full((2, 2), 0.1), 0.0, 1)
    np.testing.assert_allclose(dx.ravel(), 0, atol=1e-15)
    np.testing.assert_allclose(ds, 0, atol=1e-15)
    np.testing.assert_allclose(do, [0.2, 0.2])
    rs = np.random.default_rng(21)
    x = rs.standard_normal((3, 4, 5))
    eps = 1e-3
    y, m, v = oracle.batch_norm_training(x, np.ones(4), np.zeros(4), eps, 1)
    np.testing.assert_allclose(y.mean(axis=(0, 2)), 0, atol=1e-12)
    np.testing.assert_allclose(y.var(axis=(0, 2)), v / (v + eps), rtol=1e-12)
    sc, of, dy = rs.standard_normal(4), rs.standard_normal(4), rs.standard_normal(x.shape)
    _, m, v = oracle.batch_norm_training(x, sc, of, eps, 1)
    dx, dsc, doff = oracle.batch_norm_grad(x, sc, m, v, dy, eps, 1)
    loss = lambda z: float((dy * oracle.batch_norm_training(z, sc, of, eps, 1)[0]).sum())
    h, num = 1e-6, np.zeros_like(x)
    for i in np.ndindex(*x.shape):
        e = np.zeros_like(x)
        e[i] = h
        num[i] = (loss(x + e) - loss(x - e)) / (2 * h)
    np.testing.assert_allclose(dx, num, rtol=1e-5, atol=1e-7)
    xn = (x - m[None, :, None]) / np.sqrt(v[None, :, None] + eps)
    np.testing.assert_allclose(dsc, (dy * xn).sum(axis=(0, 2)), rtol=1e-12)
    np.testing.assert_allclose(doff, dy.sum(axis=(0, 2)), rtol=1e-12)
