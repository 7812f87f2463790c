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
