"""Pins the CPU oracle (oracle/rew_oracle.c) before anything is checked
against it: known-answer tests transcribed from rew's own eager tests,
closed forms, invariants and brute force on tiny inputs.  Each check is
chosen so that a plausible slip (a dropped term, a flipped sign or index,
a transposed operand) fails it.
"""
import numpy as np
import pytest


# ---- rng: src/rew/rng.nim:39-80; tests/trng.nim ------------------------------------

def test_threefry_invariants_from_trng(oracle):
    # tests/trng.nim: distinct seeds -> distinct keys; split deterministic,
    # children pairwise distinct and distinct from the parent; foldIn.
    k0, k1, k3 = oracle.init_key(0), oracle.init_key(1), oracle.init_key(0xDEADBEEF)
    assert len({k0, k1, k3}) == 3
    a = oracle.split(oracle.init_key(42), 4)
    assert a == oracle.split(oracle.init_key(42), 4)
    kids = oracle.split(oracle.init_key(7), 8)
    assert len(set(kids)) == 8 and oracle.init_key(7) not in kids
    assert oracle.split(oracle.init_key(99), 0) == []
    k = oracle.init_key(11)
    assert oracle.fold_in(k, 5) != k and oracle.fold_in(k, 5) != oracle.fold_in(k, 6)
    assert oracle.fold_in(k, 5) == oracle.fold_in(k, 5)
    assert oracle.init_key(0xCAFEBABE12345678) == (0x12345678, 0xCAFEBABE)


def _threefry_numpy(k0, k1, c0, c1):
    """Independent vectorised statement of the 4-round Threefry-2x32 used by
    rew (rng.nim:39-55), written against numpy uint32 wraparound."""
    k0 = np.uint32(k0); k1 = np.uint32(k1)
    k2 = k0 ^ k1 ^ np.uint32(0x1BD11BDA)
    x0 = (np.asarray(c0, np.uint32) + k0).astype(np.uint32)
    x1 = (np.asarray(c1, np.uint32) + k1).astype(np.uint32)
    for r in (13, 15, 26, 6):
        x0 = (x0 + x1).astype(np.uint32)
        x1 = ((x1 << np.uint32(r)) | (x1 >> np.uint32(32 - r))).astype(np.uint32)
        x1 = x1 ^ x0
    return (x0 + k1).astype(np.uint32), (x1 + k2 + np.uint32(1)).astype(np.uint32)


def test_threefry_matches_independent_statement(oracle):
    rng = np.random.default_rng(0)
    for _ in range(20):
        k0, k1, c0, c1 = (int(v) for v in rng.integers(0, 2**32, 4, dtype=np.uint64))
        a, b = _threefry_numpy(k0, k1, c0, c1)
        assert oracle.threefry(k0, k1, c0, c1) == (int(a), int(b))


def test_uniform_and_normal_samplers(oracle):
    key = oracle.init_key(0x5EED0001)
    u = oracle.uniform_f32(key, 100000, -2.0, 3.0)
    assert u.min() >= -2.0 and u.max() < 3.0
    assert abs(u.mean() - 0.5) < 0.02
    # each uniform sample is lo + scale * (fold_in(key, i).a >> 8) / 2^24
    a, _ = _threefry_numpy(key[0], key[1], np.arange(5, dtype=np.uint32), np.zeros(5, np.uint32))
    want = np.float32(-2.0) + np.float32(5.0) * ((a >> 8).astype(np.float32) / np.float32(2**24))
    np.testing.assert_array_equal(u[:5], want.astype(np.float32))
    # Box-Muller on (fold_in(2i).a, fold_in(2i+1).a), restated in float64.
    # (rew's 4-round Threefry correlates adjacent counters, so these samples
    # are visibly biased -- mean ~0.1 for N(0,1); that is the reference's
    # generator, reproduced as is.)
    n = 20001
    z = oracle.normal_f32(key, n, 1.0, 0.5)
    i = np.arange((n + 1) // 2, dtype=np.uint64)
    c1, c2 = (2 * i).astype(np.uint32), (2 * i + 1).astype(np.uint32)
    a1, _ = _threefry_numpy(key[0], key[1], c1, np.zeros_like(c1))
    a2, _ = _threefry_numpy(key[0], key[1], c2, np.zeros_like(c2))
    u1 = np.maximum((a1 >> 8) / 2.0**24, 1e-10)
    u2 = (a2 >> 8) / 2.0**24
    r = np.sqrt(-2 * np.log(u1))
    want = np.empty(2 * len(i))
    want[0::2] = 1.0 + 0.5 * r * np.cos(2 * np.pi * u2)
    want[1::2] = 1.0 + 0.5 * r * np.sin(2 * np.pi * u2)
    np.testing.assert_allclose(z, want[:n], rtol=2e-5, atol=2e-5)
    # odd counts keep the first element of the last pair
    z2 = oracle.normal_f32(key, n - 1, 1.0, 0.5)
    np.testing.assert_array_equal(z[: n - 1], z2)


# ---- bf16 ---------------------------------------------------------------------------

def test_bf16_rounding_is_rne(oracle):
    # 1 + 2^-8 is exactly half an ulp above 1 in bf16: ties to even -> 1.0
    x = np.array([1.0 + 2**-8, 1.0 + 3 * 2**-8, 1.0 + 2**-8 + 2**-20, -1.5, 65504.0],
                 np.float32)
    got = oracle.from_bf16(oracle.to_bf16(x))
    np.testing.assert_array_equal(got, np.array([1.0, 1.0 + 2**-6, 1.0 + 2**-7, -1.5, 65536.0],
                                                np.float32))
    nan = oracle.to_bf16(np.array([np.nan], np.float32))
    assert np.isnan(oracle.from_bf16(nan))[0]


# ---- elementwise / reductions / contractions: tests/teager_dispatch.nim KATs -------------

A = np.array([1, 2, 3, 4], np.float32)
B = np.array([10, 20, 30, 40], np.float32)


def test_kat_elementwise(oracle):
    np.testing.assert_array_equal(oracle.binary(oracle.ADD, A, B), [11, 22, 33, 44])
    np.testing.assert_array_equal(oracle.binary(oracle.MUL, A, B), [10, 40, 90, 160])
    np.testing.assert_array_equal(oracle.unary(oracle.NEG, A), [-1, -2, -3, -4])
    e = oracle.unary(oracle.EXP, A)
    assert np.all(np.abs(e - np.exp(A.astype(np.float64))) < 1e-5 * np.exp(4.0))
    mx = oracle.binary(oracle.MAX, np.array([np.nan, 1, -0.0], np.float32),
                       np.array([1, np.nan, 0.0], np.float32))
    assert np.isnan(mx[0]) and np.isnan(mx[1]) and not np.signbit(mx[2])


def test_kat_reductions(oracle):
    assert oracle.reduce(oracle.RSUM, A, [0]).item() == 10.0
    np.testing.assert_array_equal(oracle.reduce(oracle.RPROD, A.reshape(2, 2), [1]), [2, 12])
    x = np.arange(24, dtype=np.float32).reshape(2, 3, 4)
    np.testing.assert_array_equal(oracle.reduce(oracle.RSUM, x, [0, 2]), x.sum(axis=(0, 2)))
    np.testing.assert_array_equal(oracle.reduce(oracle.RMAX, x, [1]), x.max(axis=1))
    np.testing.assert_array_equal(oracle.reduce(oracle.RMIN, x, [2, 0]), x.min(axis=(0, 2)))


def test_kat_matmul_and_dot_general(oracle):
    m1, m2 = A.reshape(2, 2), B.reshape(2, 2)
    np.testing.assert_array_equal(oracle.dot_general(m1, m2, [], [], [1], [0]).ravel(),
                                  [70, 100, 150, 220])
    rng = np.random.default_rng(1)
    # integer-valued inputs make every sum exact: compare against numpy
    a = rng.integers(-4, 5, (3, 5, 7)).astype(np.float32)
    b = rng.integers(-4, 5, (3, 7, 6)).astype(np.float32)
    np.testing.assert_array_equal(oracle.dot_general(a, b, [0], [0], [2], [1]),
                                  np.einsum("bmk,bkn->bmn", a, b))
    # transposed operands and permuted contracting dims
    bt = np.ascontiguousarray(b.transpose(2, 0, 1))  # [6,3,7]
    np.testing.assert_array_equal(oracle.dot_general(a, bt, [0], [1], [2], [2]),
                                  np.einsum("bmk,nbk->bmn", a, bt))
    c = rng.integers(-3, 4, (4, 2, 3)).astype(np.float32)
    d = rng.integers(-3, 4, (3, 4, 5)).astype(np.float32)
    np.testing.assert_array_equal(oracle.dot_general(c, d, [], [], [0, 2], [1, 0]),
                                  np.einsum("kmj,jkn->mn", c, d))
    np.testing.assert_array_equal(oracle.gemm(a[0], b[0]), a[0] @ b[0])


def test_bf16_dot_rounds_result(oracle):
    a = np.array([[1.0, 2.0 ** -9]], np.float32)
    b = np.array([[1.0], [1.0]], np.float32)
    out = oracle.dot_general(oracle.to_bf16(a), oracle.to_bf16(b), [], [], [1], [0], bf16=True)
    # 1 + 2^-9 rounds to 1 in bf16
    assert oracle.from_bf16(out).item() == 1.0


# ---- composites: invariants and closed forms ------------------------------------------------

def test_softmax_invariants(oracle):
    rng = np.random.default_rng(2)
    x = rng.normal(size=(64, 100)).astype(np.float32) * 5
    p = oracle.softmax_rows(x)
    np.testing.assert_allclose(p.sum(-1), 1.0, rtol=1e-6)
    # shift invariance and ordering
    np.testing.assert_allclose(oracle.softmax_rows(x + 3.0), p, rtol=1e-5, atol=1e-7)
    assert np.all(np.argsort(p, -1) == np.argsort(x, -1))
    np.testing.assert_allclose(oracle.softmax_rows(np.zeros((2, 8), np.float32)), 1 / 8)


def test_rmsnorm_closed_form(oracle):
    g = np.array([1.0, 2.0, -1.0, 0.5], np.float32)
    x = np.full((3, 4), 2.0, np.float32)
    want = g * (2.0 / np.sqrt(np.float32(4.0 + 1e-5)))
    np.testing.assert_allclose(oracle.rmsnorm_rows(x, g), np.broadcast_to(want, (3, 4)),
                               rtol=1e-6)
    rng = np.random.default_rng(3)
    y = rng.normal(size=(16, 64)).astype(np.float32)
    out = oracle.rmsnorm_rows(y, np.ones(64, np.float32), eps=0.0)
    np.testing.assert_allclose(np.sqrt((out.astype(np.float64) ** 2).mean(-1)), 1.0, rtol=1e-5)


def test_layernorm_moments(oracle):
    rng = np.random.default_rng(4)
    x = rng.normal(3.0, 2.0, size=(32, 128)).astype(np.float32)
    out = oracle.layernorm_rows(x, np.ones(128, np.float32), np.zeros(128, np.float32), 0.0)
    np.testing.assert_allclose(out.mean(-1), 0.0, atol=1e-5)
    np.testing.assert_allclose(out.var(-1), 1.0, rtol=1e-4)


def test_layernorm_affine_float64(oracle):
    """LayerNorm with a non-trivial scale and shift (norm.nim:41-84:
    gamma * ((x - mean) * rsqrt(var + eps)) + beta) against a float64
    statement; a swapped gamma / beta, a dropped eps or the variance taken
    around 0 instead of the mean all fail it."""
    rng = np.random.default_rng(11)
    x = rng.normal(1.5, 2.0, size=(64, 300)).astype(np.float32)
    g = rng.normal(1.0, 0.3, size=300).astype(np.float32)
    b = rng.normal(0.0, 0.5, size=300).astype(np.float32)
    eps = 0.25  # large, so that dropping it shows
    out = oracle.layernorm_rows(x, g, b, eps)
    xd = x.astype(np.float64)
    m = xd.mean(-1, keepdims=True)
    v = ((xd - m) ** 2).mean(-1, keepdims=True)
    want = g * ((xd - m) / np.sqrt(v + eps)) + b
    np.testing.assert_allclose(out, want, rtol=1e-5, atol=1e-5)
    assert not np.allclose(oracle.layernorm_rows(x, b, g, eps), want, atol=1e-3)
    assert not np.allclose(oracle.layernorm_rows(x, g, b, 0.0), want, atol=1e-3)


def test_rope_properties(oracle):
    c, s = oracle.rope_tables(8, 16, 10000.0)
    np.testing.assert_allclose(c * c + s * s, 1.0, rtol=1e-6)
    np.testing.assert_array_equal(c[0], 1.0)
    np.testing.assert_array_equal(s[0], 0.0)
    # pair i at position p rotates by p * theta^(-2i/d)
    assert abs(c[3, 2] - np.cos(3 * 10000.0 ** (-2 / 8))) < 1e-6
    assert abs(s[3, 2] - np.sin(3 * 10000.0 ** (-2 / 8))) < 1e-6
    rng = np.random.default_rng(5)
    x = rng.normal(size=(2, 16, 8)).astype(np.float32)
    y = oracle.rope(x, c, s)
    np.testing.assert_array_equal(y[:, 0], x[:, 0])  # position 0 is the identity
    nx = x[..., 0::2] ** 2 + x[..., 1::2] ** 2
    ny = y[..., 0::2] ** 2 + y[..., 1::2] ** 2
    np.testing.assert_allclose(ny, nx, rtol=1e-5)
    # adjacent-pair rotation direction: (1, 0) -> (cos, sin)
    e = np.zeros((1, 16, 8), np.float32)
    e[..., 0] = 1.0
    r = oracle.rope(e, c, s)
    np.testing.assert_allclose(r[0, 5, :2], [c[5, 0], s[5, 0]], rtol=1e-6)


def test_sdpa_properties(oracle):
    rng = np.random.default_rng(6)
    B, H, Hkv, S, D = 1, 4, 2, 8, 16
    q = rng.normal(size=(B, H, S, D)).astype(np.float32)
    k = rng.normal(size=(B, Hkv, S, D)).astype(np.float32)
    v = rng.normal(size=(B, Hkv, S, D)).astype(np.float32)
    out = oracle.sdpa(q, k, v, causal=False)
    # GQA equals MHA with K/V heads repeated (kv head = h // (H/Hkv))
    rep = lambda t: np.repeat(t, H // Hkv, axis=1)
    np.testing.assert_allclose(out, oracle.sdpa(q, rep(k), rep(v), causal=False), rtol=1e-6)
    # all-equal keys -> uniform attention -> mean of V
    kc = np.broadcast_to(k[:, :, :1], k.shape).copy()
    np.testing.assert_allclose(oracle.sdpa(q, kc, v, causal=False),
                               np.broadcast_to(rep(v).mean(2, keepdims=True), out.shape),
                               rtol=1e-5, atol=1e-6)
    # rew's causal mask keeps keys j >= i: the last query sees only the last key
    oc = oracle.sdpa(q, k, v, causal=True)
    np.testing.assert_allclose(oc[:, :, -1], rep(v)[:, :, -1], rtol=1e-6)
    # and perturbing key 0 changes only query row 0
    k2 = k.copy()
    k2[:, :, 0] += 1.0
    oc2 = oracle.sdpa(q, k2, v, causal=True)
    np.testing.assert_array_equal(oc2[:, :, 1:], oc[:, :, 1:])
    assert not np.allclose(oc2[:, :, 0], oc[:, :, 0])
    # brute force against float64 on the plain formula
    sc = 1 / np.sqrt(D)
    s64 = np.einsum("bhid,bhjd->bhij", q.astype(np.float64), rep(k).astype(np.float64)) * sc
    p = np.exp(s64 - s64.max(-1, keepdims=True))
    p /= p.sum(-1, keepdims=True)
    np.testing.assert_allclose(out, np.einsum("bhij,bhjd->bhid", p, rep(v)), rtol=1e-4,
                               atol=1e-5)


def test_argmax_and_topk(oracle):
    x = np.array([[1, 3, 3, 2], [np.nan, 1, 2, 3], [-1, -1, -1, -1]], np.float32)
    np.testing.assert_array_equal(oracle.argmax_rows(x), [1, 2147483647, 0])
    v, i = oracle.topk_rows(np.array([[0.1, 0.5, 0.5, 0.2, 0.9]], np.float32), 3)
    np.testing.assert_array_equal(i, [[4, 1, 2]])
    np.testing.assert_array_equal(v, np.array([[0.9, 0.5, 0.5]], np.float32))
    rng = np.random.default_rng(7)
    y = rng.normal(size=(50, 64)).astype(np.float32)
    v, i = oracle.topk_rows(y, 6)
    np.testing.assert_array_equal(i, np.argsort(-y, axis=-1, kind="stable")[:, :6])
