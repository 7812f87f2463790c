"""GPU parity of the eager primitives: the HIP path (through the C ABI)
against the oracle on the same seeded inputs.

Tolerances (written per test): integer, index, bitwise, layout and
IEEE-exact float ops (+ - * / max min sqrt, converts) are bit-exact;
transcendentals are <= 1e-5 relative; reductions and fp32 contractions use
a normwise bound |d| <= 1e-5 * sum|terms|; bf16 contractions <= 2e-2
relative (normwise).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import nn
from rew_amd import ops as O
from rew_amd.eager import DType


def dev(a, dt=None):
    return E.fromHost(np.asarray(a), dt)


def host(t):
    return E.toHostF32(t) if t.dtype in (DType.BFLOAT16, DType.FLOAT32) else E.toHost(t)


def rng(seed):
    return np.random.default_rng(seed)


# ---- known answers from tests/teager_dispatch.nim --------------------------------------

def test_kats(gpu):
    a = dev(np.array([1, 2, 3, 4], np.float32))
    b = dev(np.array([10, 20, 30, 40], np.float32))
    np.testing.assert_array_equal(host(O.add(a, b)), [11, 22, 33, 44])
    np.testing.assert_array_equal(host(O.mul(a, b)), [10, 40, 90, 160])
    np.testing.assert_array_equal(host(O.neg(a)), [-1, -2, -3, -4])
    e = host(O.exp(a))
    assert np.all(np.abs(e - np.exp(np.arange(1, 5, dtype=np.float32))) < 1e-5 * 60)
    lo, hi = O.scalarF32(1.5), O.scalarF32(3.5)
    np.testing.assert_array_equal(host(O.clamp(lo, a, hi)), [1.5, 2, 3, 3.5])
    np.testing.assert_array_equal(E.toHost(O.iota(DType.INT32, [2, 3], 1)),
                                  [[0, 1, 2], [0, 1, 2]])
    m1, m2 = O.reshape(a, [2, 2]), O.reshape(b, [2, 2])
    np.testing.assert_array_equal(host(O.transpose(m1, [1, 0])).ravel(), [1, 3, 2, 4])
    assert host(O.reduceSum(a, [0])).item() == 10.0
    np.testing.assert_array_equal(host(O.reduceProd(m1, [1])), [2, 12])
    np.testing.assert_array_equal(host(O.matmul(m1, m2)).ravel(), [70, 100, 150, 220])
    np.testing.assert_array_equal(host(O.dot(m1, m2)).ravel(), [70, 100, 150, 220])
    np.testing.assert_array_equal(host(O.broadcastTo(dev(np.array([5], np.float32)), [3], [0])),
                                  [5, 5, 5])
    ints = dev(np.array([1, -2, 3, 4], np.int32))
    np.testing.assert_array_equal(host(O.astype(ints, DType.FLOAT32)), [1, -2, 3, 4])
    r1, r2 = O.add(a, b), O.add(a, b)  # cache reuse (teager_dispatch.nim:536-541)
    np.testing.assert_array_equal(host(r1), host(r2))


# ---- elementwise ----------------------------------------------------------------------

EXACT_BIN = [("add", 0), ("sub", 1), ("mul", 2), ("divide", 3), ("maximum", 4), ("minimum", 5)]


@pytest.mark.parametrize("name,code", EXACT_BIN)
def test_binary_f32_exact(gpu, oracle, name, code):
    r = rng(10 + code)
    x = r.normal(size=(37, 129)).astype(np.float32)
    y = r.normal(size=(37, 129)).astype(np.float32)
    x[0, :4] = [np.nan, 0.0, -0.0, np.inf]
    y[0, :4] = [1.0, -0.0, 0.0, 2.0]
    got = host(getattr(O, name)(dev(x), dev(y)))
    want = oracle.binary(code, x, y)
    # bit patterns: also pins -0/+0 ordering of maximum/minimum
    np.testing.assert_array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("name,code", [("add", 0), ("mul", 2), ("maximum", 4)])
def test_binary_bf16(gpu, oracle, name, code):
    r = rng(20 + code)
    x = oracle.round_bf16(r.normal(size=(64, 96)).astype(np.float32))
    y = oracle.round_bf16(r.normal(size=(64, 96)).astype(np.float32))
    got = host(getattr(O, name)(dev(x, DType.BFLOAT16), dev(y, DType.BFLOAT16)))
    want = oracle.round_bf16(oracle.binary(code, x, y))
    np.testing.assert_array_equal(got, want)


@pytest.mark.parametrize("name,code,tol", [
    ("exp", 2, 1e-5), ("log", 3, 1e-5), ("sqrt", 4, 0.0), ("rsqrt", 5, 1e-5),
    ("tanh", 6, 1e-5), ("logistic", 7, 1e-5), ("neg", 0, 0.0), ("abs_", 1, 0.0)])
def test_unary_f32(gpu, oracle, name, code, tol):
    r = rng(30 + code)
    x = r.normal(size=(4099,)).astype(np.float32)
    if name in ("log", "sqrt", "rsqrt"):
        x = np.abs(x) + 1e-3
    got = host(getattr(O, name)(dev(x)))
    want = oracle.unary(code, x)
    if tol == 0.0:
        np.testing.assert_array_equal(got, want)
    else:
        np.testing.assert_allclose(got, want, rtol=tol, atol=1e-30)


def test_convert_exact(gpu, oracle):
    r = rng(40)
    x = r.normal(size=(1000,)).astype(np.float32) * 100
    x[:6] = [np.inf, -np.inf, 1.0 + 2**-8, 1.0 + 3 * 2**-8, 0.0, -0.0]
    b = O.astype(dev(x), DType.BFLOAT16)
    np.testing.assert_array_equal(E.toHost(b), oracle.to_bf16(x))
    np.testing.assert_array_equal(host(O.astype(b, DType.FLOAT32)), oracle.round_bf16(x))
    np.testing.assert_array_equal(E.toHost(O.astype(dev(x), DType.INT32)),
                                  np.trunc(np.nan_to_num(x, posinf=2**31 - 1,
                                                         neginf=-2**31)).astype(np.int64)
                                  .clip(-2**31, 2**31 - 1).astype(np.int32))
    i = r.integers(-1000, 1000, 257).astype(np.int32)
    np.testing.assert_array_equal(host(O.astype(dev(i), DType.FLOAT32)), i.astype(np.float32))
    bl = E.toHost(O.compare(dev(x), dev(np.zeros_like(x)), "GT"))
    np.testing.assert_array_equal(host(O.astype(dev(bl), DType.FLOAT32)), bl.astype(np.float32))


def test_layout_ops_exact(gpu, oracle):
    r = rng(50)
    x = r.normal(size=(2, 3, 4, 5)).astype(np.float32)
    t = dev(x)
    np.testing.assert_array_equal(host(O.transpose(t, [0, 2, 1, 3])), x.transpose(0, 2, 1, 3))
    np.testing.assert_array_equal(host(O.transpose(t, [3, 1, 0, 2])), x.transpose(3, 1, 0, 2))
    np.testing.assert_array_equal(host(O.reshape(O.transpose(t, [1, 0, 2, 3]), [6, 20])),
                                  x.transpose(1, 0, 2, 3).reshape(6, 20))
    s = dev(r.normal(size=(4, 1)).astype(np.float32))
    np.testing.assert_array_equal(host(O.broadcastTo(s, [3, 4, 5], [1, 2])),
                                  oracle.broadcast_in_dim(host(s), [3, 4, 5], [1, 2]))
    np.testing.assert_array_equal(host(O.slice_(t, [0, 1, 0, 1], [2, 3, 4, 5], [1, 1, 2, 2])),
                                  x[0:2, 1:3, 0:4:2, 1:5:2])
    y = r.normal(size=(2, 2, 4, 5)).astype(np.float32)
    np.testing.assert_array_equal(host(O.concat([t, dev(y)], 1)), np.concatenate([x, y], 1))
    z = r.normal(size=(2, 3, 4, 1)).astype(np.float32)
    np.testing.assert_array_equal(host(O.concat([t, dev(z), t], 3)),
                                  np.concatenate([x, z, x], 3))
    np.testing.assert_array_equal(E.toHost(O.iota(DType.INT32, [3, 4, 5], 2)),
                                  oracle.iota([3, 4, 5], 2))
    a, b = dev(x), dev(np.round(x))
    for d in ("LT", "LE", "GT", "GE", "EQ", "NE"):
        want = {"LT": x < np.round(x), "LE": x <= np.round(x), "GT": x > np.round(x),
                "GE": x >= np.round(x), "EQ": x == np.round(x), "NE": x != np.round(x)}[d]
        np.testing.assert_array_equal(E.toHost(O.compare(a, b, d)), want)
    p = O.compare(a, b, "GT")
    np.testing.assert_array_equal(host(O.select(p, a, b)), np.where(x > np.round(x), x,
                                                                    np.round(x)))


def test_index_select_exact(gpu, oracle):
    r = rng(60)
    w = oracle.round_bf16(r.normal(size=(1000, 64)).astype(np.float32))
    ids = r.integers(0, 1000, 300).astype(np.int32)
    got = E.toHost(O.torchIndexSelect(dev(w, DType.BFLOAT16), dev(ids), 0, 0))
    np.testing.assert_array_equal(got, oracle.to_bf16(oracle.index_select(w, ids, 0)))
    x = r.normal(size=(3, 50, 7)).astype(np.float32)
    ids2 = r.integers(0, 50, (4, 5)).astype(np.int32)
    got = host(O.torchIndexSelect(dev(x), dev(ids2), 1, 0))
    np.testing.assert_array_equal(got, oracle.index_select(x, ids2, 1))


# ---- reductions -------------------------------------------------------------------------

@pytest.mark.parametrize("shape,dims", [((64, 4096), [1]), ((8, 300), [0]), ((4, 5, 6), [0, 2]),
                                        ((3, 7), [0, 1]), ((2, 3, 130), [2]), ((1000,), [0])])
def test_reductions(gpu, oracle, shape, dims):
    r = rng(70 + len(shape))
    x = r.normal(size=shape).astype(np.float32)
    t = dev(x)
    s = host(O.reduceSum(t, dims))
    want = oracle.reduce(oracle.RSUM, x, dims)
    bound = 1e-5 * oracle.reduce(oracle.RSUM, np.abs(x), dims)
    assert np.all(np.abs(s - want) <= bound + 1e-30)
    np.testing.assert_array_equal(host(O.reduceMax(t, dims)), oracle.reduce(oracle.RMAX, x, dims))
    np.testing.assert_array_equal(host(O.reduceMin(t, dims)), oracle.reduce(oracle.RMIN, x, dims))


def test_reduce_with_fused_prologue(gpu, oracle):
    """reduceSum(mul(x, x)) and reductions over a transposed view read the
    source once; results match the op-by-op oracle."""
    r = rng(80)
    x = r.normal(size=(96, 256)).astype(np.float32)
    t = dev(x)
    got = host(O.reduceSum(O.mul(t, t), [1]))
    sq = oracle.binary(oracle.MUL, x, x)
    want = oracle.reduce(oracle.RSUM, sq, [1])
    assert np.all(np.abs(got - want) <= 1e-5 * want)
    got = host(O.reduceMax(O.transpose(t, [1, 0]), [1]))
    np.testing.assert_array_equal(got, x.max(axis=0))


# ---- contractions -----------------------------------------------------------------------

@pytest.mark.parametrize("M,K,N", [(2, 3, 4), (128, 784, 128), (128, 128, 10), (65, 257, 33)])
def test_matmul_f32(gpu, oracle, M, K, N):
    r = rng(M + K + N)
    a = r.uniform(0, 1, (M, K)).astype(np.float32)
    b = r.uniform(-0.1, 0.1, (K, N)).astype(np.float32)
    got = host(O.matmul(dev(a), dev(b)))
    want = oracle.gemm(a, b)
    bound = 1e-5 * oracle.gemm(np.abs(a), np.abs(b))
    assert np.all(np.abs(got - want) <= bound + 1e-30)


@pytest.mark.parametrize("M,K,N", [(1000, 256, 64), (33, 128, 12), (8192, 2048, 64)])
def test_matmul_f32_narrow(gpu, oracle, M, K, N):
    """f32 products of at most 64 output columns (a router's [T, H] x [H, E])
    take a 16-row-tile kernel that accumulates each output in the generic
    kernel's order. The same product with the weight stored [N, K]
    (k-contiguous, which the narrow kernel does not take) runs the generic
    kernel and must give the same bits, with and without the bias add."""
    r = rng(M + K + N + 7)
    a = r.uniform(-1, 1, (M, K)).astype(np.float32)
    b = r.uniform(-0.1, 0.1, (K, N)).astype(np.float32)
    bias = r.uniform(-1, 1, (N,)).astype(np.float32)
    bt = np.ascontiguousarray(b.T)
    for with_bias in (False, True):
        def lin(y):
            return O.add(y, O.broadcastTo(dev(bias), [M, N], [1])) if with_bias else y
        E.profileBegin()
        got = host(lin(O.matmul(dev(a), dev(b))))
        names = [n for n, _, _ in E.profileEnd()]
        assert any(n.startswith("gemm_f32_narrow") for n in names), names
        E.profileBegin()
        ref = host(lin(O.dotGeneral(dev(a), dev(bt), [], [], [1], [1])))
        names = [n for n, _, _ in E.profileEnd()]
        assert not any(n.startswith("gemm_f32_narrow") for n in names), names
        np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    want = oracle.gemm(a, b) + bias
    bound = 1e-5 * (oracle.gemm(np.abs(a), np.abs(b)) + np.abs(bias))
    assert np.all(np.abs(got - want) <= bound + 1e-30)


@pytest.mark.parametrize("M,K,N", [(128, 784, 128), (128, 128, 10), (37, 100, 70),
                                   # the one-wave 8x8 form: ragged rows, K past the
                                   # last 32-step group and short of 16, K < 32, K at
                                   # its limit
                                   (37, 100, 72), (130, 52, 20), (16, 12, 8),
                                   (72, 1024, 68)])
def test_matmul_f32_small_equals_generic(gpu, oracle, M, K, N):
    """Products with too few 64x64 tiles to fill the GPU (the MNIST MLP's)
    take 16x16 tiles, or one wave per 8x8 tile when even the 16x16 tiles
    would leave most CUs idle; each output keeps the generic kernel's fmaf
    chain, so a batch of 128 of the same product (enough tiles for the
    generic kernel) gives the same bits in every slice."""
    r = rng(M * 3 + K + N)
    a = r.uniform(-1, 1, (M, K)).astype(np.float32)
    b = r.uniform(-0.1, 0.1, (K, N)).astype(np.float32)
    E.profileBegin()
    got = host(O.matmul(dev(a), dev(b)))
    names = [n for n, _, _ in E.profileEnd()]
    assert any(n.startswith("gemm_f32_small") for n in names), names
    ab = np.broadcast_to(a, (128, M, K)).copy()
    bb = np.broadcast_to(b, (128, K, N)).copy()
    E.profileBegin()
    ref = host(O.dotGeneral(dev(ab), dev(bb), [0], [0], [2], [1]))
    names = [n for n, _, _ in E.profileEnd()]
    assert any(n.startswith("gemm_generic") for n in names), names
    for i in range(128):
        np.testing.assert_array_equal(ref[i].view(np.uint32), got.view(np.uint32))
    bound = 1e-5 * oracle.gemm(np.abs(a), np.abs(b))
    assert np.all(np.abs(got - oracle.gemm(a, b)) <= bound + 1e-30)


@pytest.mark.parametrize("first", [True, False])
def test_f32_linear_relu_epilogue(gpu, oracle, first):
    """rew's relu (maximum with a broadcast zero, nn/activation.nim:21-26)
    after an f32 Linear folds into the GEMM epilogue; values equal the
    op-by-op path bit for bit, including zero signs and both operand orders."""
    r = rng(91 + first)
    M, K, N = 128, 784, 128
    a = r.uniform(0, 1, (M, K)).astype(np.float32)
    b = r.uniform(-0.05, 0.05, (K, N)).astype(np.float32)
    bias = r.uniform(-0.05, 0.05, (N,)).astype(np.float32)
    bias[:8] = 0.0

    def fwd():
        y = nn.Linear(dev(b), dev(bias)).forward(dev(a))
        zero = O.broadcastTo(O.scalarF32(0.0), [M, N], [])
        return O.maximum(y, zero) if first else O.maximum(zero, y)

    E.profileBegin()
    got = host(fwd())
    names = [n for n, _, _ in E.profileEnd()]
    assert any(n.startswith("gemm_f32_small") and "+bias+relu" in n for n in names), names
    assert len(names) == 1, names
    E.setMode(E.MODE_OP_BY_OP)
    try:
        ref = host(fwd())
    finally:
        E.setMode(E.MODE_DEFERRED)
    np.testing.assert_array_equal(got.view(np.uint32), ref.view(np.uint32))
    want = np.maximum(oracle.gemm(a, b) + bias, 0)
    assert np.all(np.abs(got - want) <= 1e-5 * (oracle.gemm(np.abs(a), np.abs(b)) + 1) + 1e-30)


def _bf16_close(got, want, tol=2e-2):
    err = np.linalg.norm((got - want).ravel()) / max(np.linalg.norm(want.ravel()), 1e-30)
    assert err <= tol, f"normwise relative error {err:.3e} > {tol}"
    assert np.max(np.abs(got - want)) <= tol * np.max(np.abs(want)) + 1e-30


@pytest.mark.parametrize("M,K,N", [(128, 128, 128), (256, 512, 384), (100, 72, 200),
                                   (1, 64, 8), (513, 1024, 264)])
def test_matmul_bf16(gpu, oracle, M, K, N):
    r = rng(3 * M + K + N)
    a = oracle.round_bf16(r.normal(size=(M, K)).astype(np.float32))
    b = oracle.round_bf16(r.normal(0, 0.02, (K, N)).astype(np.float32))
    got = host(O.matmul(dev(a, DType.BFLOAT16), dev(b, DType.BFLOAT16)))
    want = oracle.gemm(a, b, round_bf16_out=True)
    _bf16_close(got, want)


def test_dot_general_batched_transposed_bf16(gpu, oracle):
    """Attention-shaped contractions: Q.K^T (contract last with last) and
    P.V (contract last with second-to-last), batch dims [0,1]."""
    r = rng(90)
    q = oracle.round_bf16(r.normal(size=(2, 4, 64, 128)).astype(np.float32))
    k = oracle.round_bf16(r.normal(size=(2, 4, 96, 128)).astype(np.float32))
    s = O.dotGeneral(dev(q, DType.BFLOAT16), dev(k, DType.BFLOAT16), [0, 1], [0, 1], [3], [3])
    want = oracle.dot_general(oracle.to_bf16(q), oracle.to_bf16(k), [0, 1], [0, 1], [3], [3],
                              bf16=True)
    _bf16_close(host(s), oracle.from_bf16(want))
    p = oracle.round_bf16(r.uniform(0, 1, (2, 4, 64, 96)).astype(np.float32))
    o = O.dotGeneral(dev(p, DType.BFLOAT16), dev(k, DType.BFLOAT16), [0, 1], [0, 1], [3], [2])
    want = oracle.dot_general(oracle.to_bf16(p), oracle.to_bf16(k), [0, 1], [0, 1], [3], [2],
                              bf16=True)
    _bf16_close(host(o), oracle.from_bf16(want))


def test_dot_general_permuted_f32(gpu, oracle):
    r = rng(91)
    c = r.normal(size=(4, 2, 3)).astype(np.float32)
    d = r.normal(size=(3, 4, 5)).astype(np.float32)
    got = host(O.dotGeneral(dev(c), dev(d), [], [], [0, 2], [1, 0]))
    want = oracle.dot_general(c, d, [], [], [0, 2], [1, 0])
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-5)


# ---- deferred vs op-by-op -----------------------------------------------------------------

def test_deferred_equals_op_by_op(gpu):
    """Fusing an fp32 elementwise chain changes no bits (every op still
    rounds once in fp32)."""
    from rew_amd import nn
    r = rng(100)
    x = r.normal(size=(64, 300)).astype(np.float32)
    outs = []
    for mode in (E.MODE_OP_BY_OP, E.MODE_DEFERRED):
        E.setMode(mode)
        t = dev(x)
        y = nn.silu(nn.relu(O.add(t, t)))
        outs.append(host(y))
    E.setMode(E.MODE_DEFERRED)
    np.testing.assert_array_equal(outs[0], outs[1])


def test_small_constants_share_one_upload(gpu):
    """Repeated uploads of the same small constant share one device copy
    (no H2D copy), and every handle still reads back its own value."""
    E.sync()
    E.resetStats()
    vals = [1e-5, 2.5, 1e-5, -1.0, 2.5, 1e-5]
    ts = [O.scalarF32(v) for v in vals]
    got = [float(E.toHost(t)) for t in ts]
    assert got == [float(np.float32(v)) for v in vals]
    big = np.arange(1000, dtype=np.float32)
    a, b = E.fromHost(big), E.fromHost(big)  # above the size limit: two uploads
    np.testing.assert_array_equal(E.toHost(a), E.toHost(b))
    del ts, a, b
    E.clearEagerCache()
    assert float(E.toHost(O.scalarF32(3.0))) == 3.0


def test_allocation_failure_is_an_error(gpu):
    """A device allocation the HBM cannot hold fails with ERR_OOM and a
    message naming the size; the context keeps working afterwards."""
    with pytest.raises(E.EagerError, match="device allocation of .* bytes failed"):
        E.empty(DType.FLOAT32, [1 << 40])
    t = E.empty(DType.FLOAT32, [1024])
    p = E.devicePtr(t)
    assert p and p % 256 == 0
    x = np.arange(8, dtype=np.float32)
    np.testing.assert_array_equal(host(O.add(dev(x), dev(x))), x + x)


def test_ordinal_past_visible_devices(gpu):
    """mi355x:n with n >= the visible device count is refused like rew's
    selectDevice (src/rew/eager.nim:160-172): ERR_DEVICE, naming the count."""
    import ctypes as C
    from rew_amd import _lib
    lib = _lib.load()
    ctx = C.c_void_p()
    assert lib.rew_mi355x_init(E.deviceCount(), C.byref(ctx)) == 3
    assert b"not present" in lib.rew_mi355x_last_error()


CHILD_LONE = r"""
import sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from rew_amd import _lib, eager as E, ops as O, nn
E.installEagerBackend(E.mi355x(0))
x = np.linspace(-3, 3, 4096, dtype=np.float32).reshape(64, 64)
t = E.fromHost(x)
y = E.toHost(nn.silu(O.mul(O.add(t, t), t)))   # one fused program, compiled at run time
s = E.stats()
print(str(_lib.loaded_path), s["plan_cache_hits"], float(y.sum()))
"""


def test_lone_library_compiles_fused_kernels(gpu, tmp_path):
    """A copy of librew_mi355x.so alone in a directory, found through
    REW_PJRT_PLUGIN_PATH from another working directory, compiles fused
    programs with its built-in headers (a compile failure would raise)."""
    import os
    import shutil
    import subprocess
    import sys
    from pathlib import Path
    from rew_amd import _lib
    root = Path(__file__).resolve().parents[1]
    shutil.copy(_lib.LIB_PATH, tmp_path / _lib.LIB_NAME)
    env = dict(os.environ, REW_PJRT_PLUGIN_PATH=str(tmp_path))
    env.pop("REW_MI355X_JIT", None)
    r = subprocess.run([sys.executable, "-c", CHILD_LONE, str(root)], env=env, cwd=tmp_path,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    path, _, total = r.stdout.split()
    assert path == str(tmp_path / _lib.LIB_NAME)
    x = np.linspace(-3, 3, 4096, dtype=np.float32)
    z = (x + x) * x
    want = float((z / (1 + np.exp(-z))).sum())
    assert abs(float(total) - want) <= 1e-3 * abs(want)
