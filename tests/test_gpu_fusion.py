"""GPU parity of the GEMM epilogue fusions.

rew's Linear.forward bias add (src/rew/nn/linear.nim:43-49), the decoder's
residual add (src/rew/models/llama.nim:106-117) and GatedFeedForward's SiLU
gate (src/rew/nn/gated_ffn.nim:46-67, activation.nim:28-38) are recognised in
the deferred graph and run inside the GEMM.  The fused epilogue repeats the
op sequence's roundings, so it is compared BIT-EXACTLY with the unfused GPU
path (op-by-op mode: the same GEMM kernels, then the elementwise ops), and
with the oracle within the bf16 tolerance (normwise 2e-2).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import nn
from rew_amd import ops as O
from rew_amd.eager import DType


def bf16_close(got, want, tol=2e-2):
    err = np.linalg.norm((got - want).ravel()) / max(np.linalg.norm(want.ravel()), 1e-30)
    assert err <= tol, f"normwise relative error {err:.3e} > {tol}"


def _run(fn, op_by_op=False):
    if op_by_op:
        E.setMode(E.MODE_OP_BY_OP)
    try:
        E.profileBegin()
        out = E.toHost(fn())
        names = [n for n, _, _ in E.profileEnd()]
    finally:
        E.setMode(E.MODE_DEFERRED)
    return out, names


def _lin(oracle, key, fi, fo, bias_sd=0.5):
    w = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 0), fi * fo, 0.0, 0.05)
                          .reshape(fi, fo))
    b = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 1), fo, 0.0, bias_sd))
    return w, b


def _bits_f32(u16):
    return E.bf16_bits_to_f32(u16)


@pytest.mark.parametrize("T,fi,fo", [(300, 256, 520), (1024, 512, 1024), (64, 128, 72)])
def test_linear_bias_epilogue(gpu, oracle, T, fi, fo):
    key = oracle.init_key(100 + T)
    w, b = _lin(oracle, key, fi, fo)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 2), T * fi).reshape(T, fi))

    def fn():
        lin = nn.Linear(E.fromHost(w, DType.BFLOAT16), E.fromHost(b, DType.BFLOAT16))
        return lin.forward(E.fromHost(x, DType.BFLOAT16))

    got, names = _run(fn)
    assert any("+bias" in n for n in names), names
    ref, names2 = _run(fn, op_by_op=True)
    assert not any("+bias" in n for n in names2)
    np.testing.assert_array_equal(got, ref)
    want = oracle.linear(x, w, b, True)
    bf16_close(_bits_f32(got), want)


@pytest.mark.parametrize("B,S,H", [(2, 160, 256), (1, 512, 512)])
def test_residual_epilogue(gpu, oracle, B, S, H):
    key = oracle.init_key(200 + S)
    w, b = _lin(oracle, key, H, H)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 2), B * S * H).reshape(B, S, H))
    r = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 3), B * S * H).reshape(B, S, H))

    def fn():
        lin = nn.Linear(E.fromHost(w, DType.BFLOAT16), E.fromHost(b, DType.BFLOAT16))
        y = lin.forward(O.reshape(E.fromHost(x, DType.BFLOAT16), [B * S, H]))
        return O.add(E.fromHost(r, DType.BFLOAT16), O.reshape(y, [B, S, H]))

    got, names = _run(fn)
    assert any("+bias+res" in n for n in names), names
    ref, _ = _run(fn, op_by_op=True)
    np.testing.assert_array_equal(got, ref)
    want = oracle.round_bf16(r + oracle.linear(x.reshape(B * S, H), w, b, True).reshape(B, S, H))
    bf16_close(_bits_f32(got), want)


def far_apart(mats):
    """bf16 matrices of one shape placed more than 2 GiB apart inside one
    allocation: matrix i is rows R i .. R i + r of `big` [R k + r, c].
    Returns (big, R, view) with view(i) that matrix as a slice; a slice
    stays a view only while the caller does not hold it at the flush, so
    make it inside the function that is flushed."""
    r, c = mats[0].shape
    R = (1 << 31) // (c * 2) + 64
    big = O.zeros([R * (len(mats) - 1) + r, c], DType.BFLOAT16)
    for i, m in enumerate(mats):
        big = O.dynamicUpdateSlice(big, E.fromHost(m, DType.BFLOAT16),
                                   [O.scalarI32(R * i), O.scalarI32(0)])
    E.flush()
    return big, R, lambda i: O.slice_(big, [R * i, 0], [R * i + r, c])


def test_swiglu_gate_and_up_far_apart(gpu, oracle):
    """The dual SwiGLU kernel addresses both weight matrices through one
    buffer descriptor when they lie within 2 GiB of each other; allocations
    need not, and with the up weight 2 GiB past the gate weight it takes a
    descriptor per matrix.  Same bits as op by op."""
    T, E_, I = 2048, 512, 1536  # 8 x 12 dual tiles: the LDS kernel
    key = oracle.init_key(777)
    wg, bg = _lin(oracle, oracle.fold_in(key, 0), E_, I, 0.3)
    wu, bu = _lin(oracle, oracle.fold_in(key, 1), E_, I, 0.3)
    wd, bd = _lin(oracle, oracle.fold_in(key, 2), I, E_, 0.3)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 3), T * E_).reshape(1, T, E_))
    _, _, view = far_apart([wg, wu])

    def fn():
        mk = lambda w, b: nn.Linear(w, E.fromHost(b, DType.BFLOAT16))
        ffn = nn.GatedFeedForward(mk(view(0), bg), mk(view(1), bu),
                                  mk(E.fromHost(wd, DType.BFLOAT16), bd))
        return ffn.forward(E.fromHost(x, DType.BFLOAT16))

    got, names = _run(fn)
    assert any(n.startswith("gemm_lds_swiglu") for n in names), names
    ref, _ = _run(fn, op_by_op=True)
    np.testing.assert_array_equal(got, ref)
    want = oracle.gated_ffn(x.reshape(T, E_), wg, bg, wu, bu, wd, bd, True).reshape(1, T, E_)
    bf16_close(_bits_f32(got), want)


@pytest.mark.parametrize("T,E_,I", [(256, 256, 512), (300, 128, 264), (1024, 512, 1408)])
def test_swiglu_dual_gemm(gpu, oracle, T, E_, I):
    key = oracle.init_key(300 + I)
    wg, bg = _lin(oracle, oracle.fold_in(key, 0), E_, I, 0.3)
    wu, bu = _lin(oracle, oracle.fold_in(key, 1), E_, I, 0.3)
    wd, bd = _lin(oracle, oracle.fold_in(key, 2), I, E_, 0.3)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 3), T * E_).reshape(1, T, E_))

    def fn():
        mk = lambda w, b: nn.Linear(E.fromHost(w, DType.BFLOAT16), E.fromHost(b, DType.BFLOAT16))
        ffn = nn.GatedFeedForward(mk(wg, bg), mk(wu, bu), mk(wd, bd))
        return ffn.forward(E.fromHost(x, DType.BFLOAT16))

    got, names = _run(fn)
    assert any("swiglu" in n for n in names), names
    ref, names2 = _run(fn, op_by_op=True)
    assert not any("swiglu" in n for n in names2)
    np.testing.assert_array_equal(got, ref)
    want = oracle.gated_ffn(x.reshape(T, E_), wg, bg, wu, bu, wd, bd, True).reshape(1, T, E_)
    bf16_close(_bits_f32(got), want)


def test_held_intermediate_blocks_fusion(gpu, oracle):
    """A matmul result the caller still holds is materialized as is, and the
    bias add then runs on it: same values as the fused path."""
    T, fi, fo = 256, 256, 256
    key = oracle.init_key(400)
    w, b = _lin(oracle, key, fi, fo)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 2), T * fi).reshape(T, fi))
    xt, wt, bt = (E.fromHost(x, DType.BFLOAT16), E.fromHost(w, DType.BFLOAT16),
                  E.fromHost(b, DType.BFLOAT16))
    E.profileBegin()
    xw = O.matmul(xt, wt)
    y = O.add(xw, O.broadcastTo(bt, xw.shape, [1]))
    got = E.toHost(y)
    names = [n for n, _, _ in E.profileEnd()]
    assert not any("+bias" in n for n in names), names
    fused = E.toHost(nn.Linear(wt, bt).forward(xt))
    np.testing.assert_array_equal(got, fused)
    bf16_close(_bits_f32(E.toHost(xw)), oracle.gemm(x, w, True))


# ---- row composites ---------------------------------------------------------------------

@pytest.mark.parametrize("shape,bf16", [((2, 100, 4096), True), ((37, 1000), False),
                                        ((3, 9000), True), ((4100, 4096), True),
                                        ((2500, 1024), False), ((300, 4096), False),
                                        ((65, 2048), False)])
def test_rmsnorm_row_kernel(gpu, oracle, shape, bf16):
    """rew's rmsNorm chain (src/rew/nn/norm.nim:204-224) runs as one row kernel.
    Whole rows of 2, 4 or 8 chunks per lane take the pipelined kernel; more
    rows than its 2048 waves give waves of two and three rows."""
    key = oracle.init_key(500 + shape[-1])
    n = shape[-1]
    x = oracle.normal_f32(oracle.fold_in(key, 0), int(np.prod(shape))).reshape(shape)
    if bf16:
        x = oracle.round_bf16(x)
    g = oracle.normal_f32(oracle.fold_in(key, 1), n, 1.0, 0.1)

    def fn():
        xt = E.fromHost(x, DType.BFLOAT16 if bf16 else DType.FLOAT32)
        y = nn.rmsNorm(nn._f32(xt), E.fromHost(g), 1e-5)
        return nn._to(y, DType.BFLOAT16) if bf16 else y

    got, names = _run(fn)
    assert any(k.startswith("rmsnorm_rows") for k in names), names
    want = oracle.rmsnorm_rows(x.reshape(-1, n), g, 1e-5).reshape(shape)
    if bf16:
        got = _bits_f32(got)
        # within one bf16 ulp of the fp32 reference
        assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-30)
    else:
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


LN_SHAPES = [((2, 100, 4096), True), ((37, 1000), False), ((3, 9000), True),
             ((4100, 4096), True), ((2500, 1024), False), ((300, 4096), False),
             ((65, 2048), False), ((9, 7), True)]


@pytest.mark.parametrize("shape,bf16", LN_SHAPES)
def test_layernorm_row_kernel(gpu, oracle, shape, bf16):
    """rew's LayerNorm chain (src/rew/nn/norm.nim:41-84; reduceMean as
    reduceSum / n, reduce.nim:132-150) runs as one row kernel: a workgroup per
    row for rows of 256, 512 or 1024 16-byte chunks, the general kernel
    otherwise.  Checked against the oracle componentwise, relative to the
    magnitudes the op sequence rounds on the way: |gamma| (|x| + mean |x|)
    rsqrt(var + eps) + |beta| (the centring x - mean carries the mean's
    absolute error whatever the summation order, and the row sums run in
    another order than the op sequence's reductions)."""
    key = oracle.init_key(900 + shape[-1])
    n = shape[-1]
    x = oracle.normal_f32(oracle.fold_in(key, 0), int(np.prod(shape)), 0.5, 2.0).reshape(shape)
    if bf16:
        x = oracle.round_bf16(x)
    g = oracle.normal_f32(oracle.fold_in(key, 1), n, 1.0, 0.1)
    b = oracle.normal_f32(oracle.fold_in(key, 2), n, 0.0, 0.1)
    ln = nn.LayerNorm(E.fromHost(g), E.fromHost(b), [n], 1e-5)

    def fn():
        xt = E.fromHost(x, DType.BFLOAT16 if bf16 else DType.FLOAT32)
        y = ln.forward(nn._f32(xt))
        return nn._to(y, DType.BFLOAT16) if bf16 else y

    got, names = _run(fn)
    assert sum(k.startswith("layernorm_rows") for k in names) == 1, names
    assert not any(k.startswith("reduce") or k.startswith("ew_") for k in names), names
    ref, names2 = _run(fn, op_by_op=True)
    assert not any(k.startswith("layernorm_rows") for k in names2), names2
    x2 = x.reshape(-1, n)
    want = oracle.layernorm_rows(x2, g, b, 1e-5).reshape(shape)
    xd = x2.astype(np.float64)
    inv = 1.0 / np.sqrt(xd.var(-1, keepdims=True) + 1e-5)
    scale = (np.abs(g) * (np.abs(xd) + np.abs(xd).mean(-1, keepdims=True)) * inv +
             np.abs(b)).reshape(shape)
    for out in (got, ref):
        if bf16:
            out = _bits_f32(out)
            # within one bf16 rounding of the fp32 reference
            assert np.all(np.abs(out - want) <= 2.0 ** -8 * np.abs(want) + 1e-5 * scale)
        else:
            assert np.all(np.abs(out - want) <= 1e-5 * scale), \
                float(np.max(np.abs(out - want) / scale))


@pytest.mark.parametrize("ids_dt", [np.int32, np.int64])
def test_embedding_lookup_layernorm_one_pass(gpu, oracle, ids_dt):
    """rew's own decoder layer normalises with LayerNorm (models/llama.nim:
    32-33, 106-117): its first norm over Embedding.lookup's rows runs as one
    launch that writes the gathered rows (the residual) and their norm.  The
    rows equal table[ids] (ids clamped) bit for bit, and the norm equals the
    row kernel's on the same rows already in memory bit for bit."""
    V, H, T = 1000, 4096, 300
    key = oracle.init_key(4343)
    w = oracle.round_bf16(oracle.normal_f32(key, V * H).reshape(V, H))
    g = oracle.normal_f32(oracle.fold_in(key, 1), H, 1.0, 0.1)
    bt = oracle.normal_f32(oracle.fold_in(key, 2), H, 0.0, 0.1)
    ids = (np.arange(T) * 7919 % V).astype(ids_dt)
    ids[3], ids[7] = -5, V + 11
    table = E.fromHost(w, DType.BFLOAT16)
    ln = nn.LayerNorm(E.fromHost(g), E.fromHost(bt), [H], 1e-5)

    def fwd():
        x = O.reshape(nn.Embedding(table).lookup(E.fromHost(ids)), [1, T, H])
        normed = nn._to(ln.forward(nn._f32(x)), DType.BFLOAT16)
        return O.concat([normed, x], 0)   # x is needed again (the residual)

    got, names = _run(fwd)
    assert any(n.startswith("gather_layernorm") for n in names), names
    assert not any(n.startswith("gather_rows") or n.startswith("layernorm_rows")
                   for n in names), names
    rows = w[np.clip(ids.astype(np.int64), 0, V - 1)]
    xt = E.fromHost(rows.reshape(1, T, H), DType.BFLOAT16)
    plain, pn = _run(lambda: nn._to(ln.forward(nn._f32(xt)), DType.BFLOAT16))
    assert any(n.startswith("layernorm_rows") for n in pn), pn
    np.testing.assert_array_equal(got[0], plain[0])
    np.testing.assert_array_equal(E.bf16_bits_to_f32(got[1]).reshape(T, H), rows)
    want = oracle.layernorm_rows(rows, g, bt, 1e-5)
    bf16_close(E.bf16_bits_to_f32(got[0]).reshape(T, H), want, 1e-2)


@pytest.mark.parametrize("B,H,S,D,bf16", [(2, 4, 64, 128, True), (1, 3, 50, 64, False),
                                          (1, 2, 7, 32, True)])
def test_rope_pair_kernel(gpu, oracle, B, H, S, D, bf16):
    """rew's applyRotate chain (src/rew/nn/rope.nim:56-179) on a transposed
    projection view runs as one kernel, bit-exact with the op-by-op path."""
    key = oracle.init_key(600 + S)
    x = oracle.normal_f32(oracle.fold_in(key, 0), B * S * H * D).reshape(B, S, H, D)
    if bf16:
        x = oracle.round_bf16(x)
    dt = DType.BFLOAT16 if bf16 else DType.FLOAT32

    def fn():
        rope = nn.RotaryPositionEncoding.init(D, S + 8, 500000.0)
        xt = O.transpose(E.fromHost(x, dt), [0, 2, 1, 3])  # [B, H, S, D] view
        return rope.forward(xt, 3)

    got, names = _run(fn)
    assert any(k.startswith("rope_pairs") for k in names), names
    ref, names2 = _run(fn, op_by_op=True)
    assert not any(k.startswith("rope_pairs") for k in names2)
    np.testing.assert_array_equal(got, ref)
    c, s = nn.rope_tables(D, S + 8, 500000.0)
    want = oracle.rope(np.ascontiguousarray(x.transpose(0, 2, 1, 3)), c, s, 3)
    gotf = _bits_f32(got) if bf16 else got
    if bf16:
        assert np.all(np.abs(gotf - want) <= 2.0 ** -8 * np.abs(want) + 1e-6)
    else:
        np.testing.assert_allclose(gotf, want, rtol=1e-6, atol=1e-6)


# ---- attention projections: RoPE in the GEMM epilogue, q / k / v in one launch -----------

def _proj_rope(oracle, x, w, b, B, S, H, D, c, s, off, transposed):
    y = oracle.linear(x, w, b, True).reshape(B, S, H, D)  # bf16-rounded projection
    if transposed:
        y = np.ascontiguousarray(y.transpose(0, 2, 1, 3))
    return oracle.rope(y, c, s, off)


@pytest.mark.parametrize("B,S,E_,H,D,transposed", [(2, 96, 256, 4, 64, True),
                                                   (1, 300, 128, 2, 128, True),
                                                   (2, 40, 128, 3, 32, False)])
def test_rope_fused_into_projection(gpu, oracle, B, S, E_, H, D, transposed):
    """Linear -> reshape [B, S, H, D] (-> transpose [0, 2, 1, 3]) -> applyRotate
    (GroupedQueryAttention's q / k path) runs as one GEMM whose epilogue
    rotates the pairs and writes the rotated layout, bit-exact with op by op."""
    key = oracle.init_key(700 + S)
    w, b = _lin(oracle, key, E_, H * D)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 2), B * S * E_).reshape(B * S, E_))
    seq = H if not transposed else S  # the axis applyRotate treats as positions

    def fn():
        rope = nn.RotaryPositionEncoding.init(D, seq + 8, 500000.0)
        lin = nn.Linear(E.fromHost(w, DType.BFLOAT16), E.fromHost(b, DType.BFLOAT16))
        y = O.reshape(lin.forward(E.fromHost(x, DType.BFLOAT16)), [B, S, H, D])
        if transposed:
            y = O.transpose(y, [0, 2, 1, 3])
        return rope.forward(y, 3)

    got, names = _run(fn)
    assert any("+bias+rope" in n for n in names), names
    assert not any(k.startswith("rope_pairs") for k in names), names
    ref, names2 = _run(fn, op_by_op=True)
    assert not any("+rope" in n for n in names2)
    np.testing.assert_array_equal(got, ref)
    c, s = nn.rope_tables(D, seq + 8, 500000.0)
    want = _proj_rope(oracle, x, w, b, B, S, H, D, c, s, 3, transposed)
    bf16_close(_bits_f32(got), want)


@pytest.mark.parametrize("tables", ["transposed", "pairs_broadcast"])
def test_rope_fused_table_layouts(gpu, oracle, tables):
    """applyRotate called directly with cos / sin tables in other layouts: a
    [D, S] table read through a transpose (angle stride S: the epilogue's
    element-wise table loads) and a [S, D / 2] table broadcast over the pair
    axis (unit angle stride).  Fused or not, the result is bit-exact with op
    by op and within the bf16 tolerance of the oracle."""
    B, S, E_, H, D = 2, 48, 128, 2, 64
    key = oracle.init_key(760)
    w, b = _lin(oracle, key, E_, H * D)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 2), B * S * E_).reshape(B * S, E_))
    c, s = nn.rope_tables(D, S, 10000.0)

    def table(t):
        if tables == "transposed":
            return O.transpose(O.constantF32([D, S], np.ascontiguousarray(t.T)), [1, 0])
        half = O.constantF32([S, D // 2], np.ascontiguousarray(t[:, 0::2]))
        return O.reshape(O.broadcastTo(half, [S, D // 2, 2], [0, 1]), [S, D])

    def fn():
        lin = nn.Linear(E.fromHost(w, DType.BFLOAT16), E.fromHost(b, DType.BFLOAT16))
        y = O.transpose(O.reshape(lin.forward(E.fromHost(x, DType.BFLOAT16)), [B, S, H, D]),
                        [0, 2, 1, 3])
        cb = O.broadcastTo(table(c), [B, H, S, D], [2, 3])
        sb = O.broadcastTo(table(s), [B, H, S, D], [2, 3])
        return nn._to(nn.applyRotate(nn._f32(y), cb, sb), DType.BFLOAT16)

    got, names = _run(fn)
    ref, _ = _run(fn, op_by_op=True)
    np.testing.assert_array_equal(got, ref)
    want = _proj_rope(oracle, x, w, b, B, S, H, D, c, s, 0, True)
    bf16_close(_bits_f32(got), want)
    if tables == "transposed":
        assert any("+bias+rope" in n for n in names), names


@pytest.mark.parametrize("B,S,E_,H,KV,D", [(2, 96, 256, 4, 2, 64), (1, 200, 128, 2, 1, 136)])
def test_qkv_projections_one_launch(gpu, oracle, B, S, E_, H, KV, D):
    """The q (rotated), k (rotated) and v projections of one input run as one
    multi-segment GEMM launch; each output equals the op-by-op path."""
    key = oracle.init_key(800 + S)
    wq, bq = _lin(oracle, oracle.fold_in(key, 0), E_, H * D)
    wk, bk = _lin(oracle, oracle.fold_in(key, 1), E_, KV * D)
    wv, bv = _lin(oracle, oracle.fold_in(key, 2), E_, KV * D)
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 3), B * S * E_).reshape(B * S, E_))
    outs = {}

    def run(op_by_op):
        if op_by_op:
            E.setMode(E.MODE_OP_BY_OP)
        try:
            E.profileBegin()
            rope = nn.RotaryPositionEncoding.init(D, S, 10000.0)
            xt = E.fromHost(x, DType.BFLOAT16)
            mk = lambda w_, b_: nn.Linear(E.fromHost(w_, DType.BFLOAT16),
                                          E.fromHost(b_, DType.BFLOAT16))
            q = O.transpose(O.reshape(mk(wq, bq).forward(xt), [B, S, H, D]), [0, 2, 1, 3])
            k = O.transpose(O.reshape(mk(wk, bk).forward(xt), [B, S, KV, D]), [0, 2, 1, 3])
            v = O.transpose(O.reshape(mk(wv, bv).forward(xt), [B, S, KV, D]), [0, 2, 1, 3])
            q, k = rope.forward(q, 0), rope.forward(k, 0)
            res = [E.toHost(t) for t in (q, k, v)]
            names = [n for n, _, _ in E.profileEnd()]
        finally:
            E.setMode(E.MODE_DEFERRED)
        return res, names

    got, names = run(False)
    assert any(n.startswith("gemm_lds_nn{") and n.count("+rope") == 2 for n in names), names
    ref, _ = run(True)
    for g_, r_ in zip(got, ref):
        np.testing.assert_array_equal(g_, r_)
    c, s = nn.rope_tables(D, S, 10000.0)
    bf16_close(_bits_f32(got[0]), _proj_rope(oracle, x, wq, bq, B, S, H, D, c, s, 0, True))
    bf16_close(_bits_f32(got[1]), _proj_rope(oracle, x, wk, bk, B, S, KV, D, c, s, 0, True))
    want_v = np.ascontiguousarray(oracle.linear(x, wv, bv, True).reshape(B, S, KV, D)
                                  .transpose(0, 2, 1, 3))
    bf16_close(_bits_f32(got[2]), want_v)


_SOFTMAX_WG = (1024, 2048, 4096)  # row widths of the workgroup-per-row kernel


@pytest.mark.parametrize("shape", [(64, 4096), (33, 100), (16, 2048), (5, 8192), (7, 132),
                                   (2, 3, 256), (3, 130), (4099, 1024), (2100, 2048),
                                   (2050, 4096)])
def test_softmax_row_kernel(gpu, oracle, shape):
    """rew's softmax chain (src/rew/nn/activation.nim:64-77) over the last axis
    runs as one row kernel.  Rows of 1024, 2048 and 4096 run a workgroup per
    row, whose sum runs in another order than the compiled row reduction's:
    within 4e-6 of the op-by-op path.  Other widths follow that order and
    equal the op-by-op path bit for bit; rows of n % 4 != 0 at n >= 128 take
    the generic path."""
    n = shape[-1]
    x = oracle.normal_f32(oracle.init_key(900 + n), int(np.prod(shape))).reshape(shape) * 3
    x[(0,) * (len(shape) - 1)][min(5, n - 1)] = np.nan  # a NaN row
    if x.shape[-2] > 1:
        x[(0,) * (len(shape) - 2) + (1,)][:] = -np.inf   # an all -inf row

    def fn():
        return nn.softmax(E.fromHost(x), len(shape) - 1)

    got, names = _run(fn)
    fused = any(k.startswith("softmax_rows") for k in names)
    assert fused == (n < 128 or n % 4 == 0), names
    ref, names2 = _run(fn, op_by_op=True)
    assert not any(k.startswith("softmax_rows") for k in names2)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    num = ~np.isnan(got)
    if n in _SOFTMAX_WG:
        np.testing.assert_allclose(got[num], ref[num], rtol=4e-6, atol=1e-37)
    else:  # bit-exact, NaN payloads aside
        np.testing.assert_array_equal(got[num].view(np.uint32), ref[num].view(np.uint32))
    ok = np.isfinite(x).all(axis=-1)
    want = oracle.softmax_rows(x.reshape(-1, n)).reshape(shape)
    np.testing.assert_allclose(got[ok], want[ok], rtol=1e-5, atol=1e-9)


@pytest.mark.parametrize("n", [1024, 4096])
def test_softmax_wide_range_rows(gpu, oracle, n):
    """Rows scaled from 1 to 40 (spreads max - min from about 8 to 300, so
    probabilities from 1 down to the subnormal range): the workgroup-per-row
    kernel's quotients stay within 4e-6 of the op-by-op ones over 4-16 M
    values (subnormal quotients within 1e-37 absolute), and against the oracle
    within the 1e-5 fp32 tolerance."""
    rows = 4096
    x = oracle.normal_f32(oracle.init_key(950 + n), rows * n).reshape(rows, n)
    x *= np.linspace(1.0, 40.0, rows, dtype=np.float32)[:, None]

    def fn():
        return nn.softmax(E.fromHost(x), 1)

    got, names = _run(fn)
    assert any(k.startswith("softmax_rows") for k in names), names
    ref, _ = _run(fn, op_by_op=True)
    np.testing.assert_allclose(got, ref, rtol=4e-6, atol=1e-37)
    want = oracle.softmax_rows(x)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-37)


def test_repeated_reduction_runs_once(gpu, oracle):
    """reduceMean(y) is reduceSum(y) / n (src/rew/ops/reduce.nim): next to a
    reduceSum of the same tensor the sum is computed once and shared."""
    x = oracle.normal_f32(oracle.init_key(950), 256 * 1024).reshape(256, 1024)

    def fn():
        y = nn.relu(O.add(E.fromHost(x), E.fromHost(x)))
        return O.add(O.reduceSum(y, [1]), O.reduceMean(y, [1]))

    E.profileBegin()
    got = E.toHost(fn())
    prof = E.profileEnd()
    assert sum(c for n, c, _ in prof if n.startswith("reduce")) == 1, prof
    ref, _ = _run(fn, op_by_op=True)
    np.testing.assert_array_equal(got, ref)
    y = np.maximum(x + x, 0)
    s = y.astype(np.float64).sum(1)
    np.testing.assert_allclose(got, (s + s / 1024).astype(np.float32), rtol=1e-5)


MEAN_CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from rew_amd import eager as E, nn, ops as O
E.installEagerBackend(E.mi355x(0))
shape, axes = json.loads(sys.argv[2])
x = np.load(sys.argv[3])
y = nn.relu(O.add(E.fromHost(x), E.fromHost(x)))
outs = [O.reduceSum(y, axes), O.reduceMean(y, axes), O.reduceMax(y, axes)]
np.save(sys.argv[4], np.stack([E.toHost(t) for t in outs]))
"""


@pytest.mark.parametrize("shape,axes", [((128, 1024), [1]), ((64, 100), [1]), ((8, 16, 300), [2])])
def test_reduce_mean_divide_in_the_reduction(gpu, oracle, shape, axes, tmp_path):
    """reduceMean is reduceSum then divide by the broadcast count
    (src/rew/ops/reduce.nim:132-150).  Next to a reduceSum and a reduceMax of
    the same tensor (the C2 chain), the divide is stored by the reduction's
    own pass: one launch for the three results, equal to op-by-op bit for
    bit (the same sum divided by the same fp32 constant).  The interpreter
    (REW_MI355X_JIT=0) stores the sums and divides them afterwards: its mean
    is its own sum / n exactly."""
    import json
    import subprocess
    import sys
    from pathlib import Path
    x = oracle.normal_f32(oracle.init_key(970 + shape[-1]), int(np.prod(shape))).reshape(shape)

    def fn():
        y = nn.relu(O.add(E.fromHost(x), E.fromHost(x)))
        return [O.reduceSum(y, axes), O.reduceMean(y, axes), O.reduceMax(y, axes)]

    E.profileBegin()
    got = [E.toHost(t) for t in fn()]
    prof = E.profileEnd()
    assert [n for n, _, _ in prof if n.startswith("reduce")] and \
        sum(c for n, c, _ in prof if n.startswith("reduce") and ",mean" in n) == 1, prof
    assert not any(n.startswith("ew_") for n, _, _ in prof), prof
    E.setMode(E.MODE_OP_BY_OP)
    try:
        ref = [E.toHost(t) for t in fn()]
    finally:
        E.setMode(E.MODE_DEFERRED)
    for g_, r_ in zip(got, ref):
        np.testing.assert_array_equal(g_, r_)
    n = int(np.prod([shape[a] for a in axes]))
    np.testing.assert_array_equal(got[1], got[0] / np.float32(n))
    np.save(tmp_path / "x.npy", x)
    root = Path(__file__).resolve().parents[1]
    env = dict(__import__("os").environ, REW_MI355X_JIT="0")
    r = subprocess.run([sys.executable, "-c", MEAN_CHILD, str(root), json.dumps([shape, axes]),
                        str(tmp_path / "x.npy"), str(tmp_path / "out.npy")], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    interp = np.load(tmp_path / "out.npy")
    # the interpreter sums in its own order: its mean is its sum / n exactly
    np.testing.assert_array_equal(interp[1], interp[0] / np.float32(n))
    np.testing.assert_allclose(interp[0], got[0], rtol=1e-5)
    np.testing.assert_array_equal(interp[2], got[2])


@pytest.mark.parametrize("shape,axes", [((128, 1024), [1]), ((64, 100), [1]), ((8, 16, 300), [2])])
def test_sibling_reductions_one_pass(gpu, oracle, shape, axes):
    """reduceSum, reduceMax and reduceMin of one tensor over the same axes
    run as one pass with an accumulator per op, each in the single-op order:
    equal to the op-by-op path bit for bit."""
    x = oracle.normal_f32(oracle.init_key(960 + shape[-1]), int(np.prod(shape))).reshape(shape)

    def fn():
        y = nn.relu(O.add(E.fromHost(x), E.fromHost(x)))
        return [O.reduceSum(y, axes), O.reduceMax(y, axes), O.reduceMin(y, axes)]

    E.profileBegin()
    outs = fn()
    got = [E.toHost(t) for t in outs]
    prof = E.profileEnd()
    assert sum(c for n, c, _ in prof if n.startswith("reduce")) == 1, prof
    E.setMode(E.MODE_OP_BY_OP)
    try:
        ref = [E.toHost(t) for t in fn()]
    finally:
        E.setMode(E.MODE_DEFERRED)
    for g_, r_ in zip(got, ref):
        np.testing.assert_array_equal(g_, r_)
    y = np.maximum(x + x, 0)
    np.testing.assert_allclose(got[0], y.astype(np.float64).sum(axis=tuple(axes)), rtol=1e-5)
    np.testing.assert_array_equal(got[1], y.max(axis=tuple(axes)))
    np.testing.assert_array_equal(got[2], y.min(axis=tuple(axes)))


@pytest.mark.parametrize("ids_dt", [np.int32, np.int64])
def test_embedding_lookup_rmsnorm_one_pass(gpu, oracle, ids_dt):
    """LlamaDecoderLayer's first norm over Embedding.lookup's rows
    (embedding.nim, norm.nim:204-224): the lookup and the norm run as one
    launch that writes both the gathered rows (the layer's residual) and
    their norm; ids out of range clamp like torchIndexSelect.  The rows equal
    the op-by-op gather bit for bit, and the norm equals the row-norm
    kernel's on the same rows already in memory bit for bit."""
    V, H, T = 1000, 4096, 300
    key = oracle.init_key(4242)
    w = oracle.round_bf16(oracle.normal_f32(key, V * H).reshape(V, H))
    g = oracle.normal_f32(oracle.fold_in(key, 1), H, 1.0, 0.1)
    ids = (np.arange(T) * 7919 % V).astype(ids_dt)
    ids[3], ids[7] = -5, V + 11
    table, gamma = E.fromHost(w, DType.BFLOAT16), E.fromHost(g)

    def fwd():
        x = O.reshape(nn.Embedding(table).lookup(E.fromHost(ids)), [1, T, H])
        normed = nn._to(nn.RMSNorm(gamma).forward(nn._f32(x)), DType.BFLOAT16)
        return O.concat([normed, x], 0)   # x is needed again (the residual)

    got, names = _run(fwd)
    assert any(n.startswith("gather_rmsnorm") for n in names), names
    assert not any(n.startswith("gather_rows") or n.startswith("rmsnorm_rows") for n in names), names
    ref, _ = _run(fwd, op_by_op=True)
    np.testing.assert_array_equal(got[1], ref[1])
    rows = w[np.clip(ids.astype(np.int64), 0, V - 1)]
    xt = E.fromHost(rows.reshape(1, T, H), DType.BFLOAT16)
    plain, pn = _run(lambda: nn._to(nn.RMSNorm(gamma).forward(nn._f32(xt)), DType.BFLOAT16))
    assert any(n.startswith("rmsnorm_rows") for n in pn), pn
    np.testing.assert_array_equal(got[0], plain[0])
    np.testing.assert_array_equal(E.bf16_bits_to_f32(got[1]).reshape(T, H), rows)
    want = oracle.rmsnorm_rows(rows, g, 1e-5)
    bf16_close(E.bf16_bits_to_f32(got[0]).reshape(T, H), want, 1e-2)
