"""GPU parity of the rew.nn composites and layers (fused by the backend's
deferred graph) against the oracle's restatement of the same op sequences.

Tolerances: fp32 composites <= 1e-5 relative (normwise for sums);
bf16 layers <= 2e-2 relative (normwise and max-abs vs max |ref|).
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
    return E.toHostF32(t)


def bf16_close(got, want, tol=2e-2):
    err = np.linalg.norm((got - want).ravel()) / max(np.linalg.norm(want.ravel()), 1e-30)
    assert err <= tol, f"normwise relative error {err:.3e} > {tol}"
    assert np.max(np.abs(got - want)) <= 5 * tol * np.max(np.abs(want)) + 1e-30


def test_relu_chain_exact(gpu, oracle):
    x = oracle.normal_f32(oracle.init_key(0x5EED0002), 64 * 4096).reshape(64, 4096)
    t = dev(x)
    y = host(nn.relu(O.add(t, t)))
    want = oracle.binary(oracle.MAX, oracle.binary(oracle.ADD, x, x), np.zeros_like(x))
    np.testing.assert_array_equal(y.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("rows,cols", [(64, 4096), (33, 100), (16, 2048)])
def test_softmax(gpu, oracle, rows, cols):
    x = oracle.normal_f32(oracle.init_key(rows + cols), rows * cols).reshape(rows, cols) * 3
    got = host(nn.softmax(dev(x), 1))
    np.testing.assert_allclose(got, oracle.softmax_rows(x), rtol=1e-5, atol=1e-9)


def test_rmsnorm_and_mean(gpu, oracle):
    key = oracle.init_key(0x5EED0002)
    x = oracle.normal_f32(key, 64 * 4096).reshape(64, 4096)
    g = oracle.normal_f32(oracle.fold_in(key, 1), 4096, 1.0, 0.1)
    got = host(nn.rmsNorm(dev(x), dev(g), 1e-5))
    np.testing.assert_allclose(got, oracle.rmsnorm_rows(x, g, 1e-5), rtol=1e-5, atol=1e-6)
    y = np.maximum(x + x, 0)
    m = host(O.reduceMean(dev(y), [1]))
    want = oracle.reduce(oracle.RSUM, y, [1]) / np.float32(4096)
    np.testing.assert_allclose(m, want, rtol=1e-5)


def test_layernorm(gpu, oracle):
    x = oracle.normal_f32(oracle.init_key(5), 32 * 512, 2.0, 3.0).reshape(32, 512)
    ln = nn.LayerNorm.init([512], 1e-5)
    got = host(ln.forward(dev(x)))
    want = oracle.layernorm_rows(x, np.ones(512, np.float32), np.zeros(512, np.float32), 1e-5)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=2e-5)


def test_rope_f32(gpu, oracle):
    rope = nn.RotaryPositionEncoding.init(128, 256, 500000.0)
    c, s = nn.rope_tables(128, 256, 500000.0)
    x = oracle.normal_f32(oracle.init_key(6), 2 * 4 * 64 * 128).reshape(2, 4, 64, 128)
    got = host(rope.forward(dev(x), offset=3))
    want = oracle.rope(x, c, s, offset=3)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)


@pytest.mark.parametrize("causal", [False, True])
def test_sdpa_gqa_f32(gpu, oracle, causal):
    B, H, Hkv, S, D = 1, 4, 2, 48, 32
    key = oracle.init_key(7)
    q = oracle.normal_f32(oracle.fold_in(key, 0), B * H * S * D).reshape(B, H, S, D)
    k = oracle.normal_f32(oracle.fold_in(key, 1), B * Hkv * S * D).reshape(B, Hkv, S, D)
    v = oracle.normal_f32(oracle.fold_in(key, 2), B * Hkv * S * D).reshape(B, Hkv, S, D)
    g = H // Hkv
    kt, vt = dev(k), dev(v)
    kf = O.reshape(O.broadcastTo(O.reshape(kt, [B, Hkv, 1, S, D]), [B, Hkv, g, S, D],
                                 [0, 1, 2, 3, 4]), [B, H, S, D])
    vf = O.reshape(O.broadcastTo(O.reshape(vt, [B, Hkv, 1, S, D]), [B, Hkv, g, S, D],
                                 [0, 1, 2, 3, 4]), [B, H, S, D])
    got = host(nn.scaledDotProductAttention(dev(q), kf, vf, causal=causal))
    want = oracle.sdpa(q, k, v, causal)
    np.testing.assert_allclose(got, want, rtol=1e-4, atol=1e-5)


def _linear(oracle, key, fin, fout, bf16=True):
    w = oracle.normal_f32(key, fin * fout, 0.0, 0.02).reshape(fin, fout)
    b = np.zeros(fout, np.float32)
    if bf16:
        w = oracle.round_bf16(w)
    dt = DType.BFLOAT16 if bf16 else DType.FLOAT32
    return nn.Linear(dev(w, dt), dev(b, dt)), w, b


def test_gated_ffn_bf16(gpu, oracle):
    E_, I, T = 256, 512, 128
    key = oracle.init_key(0x5EED0003)
    ks = oracle.split(key, 4)
    x = oracle.round_bf16(oracle.normal_f32(ks[0], T * E_).reshape(1, T, E_))
    lg, wg, bg = _linear(oracle, ks[1], E_, I)
    lu, wu, bu = _linear(oracle, ks[2], E_, I)
    ld, wd, bd = _linear(oracle, ks[3], I, E_)
    ffn = nn.GatedFeedForward(lg, lu, ld)
    got = host(ffn.forward(dev(x, DType.BFLOAT16)))
    want = oracle.gated_ffn(x.reshape(T, E_), wg, bg, wu, bu, wd, bd, True).reshape(1, T, E_)
    bf16_close(got, want)


def _llama_params(oracle, key, E_, nh, nkv, I):
    hd = E_ // nh
    ks = oracle.split(key, 9)
    p, mods = {}, {}
    for i, (name, fi, fo) in enumerate([("q", E_, E_), ("k", E_, nkv * hd), ("v", E_, nkv * hd),
                                        ("o", E_, E_), ("g", E_, I), ("u", E_, I),
                                        ("d", I, E_)]):
        lin, w, b = _linear(oracle, ks[i], fi, fo)
        p["w" + name], p["b" + name] = w, b
        mods[name] = lin
    p["g1"] = oracle.normal_f32(ks[7], E_, 1.0, 0.1)
    p["g2"] = oracle.normal_f32(ks[8], E_, 1.0, 0.1)
    return p, mods


@pytest.mark.parametrize("causal", [True, False])
def test_llama_layer_bf16(gpu, oracle, causal):
    B, S, E_, nh, nkv, I = 2, 64, 256, 4, 2, 512
    key = oracle.init_key(0x5EED0004)
    p, m = _llama_params(oracle, key, E_, nh, nkv, I)
    hd = E_ // nh
    rope = nn.RotaryPositionEncoding.init(hd, S, 500000.0)
    c, s = nn.rope_tables(hd, S, 500000.0)
    attn = nn.GroupedQueryAttention(m["q"], m["k"], m["v"], m["o"], nh, nkv, hd, rope)
    ffn = nn.GatedFeedForward(m["g"], m["u"], m["d"])
    layer = nn.LlamaDecoderLayer(attn, ffn, nn.RMSNorm(dev(p["g1"]), 1e-5),
                                 nn.RMSNorm(dev(p["g2"]), 1e-5))
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 99), B * S * E_)
                          .reshape(B, S, E_))
    got = host(layer.forward(dev(x, DType.BFLOAT16), causal=causal))
    want = oracle.llama_layer(x, p, nh, nkv, c, s, 1e-5, causal, True, "rms")
    bf16_close(got, want)


def test_llama_layer_kernel_plan(gpu, oracle):
    """The decoder layer runs as its fused kernels: one launch for the q / k / v
    projections with RoPE in the q and k epilogues, flash attention, the
    O projection with bias + residual, the SwiGLU dual GEMM, the down
    projection with bias + residual, and the two rmsNorm row kernels."""
    B, S, E_, nh, nkv, I = 2, 64, 256, 4, 2, 512
    key = oracle.init_key(0x5EED0005)
    p, m = _llama_params(oracle, key, E_, nh, nkv, I)
    hd = E_ // nh
    rope = nn.RotaryPositionEncoding.init(hd, S, 500000.0)
    attn = nn.GroupedQueryAttention(m["q"], m["k"], m["v"], m["o"], nh, nkv, hd, rope)
    ffn = nn.GatedFeedForward(m["g"], m["u"], m["d"])
    layer = nn.LlamaDecoderLayer(attn, ffn, nn.RMSNorm(dev(p["g1"]), 1e-5),
                                 nn.RMSNorm(dev(p["g2"]), 1e-5))
    x = oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 99), B * S * E_)
                          .reshape(B, S, E_))
    xt = dev(x, DType.BFLOAT16)
    E.profileBegin()
    got = host(layer.forward(xt, causal=True))
    prof = E.profileEnd()  # (kernel name, launches, ms)
    names = [n for n, _, _ in prof]

    def launches(pred):
        return sum(cnt for n, cnt, _ in prof if pred(n))

    assert launches(lambda n: n.startswith("gemm_lds_nn{") and n.count("+rope") == 2) == 1, names
    assert launches(lambda n: n.startswith("rope_pairs")) == 0, names
    assert launches(lambda n: n.startswith("flash_attn")) == 1, names
    assert launches(lambda n: "swiglu" in n) == 1, names
    assert launches(lambda n: "+bias+res" in n) == 2, names
    assert launches(lambda n: n.startswith("rmsnorm_rows")) == 2, names
    assert sum(cnt for _, cnt, _ in prof) == 7, names
    c, s = nn.rope_tables(hd, S, 500000.0)
    want = oracle.llama_layer(x, p, nh, nkv, c, s, 1e-5, True, True, "rms")
    bf16_close(got, want)


def test_embedding_gather_equals_one_hot(gpu, oracle):
    V, H, T = 512, 64, 40
    w = oracle.round_bf16(oracle.normal_f32(oracle.init_key(8), V * H).reshape(V, H))
    ids = (np.arange(T) * 37 % V).astype(np.int32)
    emb = nn.Embedding(dev(w, DType.BFLOAT16))
    got = E.toHost(emb.lookup(dev(ids)))
    np.testing.assert_array_equal(got, oracle.to_bf16(w[ids]))
    onehot = np.zeros((T, V), np.float32)
    onehot[np.arange(T), ids] = 1
    got2 = E.toHost(emb.forward(dev(onehot, DType.BFLOAT16)))
    np.testing.assert_array_equal(got2, got)
