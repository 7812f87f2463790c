"""Pins the oracle's composite restatements (oracle/oracle.py: linear, silu,
gated_ffn, gqa, llama_layer, deepseek_moe, and orc_sdpa's bf16 mode)
before any GPU result is checked against them.

Each composite is compared with an independent float64 numpy statement of
the reference's definition, written here from the cited Nim source, on
tiny inputs, plus closed forms that fix structure exactly:

* silu: 0 -> 0, large x -> x, very negative x -> -0 (src/rew/nn/activation.nim:28-38);
* linear / gated_ffn: brute force, bias and gate/up roles distinguishable
  (src/rew/nn/linear.nim:43-49, src/rew/nn/gated_ffn.nim:46-67);
* gqa: projections, adjacent-pair RoPE, K/V head h // G, rew's additive
  mask (row <= col visible), output projection
  (src/rew/nn/groupedqueryattention.nim:75-144, src/rew/nn/rope.nim:56-179,
  src/rew/nn/attention.nim:18-81);
* llama_layer: zero output projections give x back exactly; brute force
  otherwise (src/rew/models/llama.nim:106-117, src/rew/nn/norm.nim:204-224);
* deepseek_moe: one expert with k = 1 is shared + that expert; k = E is the
  probability-weighted sum; general k against brute-force top-k
  (src/rew/models/deepseek.nim:114-145);
* sdpa(mixed=True): brute force with each bf16 rounding point of the op
  sequence written out.

A plausible slip -- a dropped bias, swapped gate and up, K/V head h % Hkv
instead of h // G, a mirrored mask, rotation of split halves instead of
adjacent pairs, a missing renormalisation -- moves the result by O(1) and
fails the tolerance, which is written next to each check.
"""
import numpy as np
import pytest


def rb(x):
    """float64 -> float32 -> bf16 (round to nearest even) -> float64, in numpy bits."""
    f = np.asarray(x, np.float64).astype(np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    out = r.astype(np.uint32).view(np.float32)
    out = np.where(np.isnan(f), f, out)
    return out.astype(np.float64)


def f32(x):
    return np.asarray(x, np.float64).astype(np.float32).astype(np.float64)


def rel(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


def bf16_vals(rng, shape, sd=1.0):
    return rb(rng.normal(0, sd, shape)).astype(np.float32)


# ---- brute-force statements ---------------------------------------------------------------

def lin_bf(x, w, b, bf16):
    xw = np.asarray(x, np.float64) @ np.asarray(w, np.float64)
    xw = rb(xw) if bf16 else f32(xw)
    y = f32(xw + np.asarray(b, np.float64))
    return rb(y) if bf16 else y


def silu_bf(x):
    x = np.asarray(x, np.float64)
    return x / (1.0 + np.exp(-x))


def ffn_bf(x, wg, bg, wu, bu, wd, bd, bf16):
    g = lin_bf(x, wg, bg, bf16)
    u = lin_bf(x, wu, bu, bf16)
    h = silu_bf(g) * u
    h = rb(h) if bf16 else f32(h)
    return lin_bf(h, wd, bd, bf16)


def rope_bf(x, theta):
    """Adjacent pairs (2i, 2i+1) rotated by pos * theta^(-2i/d), x [..., S, D]."""
    S, D = x.shape[-2], x.shape[-1]
    inv = theta ** (-np.arange(0, D, 2, dtype=np.float64) / D)
    ang = np.arange(S, dtype=np.float64)[:, None] * inv[None, :]
    c, s = np.cos(ang), np.sin(ang)
    x0, x1 = x[..., 0::2], x[..., 1::2]
    out = np.empty_like(x, dtype=np.float64)
    out[..., 0::2] = c * x0 - s * x1
    out[..., 1::2] = s * x0 + c * x1
    return out


def attn_bf(q, k, v, causal):
    """q [B,H,S,D], k / v [B,Hkv,S,D]; query head h reads KV head h // (H / Hkv)."""
    B, H, S, D = q.shape
    G = H // k.shape[1]
    out = np.zeros_like(q, dtype=np.float64)
    for b in range(B):
        for h in range(H):
            sc = (q[b, h] @ k[b, h // G].T) / np.sqrt(D)
            if causal:
                i, j = np.indices(sc.shape)
                sc = sc + np.where(i <= j, 0.0, -1e9)
            p = np.exp(sc - sc.max(1, keepdims=True))
            p /= p.sum(1, keepdims=True)
            out[b, h] = p @ v[b, h // G]
    return out


def gqa_bf(x, p, nh, nkv, theta, causal):
    B, S, E = x.shape
    hd = E // nh
    x2 = x.reshape(B * S, E).astype(np.float64)
    q = (x2 @ p["wq"] + p["bq"]).reshape(B, S, nh, hd).transpose(0, 2, 1, 3)
    k = (x2 @ p["wk"] + p["bk"]).reshape(B, S, nkv, hd).transpose(0, 2, 1, 3)
    v = (x2 @ p["wv"] + p["bv"]).reshape(B, S, nkv, hd).transpose(0, 2, 1, 3)
    a = attn_bf(rope_bf(q, theta), rope_bf(k, theta), v, causal)
    a2 = a.transpose(0, 2, 1, 3).reshape(B * S, E)
    return (a2 @ p["wo"] + p["bo"]).reshape(B, S, E)


def rms_bf(x, g, eps):
    x = np.asarray(x, np.float64)
    return g * (x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps))


# ---- silu -----------------------------------------------------------------------------------

def test_silu_closed_forms(oracle):
    x = np.array([0.0, 30.0, 100.0, -100.0, -200.0], np.float32)
    y = oracle.silu(x)
    assert y[0] == 0.0
    assert y[1] == 30.0 and y[2] == 100.0          # sigmoid rounds to exactly 1
    assert y[3] == 0.0 and np.signbit(y[3])         # exp(100) overflows: -100 * 0 = -0
    assert y[4] == 0.0 and np.signbit(y[4])


def test_silu_brute_force(oracle):
    x = np.random.default_rng(1).normal(0, 4, 4096).astype(np.float32)
    y = oracle.silu(x)
    np.testing.assert_allclose(y, silu_bf(x), rtol=1e-6, atol=1e-30)
    # silu(x) - silu(-x) == x: sigmoid(x) + sigmoid(-x) == 1
    np.testing.assert_allclose(y - oracle.silu(-x), x, rtol=1e-5, atol=1e-6)


# ---- linear / gated FFN ---------------------------------------------------------------------

@pytest.mark.parametrize("bf16", [False, True])
def test_linear_brute_force(oracle, bf16):
    rng = np.random.default_rng(2)
    x, w = bf16_vals(rng, (24, 40)), bf16_vals(rng, (40, 16), 0.2)
    b = bf16_vals(rng, (16,), 0.5)
    got = oracle.linear(x, w, b, bf16)
    if bf16:
        # one bf16 ulp at most, and only where the float64 sum sits on a tie
        assert np.all(np.abs(got - lin_bf(x, w, b, True)) <= 2.0 ** -7 * np.abs(got) + 1e-30)
        assert rel(got, lin_bf(x, w, b, True)) <= 1e-3
    else:
        np.testing.assert_allclose(got, lin_bf(x, w, b, False), rtol=3e-7, atol=1e-30)
    # the bias is added once, broadcast along rows
    assert rel(got, lin_bf(x, w, np.zeros_like(b), bf16)) > 0.05


@pytest.mark.parametrize("bf16", [False, True])
def test_gated_ffn_brute_force(oracle, bf16):
    rng = np.random.default_rng(3)
    T, E, I = 16, 32, 48
    x = bf16_vals(rng, (T, E))
    wg, wu = bf16_vals(rng, (E, I), 0.3), bf16_vals(rng, (E, I), 0.3)
    wd = bf16_vals(rng, (I, E), 0.3)
    bg, bu, bd = bf16_vals(rng, (I,), 0.3), bf16_vals(rng, (I,), 0.3), bf16_vals(rng, (E,), 0.3)
    got = oracle.gated_ffn(x, wg, bg, wu, bu, wd, bd, bf16)
    tol = 5e-3 if bf16 else 1e-5
    assert rel(got, ffn_bf(x, wg, bg, wu, bu, wd, bd, bf16)) <= tol
    # gate and up play different roles: swapping them changes the result
    assert rel(got, ffn_bf(x, wu, bu, wg, bg, wd, bd, bf16)) > 0.05


# ---- attention --------------------------------------------------------------------------------

def test_sdpa_mixed_brute_force(oracle):
    """orc_sdpa(mixed=True) restates rew's bf16 op stream: bf16 scores (the
    dot_general keeps the operand dtype), f32 scale and mask, f32 softmax,
    probabilities rounded to bf16, bf16 output."""
    rng = np.random.default_rng(4)
    B, H, Hkv, S, D = 1, 4, 2, 12, 16
    q, k, v = (bf16_vals(rng, (B, n, S, D)) for n in (H, Hkv, Hkv))
    sc = np.float32(1.0) / np.sqrt(np.float32(D))
    want = np.zeros((B, H, S, D))
    for h in range(H):
        s = rb(q[0, h].astype(np.float64) @ k[0, h // 2].T.astype(np.float64))
        s = f32(s * np.float64(sc))
        i, j = np.indices(s.shape)
        s = f32(s + np.where(i <= j, 0.0, -1e9))
        e = f32(np.exp(s - s.max(1, keepdims=True)))
        pr = rb(e / f32(e.sum(1, keepdims=True)))
        want[0, h] = rb(pr @ v[0, h // 2].astype(np.float64))
    got = oracle.sdpa(q, k, v, 1, mixed=True)
    assert np.all(np.abs(got - want) <= 2.0 ** -7 * np.abs(want) + 1e-6)
    # the fp32 mode is plain attention
    assert rel(oracle.sdpa(q, k, v, 1), attn_bf(q, k, v, True)) <= 1e-5
    # the mask direction matters: the mirrored mask gives another result
    assert rel(oracle.sdpa(q, k, v, 2), attn_bf(q, k, v, True)) > 0.05


@pytest.mark.parametrize("code,visible", [(1, "le"), (2, "ge"), (3, "lt"), (4, "gt")])
def test_sdpa_mask_directions(oracle, code, visible):
    """Each ordered mask against brute force; a row with no visible key
    (the last row under i < j, the first under i > j) softmaxes scores that
    all round to -1e9, so it averages V."""
    rng = np.random.default_rng(40 + code)
    B, H, S, D = 1, 2, 9, 8
    q, k, v = (rng.normal(0, 1, (B, H, S, D)).astype(np.float32) for _ in range(3))
    sc = np.float32(1.0) / np.sqrt(np.float32(D))
    i, j = np.indices((S, S))
    vis = {"le": i <= j, "ge": i >= j, "lt": i < j, "gt": i > j}[visible]
    want = np.zeros((B, H, S, D))
    for h in range(H):
        s = f32(f32(q[0, h].astype(np.float64) @ k[0, h].T.astype(np.float64)) * np.float64(sc))
        s = f32(s + np.where(vis, 0.0, -1e9))
        p = np.exp(s - s.max(1, keepdims=True))
        want[0, h] = (p / p.sum(1, keepdims=True)) @ v[0, h]
    got = oracle.sdpa(q, k, v, code)
    assert rel(got, want) <= 1e-5
    empty = np.where(~vis.any(1))[0]
    for r in empty:
        np.testing.assert_allclose(got[0, :, r], v[0].mean(1), rtol=1e-5, atol=1e-6)


def _gqa_params(rng, E, nkv, hd, bias=0.2):
    p = {}
    for n, fo in [("q", E), ("k", nkv * hd), ("v", nkv * hd), ("o", E)]:
        p["w" + n] = bf16_vals(rng, (E, fo), 0.15)
        p["b" + n] = bf16_vals(rng, (fo,), bias)
    return p


def test_gqa_brute_force(oracle):
    rng = np.random.default_rng(5)
    B, S, E, nh, nkv, theta = 2, 10, 32, 4, 2, 10000.0
    hd = E // nh
    p = _gqa_params(rng, E, nkv, hd)
    x = bf16_vals(rng, (B, S, E))
    c, s = oracle.rope_tables(hd, S, theta)
    for causal in (True, False):
        got = oracle.gqa(x, p, nh, nkv, c, s, causal, False)
        assert rel(got, gqa_bf(x, p, nh, nkv, theta, causal)) <= 1e-5
    # K/V head h // G, not h % Hkv: swapping the KV heads' weights changes the result
    p2 = dict(p)
    for n in ("wk", "wv"):
        p2[n] = np.concatenate([p[n][:, hd:], p[n][:, :hd]], axis=1)
    for n in ("bk", "bv"):
        p2[n] = np.concatenate([p[n][hd:], p[n][:hd]])
    assert rel(oracle.gqa(x, p2, nh, nkv, c, s, True, False),
               oracle.gqa(x, p, nh, nkv, c, s, True, False)) > 0.05
    # bf16 mode stays within the layer tolerance of the float64 statement
    got16 = oracle.gqa(x, p, nh, nkv, c, s, True, True)
    assert rel(got16, gqa_bf(x, p, nh, nkv, theta, True)) <= 2e-2


# ---- decoder layer ----------------------------------------------------------------------------

def _layer_params(rng, E, nkv, hd, I):
    p = _gqa_params(rng, E, nkv, hd)
    for n, fi, fo in [("g", E, I), ("u", E, I), ("d", I, E)]:
        p["w" + n] = bf16_vals(rng, (fi, fo), 0.15)
        p["b" + n] = bf16_vals(rng, (fo,), 0.2)
    p["g1"] = rng.normal(1.0, 0.1, E).astype(np.float32)
    p["g2"] = rng.normal(1.0, 0.1, E).astype(np.float32)
    return p


def test_llama_layer_zero_projections_return_x(oracle):
    """With W_o, b_o, W_down and b_down zero both branches add exact zeros."""
    rng = np.random.default_rng(6)
    B, S, E, nh, nkv, I = 1, 8, 32, 4, 2, 64
    p = _layer_params(rng, E, nkv, E // nh, I)
    for n in ("wo", "bo", "wd", "bd"):
        p[n] = np.zeros_like(p[n])
    x = bf16_vals(rng, (B, S, E))
    c, s = oracle.rope_tables(E // nh, S, 500000.0)
    for norm in ("rms", "layer"):
        got = oracle.llama_layer(x, p, nh, nkv, c, s, 1e-5, True, True, norm)
        np.testing.assert_array_equal(got, x)


def test_llama_layer_brute_force(oracle):
    rng = np.random.default_rng(7)
    B, S, E, nh, nkv, I, theta = 2, 8, 32, 4, 2, 64, 500000.0
    p = _layer_params(rng, E, nkv, E // nh, I)
    x = bf16_vals(rng, (B, S, E))
    c, s = oracle.rope_tables(E // nh, S, theta)
    h = x + gqa_bf(rms_bf(x, p["g1"], 1e-5), p, nh, nkv, theta, True)
    n2 = rms_bf(h, p["g2"], 1e-5).reshape(B * S, E)
    g = n2 @ p["wg"] + p["bg"]
    u = n2 @ p["wu"] + p["bu"]
    want = h + ((silu_bf(g) * u) @ p["wd"] + p["bd"]).reshape(B, S, E)
    assert rel(oracle.llama_layer(x, p, nh, nkv, c, s, 1e-5, True, False, "rms"), want) <= 1e-5
    assert rel(oracle.llama_layer(x, p, nh, nkv, c, s, 1e-5, True, True, "rms"), want) <= 2e-2


# ---- mixture of experts ---------------------------------------------------------------------

def _experts(rng, n, H, I):
    out = []
    for _ in range(n):
        out.append((bf16_vals(rng, (H, I), 0.2), bf16_vals(rng, (I,), 0.2),
                    bf16_vals(rng, (H, I), 0.2), bf16_vals(rng, (I,), 0.2),
                    bf16_vals(rng, (I, H), 0.2), bf16_vals(rng, (H,), 0.2)))
    return out


def test_moe_single_expert_is_shared_plus_expert(oracle):
    rng = np.random.default_rng(8)
    T, H, I = 12, 16, 24
    x = bf16_vals(rng, (T, H))
    shared, routed = _experts(rng, 1, H, I), _experts(rng, 1, H, I)
    wr = rng.normal(0, 0.3, (H, 1)).astype(np.float32)
    out, ti, tw = oracle.deepseek_moe(x, shared, routed, wr, np.zeros(1, np.float32), 1)
    assert np.all(ti == 0) and np.all(tw == 1.0)
    want = oracle.round_bf16(oracle.gated_ffn(x, *shared[0], True) +
                             oracle.gated_ffn(x, *routed[0], True))
    np.testing.assert_array_equal(out, want)
    # without shared experts the output is exactly the routed expert
    out2, _, _ = oracle.deepseek_moe(x, [], routed, wr, np.zeros(1, np.float32), 1)
    np.testing.assert_array_equal(out2, oracle.gated_ffn(x, *routed[0], True))


def _moe_bf(x, shared, routed, wr, k):
    """Float64 statement with explicit stable top-k: out = sum_shared E_s(x)
    + sum_e E_e(x) * w_e, w = renormalised top-k of softmax(x W_r)."""
    logits = x.astype(np.float64) @ wr
    pr = np.exp(logits - logits.max(1, keepdims=True))
    pr /= pr.sum(1, keepdims=True)
    order = np.argsort(-pr, axis=1, kind="stable")[:, :k]
    w = np.zeros_like(pr)
    for t in range(x.shape[0]):
        sel = pr[t, order[t]]
        w[t, order[t]] = sel / sel.sum()
    out = sum(ffn_bf(x, *s, False) for s in shared) if shared else 0.0
    for e, ex in enumerate(routed):
        out = out + ffn_bf(x, *ex, False) * w[:, e:e + 1]
    return out, order


@pytest.mark.parametrize("k", [2, 6])
def test_moe_brute_force(oracle, k):
    rng = np.random.default_rng(9 + k)
    T, H, I, E = 16, 16, 24, 6
    x = bf16_vals(rng, (T, H))
    shared, routed = _experts(rng, 2, H, I), _experts(rng, E, H, I)
    wr = rng.normal(0, 0.5, (H, E)).astype(np.float32)
    out, ti, tw = oracle.deepseek_moe(x, shared, routed, wr, np.zeros(E, np.float32), k)
    want, order = _moe_bf(x, shared, routed, wr, k)
    np.testing.assert_array_equal(ti, order)
    np.testing.assert_allclose(tw.sum(1), 1.0, rtol=1e-6)
    assert rel(out, want) <= 2e-2
    if k == E:
        # every expert is selected: the weights are the router probabilities
        # and the output is the probability-weighted sum over all experts
        pr = oracle.softmax_rows(oracle.linear(x, wr, np.zeros(E, np.float32), False))
        w_by_e = np.zeros_like(pr)
        np.put_along_axis(w_by_e, ti.astype(np.int64), tw, axis=1)
        np.testing.assert_allclose(w_by_e, pr, rtol=1e-6)
    # without renormalisation (raw top-k probabilities) the result differs
    if k < E:
        raw = np.zeros((T, E))
        logits = x.astype(np.float64) @ wr
        pr = np.exp(logits - logits.max(1, keepdims=True))
        pr /= pr.sum(1, keepdims=True)
        np.put_along_axis(raw, order, np.take_along_axis(pr, order, 1), axis=1)
        unnorm = sum(ffn_bf(x, *s, False) for s in shared) + sum(
            ffn_bf(x, *ex, False) * raw[:, e:e + 1] for e, ex in enumerate(routed))
        assert rel(out, unnorm) > 3 * rel(out, want)
