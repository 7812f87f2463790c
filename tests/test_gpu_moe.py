"""GPU parity of the routed MoE path (config C5 shape family).

rew's DeepSeekMoE.forward (src/rew/models/deepseek.nim:114-145) is a dense
formulation: every routed expert runs on every token and is added in expert
order with a routing weight that is zero off the token's top-k.  The backend
recognises that op chain and evaluates it sparsely (routing, grouped
SwiGLU / down GEMMs over the routed rows, ordered combine).  Checks:

* against the oracle's dense restatement: bf16 layer tolerance (normwise
  relative error <= 2e-2); expert ids bit-exact except where the oracle's
  router probabilities hold a near-tie at the selection boundary;
* against the backend's own op-by-op (dense, unfused) execution of the same
  op sequence: equal values (the skipped terms are exact zeros and the
  kernels share one MFMA accumulation order).  This holds while every
  expert's output is finite: the dense chain turns a token's sum into NaN
  when an expert it is NOT routed to yields inf or NaN (bf16(inf * 0) is
  NaN), while the routed path never evaluates that expert on that token;
* that the sparse kernels really ran (profile names).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

import ctypes as C

from rew_amd import _lib
from rew_amd import eager as E
from rew_amd import nn, rng
from rew_amd import ops as O
from rew_amd import ops as O
from rew_amd.eager import DType


def build_moe(oracle, T, H, I, E_, k, n_shared, seed):
    keys = rng.split(rng.initKey(seed), 3 + n_shared + E_)
    x = oracle.round_bf16(rng.normalF32(keys[0], T * H).reshape(T, H))
    wr = rng.normalF32(keys[1], H * E_, 0.0, 0.02).reshape(H, E_)
    br = np.zeros(E_, np.float32)

    def expert(key):
        ks = rng.split(key, 3)
        ws = [oracle.round_bf16(rng.normalF32(ks[i], fi * fo, 0.0, 0.02).reshape(fi, fo))
              for i, (fi, fo) in enumerate([(H, I), (H, I), (I, H)])]
        zI, zH = np.zeros(I, np.float32), np.zeros(H, np.float32)
        host = (ws[0], zI, ws[1], zI, ws[2], zH)
        dev = nn.DeepSeekExpert(*[nn.Linear(E.fromHost(w, DType.BFLOAT16),
                                            E.fromHost(b, DType.BFLOAT16))
                                  for w, b in [(ws[0], zI), (ws[1], zI), (ws[2], zH)]])
        return host, dev

    shared = [expert(keys[3 + i]) for i in range(n_shared)]
    routed = [expert(keys[3 + n_shared + e]) for e in range(E_)]
    moe = nn.DeepSeekMoE(nn.Linear(E.fromHost(wr), E.fromHost(br)),
                         [d for _, d in shared], [d for _, d in routed], k)
    host = dict(x=x, wr=wr, br=br, shared=[h for h, _ in shared],
                routed=[h for h, _ in routed])
    return moe, host


def ids_match_off_near_ties(oracle, host, k, got_ids, probs_tol=1e-6):
    """Expert ids must equal the oracle's except on rows whose router
    probabilities have a near-tie at or above the k-th place."""
    x = host["x"]
    probs = oracle.softmax_rows(oracle.linear(x, host["wr"], host["br"], False))
    _, want = oracle.topk_rows(probs, k)
    srt = -np.sort(-probs, axis=1)
    gaps = srt[:, :k] - srt[:, 1:k + 1]
    near = np.any(gaps <= probs_tol * srt[:, :1], axis=1)
    bad = np.any(got_ids != want, axis=1) & ~near
    assert not bad.any(), f"expert ids differ off near-ties in rows {np.where(bad)[0][:10]}"
    return int(near.sum())


def check_expert_ids(oracle, moe, xt, host, k):
    """The routing contract: expert ids are bit-exact given identical router
    probabilities.  The backend's top-k ids must equal the oracle's top-k of
    the backend's own probabilities; those probabilities must match the
    oracle's fp32 router within fp32 tolerance (normwise 1e-5); and a row
    whose ids differ from the oracle's top-k of the oracle's probabilities
    must hold two candidates closer together than the probability error
    actually observed on that row (a near-tie).  Returns that row count."""
    probs_dev = E.toHost(nn.softmax(moe.gate.forward(O.astype(xt, DType.FLOAT32)), 1))
    _, ids = moe.route(xt)
    ids = E.toHost(ids)
    _, want_same = oracle.topk_rows(probs_dev, k)
    np.testing.assert_array_equal(ids, want_same)
    probs = oracle.softmax_rows(oracle.linear(host["x"], host["wr"], host["br"], False))
    err = np.linalg.norm(probs_dev - probs) / np.linalg.norm(probs)
    assert err <= 1e-5, f"router probabilities normwise relative error {err:.3e}"
    _, want = oracle.topk_rows(probs, k)
    diff = np.where(np.any(ids != want, axis=1))[0]
    for r in diff:
        row_err = np.max(np.abs(probs_dev[r] - probs[r]))
        srt = np.sort(probs[r])[::-1]
        gap = np.min(srt[:k] - srt[1:k + 1])
        assert gap <= 2 * row_err, (r, gap, row_err)
    return len(diff)


@pytest.mark.parametrize("T,H,I,E_,k,n_shared", [(256, 256, 128, 16, 4, 2),
                                                  (200, 264, 136, 8, 2, 1),
                                                  (32, 128, 64, 64, 2, 2)])
def test_moe_matches_oracle(gpu, oracle, T, H, I, E_, k, n_shared):
    moe, host = build_moe(oracle, T, H, I, E_, k, n_shared, 0x5EED0005 + T)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    E.profileBegin()
    out = E.toHostF32(moe.forward(xt))
    prof = [name for name, _, _ in E.profileEnd()]
    assert any(n.startswith("moe_gemm_swiglu") for n in prof), prof
    assert any(n.startswith("moe_combine") for n in prof), prof
    # the shared experts belong to the group: their SwiGLU and down GEMMs
    # are groups of all T rows in the members' two grouped launches
    sw = [n for n in prof if "swiglu" in n]
    assert sw == [f"moe_gemm_swiglu[{E_ + n_shared},{T * k + n_shared * T},{I},{H}]"], prof
    dn = [n for n in prof if n.startswith("moe_gemm_down")]
    assert dn == [f"moe_gemm_down[{E_ + n_shared},{T * k + n_shared * T},{H},{I}]"], prof
    assert not any(n.startswith("moe_shared_down") for n in prof), prof
    want, ti, tw = oracle.deepseek_moe(host["x"], host["shared"], host["routed"], host["wr"],
                                       host["br"], k)
    err = np.linalg.norm(out - want) / np.linalg.norm(want)
    assert err <= 2e-2, f"normwise relative error {err:.3e}"
    check_expert_ids(oracle, moe, xt, host, k)


def test_moe_sparse_equals_dense_op_by_op(gpu, oracle):
    moe, host = build_moe(oracle, 256, 256, 128, 16, 4, 2, 0x5EED0105)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    sparse = E.toHostF32(moe.forward(xt))
    E.setMode(1)
    try:
        dense = E.toHostF32(moe.forward(xt))
    finally:
        E.setMode(0)
    # equal values (an exact zero's sign may differ: dense adds +-0 terms)
    np.testing.assert_array_equal(sparse, dense)


def small_and_large_groups(oracle):
    """Groups of more than 128 rows (256-row tiles, ragged last ones), of
    65-128 rows (two 64-row tiles) and of at most 64 rows (one) in the same
    grouped launches (this seed's router, two experts biased: rows per
    expert 215, 37, 500, 334, 4, 105, 22, 62, 1 and zeros).  Returns the
    sparse and the dense op-by-op results and the oracle's."""
    T, H, I, E_, k = 640, 256, 128, 16, 2
    moe, host = build_moe(oracle, T, H, I, E_, k, 1, 0x5EED0205)
    br = np.zeros(E_, np.float32)
    br[1] = 0.33
    br[9] = 0.165
    moe.gate = nn.Linear(E.fromHost(host["wr"]), E.fromHost(br))
    probs = oracle.softmax_rows(oracle.linear(host["x"], host["wr"], br, False))
    _, ids = oracle.topk_rows(probs, k)
    rows = np.bincount(ids.ravel(), minlength=E_)
    assert (rows > 256).any() and (rows % 256 != 0)[rows > 256].any(), rows
    assert ((rows > 64) & (rows <= 128)).any() and ((rows > 0) & (rows <= 64)).any(), rows
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    sparse = E.toHostF32(moe.forward(xt))
    E.setMode(E.MODE_OP_BY_OP)
    try:
        dense = E.toHostF32(moe.forward(xt))
    finally:
        E.setMode(E.MODE_DEFERRED)
    want, _, _ = oracle.deepseek_moe(host["x"], host["shared"], host["routed"], host["wr"],
                                     br, k)
    return sparse, dense, want


def test_moe_small_and_large_groups(gpu, oracle):
    """The 64-row tiles of the small groups run the same MFMA sequence per
    output as the 256-row tiles, so the sparse result equals the dense
    op-by-op one and stays within the oracle's tolerance."""
    sparse, dense, want = small_and_large_groups(oracle)
    np.testing.assert_array_equal(sparse, dense)
    err = np.linalg.norm(sparse - want) / np.linalg.norm(want)
    assert err <= 2e-2, f"normwise relative error {err:.3e}"


MIXED_CHILD = r"""
import json, sys
import numpy as np
root = sys.argv[1]
for p in (root, root + "/tests", root + "/oracle"):
    sys.path.insert(0, p)
import oracle as orc
from test_gpu_moe import small_and_large_groups
from rew_amd import eager as E
E.installEagerBackend(E.mi355x(0))
sparse, dense, want = small_and_large_groups(orc)
print(json.dumps({"equal": bool(np.array_equal(sparse, dense)),
                  "err": float(np.linalg.norm(sparse - want) / np.linalg.norm(want))}))
"""


def test_moe_small_groups_on_the_register_staged_kernel(gpu, oracle):
    """REW_MI355X_GEMM_TILE=256 sends the grouped GEMMs to the register-staged
    256 x 256 kernel, which reads the same 64-row tiles of the small groups
    (as 256-row tiles with the rows past 64 unused)."""
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ, REW_MI355X_GEMM_TILE="256")
    r = subprocess.run([sys.executable, "-c", MIXED_CHILD, str(root)], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["equal"] and res["err"] <= 2e-2, res


def test_moe_expert_matrices_far_apart(gpu, oracle):
    """Expert gate and up weights more than 2 GiB apart (allocations need
    not be near each other).  Shared expert 1's: the two shared SwiGLU GEMMs
    still run as one launch, reading B through per-lane addresses; routed
    expert 5's through the C-ABI entry point: the grouped GEMM does the same
    for every expert.  Same bits as with the weights near each other."""
    from test_gpu_fusion import far_apart
    moe, host = build_moe(oracle, 512, 256, 128, 16, 4, 2, 0x5EED0905)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    near = E.toHost(moe.forward(xt))
    sh = host["shared"][1]
    _, _, view = far_apart([sh[0], sh[2]])
    ex1 = moe.sharedExperts[1]
    saved = (ex1.gateProj, ex1.upProj)

    def forward_far():
        # the views are dropped again before the flush, so they stay views
        ex1.gateProj = nn.Linear(view(0), saved[0].bias)
        ex1.upProj = nn.Linear(view(1), saved[1].bias)
        y = moe.forward(xt)
        ex1.gateProj, ex1.upProj = saved
        return y

    E.profileBegin()
    far = E.toHost(forward_far())
    prof = [n for n, _, _ in E.profileEnd()]
    # (weights seen through pending views stay out of the MoE group: the two
    # shared SwiGLU GEMMs run as their own two-segment launch)
    assert any(n.startswith("gemm_lds_swiglu{128,128}") for n in prof), prof
    np.testing.assert_array_equal(far, near)

    # the routed grouped GEMM: expert 5's up weight read 2 GiB past a copy
    # of its gate weight
    rt = host["routed"][5]
    big, R, _ = far_apart([rt[0], rt[2]])
    start = moe.sharedExperts[0].forward(xt)
    topW, topI = moe.route(xt)
    ref = E.toHost(E.moeRoutedFfn(xt, start, topW, topI, moe.routedExperts,
                                  list(range(16)), 16))
    lib = _lib.load()
    out = E.empty(DType.BFLOAT16, xt.shape)
    a, keep = E._moe_args(xt, start, topW, topI, moe.routedExperts, list(range(16)), 16, out)
    gp = E.devicePtr(big)
    up = gp + R * rt[0].shape[1] * 2
    C.cast(a.gate_w, C.POINTER(C.c_void_p))[5] = gp
    C.cast(a.up_w, C.POINTER(C.c_void_p))[5] = up
    assert lib.rew_mi355x_moe_routed_ffn(E.context(), C.byref(a)) == 0, lib.rew_mi355x_last_error()
    np.testing.assert_array_equal(E.toHost(out), ref)


def test_moe_routing_weights(gpu, oracle):
    """topK + renormalisation of the router (deepseek.nim:132-137): the
    renormalised weights sum to 1 per token and every id is distinct."""
    keys = rng.split(rng.initKey(0x5EED0205), 2)
    T, H, E_ = 512, 128, 64
    x = oracle.round_bf16(rng.normalF32(keys[0], T * H).reshape(T, H))
    wr = rng.normalF32(keys[1], H * E_, 0.0, 0.02).reshape(H, E_)
    router = nn.Linear(E.fromHost(wr), E.fromHost(np.zeros(E_, np.float32)))
    m = nn.DeepSeekMoE(router, [], [], 6)
    tw, ti = m.route(E.fromHost(x, DType.BFLOAT16))
    tw, ti = E.toHost(tw), E.toHost(ti)
    np.testing.assert_allclose(tw.sum(1), 1.0, rtol=1e-6)
    assert all(len(set(r)) == 6 for r in ti)
    assert np.all(np.diff(tw, axis=1) <= 0)


class _TransposedLinear(nn.Linear):
    """Linear.forward over a weight stored [out, in]: the transposed view is
    made inside forward, so it is a pending view nobody holds."""

    def forward(self, x):
        xw = O.matmul(x, O.transpose(self.weight, [1, 0]))
        return O.add(xw, O.broadcastTo(self.bias, xw.shape, [1]))


@pytest.mark.parametrize("which", ["down", "gate", "held"])
def test_moe_unlowerable_weight_falls_back(gpu, oracle, which):
    """Expert 3's gate or down weight seen through a transposed view.
    * down / gate: the view is made inside forward, pending and unheld.
      Expert 3 keeps its SwiGLU and bias-GEMM plans, so the chain matches,
      but the grouped GEMM cannot read the view in place: the chain must not
      be claimed by the MoE lowering and runs through the ordinary GEMMs.
    * held: a view the caller holds is materialized densely, so the whole
      chain stays one routed group.
    Each way the flush succeeds with the op-by-op values."""
    moe, host = build_moe(oracle, 64, 128, 64, 8, 2, 1, 0x5EED0305)
    ex = moe.routedExperts[3]
    attr = "gateProj" if which == "gate" else "downProj"
    w = host["routed"][3][0 if which == "gate" else 4]
    wt = E.fromHost(np.ascontiguousarray(w.T), DType.BFLOAT16)
    bias = getattr(ex, attr).bias
    if which == "held":
        setattr(ex, attr, nn.Linear(O.transpose(wt, [1, 0]), bias))
    else:
        setattr(ex, attr, _TransposedLinear(wt, bias))
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    E.profileBegin()
    got = E.toHostF32(moe.forward(xt))
    prof = E.profileEnd()
    groups = sum(c for n, c, _ in prof if n.startswith("moe_gemm_swiglu"))
    assert groups == (1 if which == "held" else 0), [n for n, _, _ in prof]
    E.setMode(1)
    try:
        dense = E.toHostF32(moe.forward(xt))
    finally:
        E.setMode(0)
    np.testing.assert_array_equal(got, dense)
    want, _, _ = oracle.deepseek_moe(host["x"], host["shared"], host["routed"], host["wr"],
                                     host["br"], 2)
    assert np.linalg.norm(got - want) / np.linalg.norm(want) <= 2e-2


@pytest.mark.parametrize("T", [256, 37])
def test_direct_routed_ffn_equals_graph_lowering(gpu, oracle, T):
    """rew_mi355x_moe_routed_ffn on the router's top-k and the shared
    experts' sum gives the same bits as the deferred graph's lowering of
    DeepSeekMoE.forward's dense chain (both run the same kernels)."""
    moe, host = build_moe(oracle, T, 256, 128, 16, 4, 2, 0x5EED0405 + T)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    graph = E.toHost(moe.forward(xt))
    start = O.add(moe.sharedExperts[0].forward(xt), moe.sharedExperts[1].forward(xt))
    topW, topI = moe.route(xt)
    E.profileBegin()
    direct = E.toHost(E.moeRoutedFfn(xt, start, topW, topI, moe.routedExperts,
                                     list(range(16)), 16))
    names = [n for n, _, _ in E.profileEnd()]
    assert any(n.startswith("moe_gemm_swiglu") for n in names), names
    np.testing.assert_array_equal(direct, graph)
    # a chain of some experts only: the others' routed rows add nothing
    sub = [3, 7, 11]
    part = E.toHostF32(E.moeRoutedFfn(xt, start, topW, topI,
                                      [moe.routedExperts[e] for e in sub], sub, 16))
    tw, ti = E.toHost(topW), E.toHost(topI)
    want = E.toHostF32(start)
    for e in sub:
        ex = host["routed"][e]
        w = np.where(ti == e, tw, 0).sum(1, dtype=np.float32)[:, None]
        y = oracle.gated_ffn(host["x"], *ex, True)
        want = oracle.round_bf16(want + oracle.round_bf16(y * w))
    err = np.linalg.norm(part - want) / np.linalg.norm(want)
    assert err <= 2e-2


@pytest.mark.parametrize("T,E_,chain", [
    (37, 16, [0, 2, 3, 5, 8, 9, 13, 15]),
    (300, 16, [0, 2, 3, 5, 8, 9, 13, 15]),
    # 1094 blocks of 256 tokens x 60 members: past the placement's fused
    # count-table limit (65536 entries), so the block prefixes run as their
    # own launch
    (280000, 64, [e for e in range(64) if e % 16 != 7]),
])
def test_direct_routed_ffn_repeated_and_off_chain_ids(gpu, oracle, T, E_, chain):
    """Top-k tables a router never produces, through the C-ABI entry point:
    a repeated id (its rows computed once and weighted by the sum of its
    slots' weights, as routedWeightForExpert sums topWeights * (ids == e)),
    ids outside [0, width) and ids of experts off the chain (no
    contribution).  Equal bit for bit to rew's dense chain over the same
    tables, evaluated op by op."""
    moe, host = build_moe(oracle, T, 256, 128, E_, 4, 1, 0x5EED0705 + T)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    start = moe.sharedExperts[0].forward(xt)
    g = np.random.default_rng(T)
    ti = np.argsort(g.random((T, E_)), axis=1)[:, :4].astype(np.int32)  # distinct
    ti[::5, 1] = ti[::5, 0]          # one repeated pair (at most two equal ids)
    ti[::7, 2] = -1                  # outside the router width
    ti[::11, 3] = E_ + 3
    tw = (g.random((T, 4), dtype=np.float32) + np.float32(0.05)).astype(np.float32)
    topW, topI = E.fromHost(tw), E.fromHost(ti)
    experts = [moe.routedExperts[e] for e in chain]
    direct = E.toHost(E.moeRoutedFfn(xt, start, topW, topI, experts, chain, E_))
    E.setMode(1)
    try:
        out = start
        for e in chain:
            w = nn.routedWeightForExpert(topW, topI, e)
            wB = O.broadcastTo(O.unsqueeze(w, 1), list(xt.shape), [0, 1])
            y = O.astype(moe.routedExperts[e].forward(xt), DType.FLOAT32)
            out = O.add(out, O.astype(O.mul(y, wB), DType.BFLOAT16))
        dense = E.toHost(out)
    finally:
        E.setMode(0)
    assert np.isfinite(E.toHostF32(out)).all()
    np.testing.assert_array_equal(direct, dense)


def test_direct_routed_ffn_rejects_bad_arguments(gpu, oracle):
    moe, host = build_moe(oracle, 16, 128, 64, 8, 2, 0, 0x5EED0505)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    topW, topI = moe.route(xt)
    start = O.zerosLike(xt)
    with pytest.raises(E.EagerError, match="repeated"):
        E.moeRoutedFfn(xt, start, topW, topI, moe.routedExperts[:2], [1, 1], 8)
    with pytest.raises(E.EagerError, match="outside"):
        E.moeRoutedFfn(xt, start, topW, topI, moe.routedExperts[:1], [8], 8)


DENSE_CHILD = r"""
import json, os, sys
import numpy as np
root = sys.argv[1]
for p in (root, root + "/tests", root + "/oracle"):
    sys.path.insert(0, p)
import oracle as orc
from test_gpu_moe import build_moe, inf_expert
from rew_amd import eager as E
from rew_amd.eager import DType
E.installEagerBackend(E.mi355x(0))
moe, host = build_moe(orc, 64, 128, 64, 8, 2, 1, 0x5EED0606)
inf_expert(moe, 3)
xt = E.fromHost(host["x"], DType.BFLOAT16)
E.profileBegin()
got = E.toHostF32(moe.forward(xt))
names = [n for n, _, _ in E.profileEnd()]
E.setMode(E.MODE_OP_BY_OP)
ref = E.toHostF32(moe.forward(xt))
E.setMode(E.MODE_DEFERRED)
print(json.dumps({"names": names, "equal": bool(np.array_equal(got, ref, equal_nan=True)),
                  "finite_rows": int(np.all(np.isfinite(got), axis=1).sum())}))
"""


def inf_expert(moe, e):
    """Routed expert e's down projection gets a bias of +inf (bf16 0x7F80), so
    its output is inf on every token."""
    d = moe.routedExperts[e].downProj
    H = d.weight.shape[1]
    d.bias = E.fromHost(np.full(H, 0x7F80, np.uint16), DType.BFLOAT16)


def test_dense_moe_switch_keeps_rews_nonfinite_semantics(gpu, oracle):
    """REW_MI355X_DENSE_MOE=1 runs DeepSeekMoE's expert loop as written: with
    one routed expert overflowing, every token's dense sum picks up
    bf16(inf * 0) = NaN from it, exactly as the op-by-op chain does.  By
    default the routed rewrite evaluates that expert only on its own tokens,
    so the other tokens stay finite (the documented difference)."""
    import json
    import os
    import subprocess
    import sys
    from pathlib import Path
    root = Path(__file__).resolve().parents[1]
    env = dict(os.environ, REW_MI355X_DENSE_MOE="1")
    r = subprocess.run([sys.executable, "-c", DENSE_CHILD, str(root)], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert not any(n.startswith("moe_gemm") or n.startswith("moe_combine")
                   for n in res["names"]), res["names"]
    assert res["equal"] and res["finite_rows"] == 0, res
    moe, host = build_moe(oracle, 64, 128, 64, 8, 2, 1, 0x5EED0606)
    inf_expert(moe, 3)
    E.profileBegin()
    got = E.toHostF32(moe.forward(E.fromHost(host["x"], DType.BFLOAT16)))
    names = [n for n, _, _ in E.profileEnd()]
    assert any(n.startswith("moe_gemm_swiglu") for n in names), names
    _, ids = moe.route(E.fromHost(host["x"], DType.BFLOAT16))
    off = ~np.any(E.toHost(ids) == 3, axis=1)
    assert off.any() and np.all(np.isfinite(got[off])), int(off.sum())


@pytest.mark.parametrize("T,H,E_,k,bf16", [(8192, 2048, 64, 6, True), (200, 128, 16, 4, True),
                                           (77, 256, 60, 3, False), (300, 1024, 64, 8, False),
                                           # H % 128 != 0: the 16-row narrow form
                                           (50, 192, 32, 2, True)])
def test_router_one_launch(gpu, T, H, E_, k, bf16):
    """DeepSeekMoE.route (deepseek.nim:132-137): the router Linear on
    astype(x, f32), softmax, topK and the renormalisation run as one launch
    (and topK of the softmax alone, without the renormalisation, too), equal
    to the op-by-op kernels bit for bit: the same fmaf chain per logit, the
    softmax and the ranking in the same order, the renormalising sum in rank
    order.  A row of x holding NaN ranks its NaN probabilities last."""
    rs = np.random.default_rng(T + E_)
    x = rs.standard_normal((T, H)).astype(np.float32)
    x[3, 5] = np.nan
    wr = (rs.standard_normal((H, E_)) * 0.05).astype(np.float32)
    br = (rs.standard_normal(E_) * 0.1).astype(np.float32)
    if bf16:
        xt = E.fromHost(E.f32_to_bf16_bits(x), DType.BFLOAT16)
    else:
        xt = E.fromHost(x)
    m = nn.DeepSeekMoE(nn.Linear(E.fromHost(wr), E.fromHost(br)), [], [], k)

    def route():
        tw, ti = m.route(xt)
        return E.toHost(tw), E.toHost(ti)

    def raw():
        tv, ti = O.topK(nn.softmax(m.gate.forward(nn._f32(xt)), 1), k, 1, True)
        return E.toHost(tv), E.toHost(ti)

    for fn, tag in ((route, ",norm}"), (raw, "}")):
        E.profileBegin()
        got = fn()
        names = [n for n, _, _ in E.profileEnd()]
        assert names == [f"moe_router{{{T}x{H}x{E_},k{k}{tag}"], names
        E.setMode(E.MODE_OP_BY_OP)
        try:
            ref = fn()
        finally:
            E.setMode(E.MODE_DEFERRED)
        np.testing.assert_array_equal(got[1], ref[1])
        np.testing.assert_array_equal(got[0].view(np.uint32), ref[0].view(np.uint32))
        assert np.all(np.isnan(got[0][3]))
