"""GPU checks of the flush-plan cache (the per-graph analogue of rew's
executable cache, src/rew/eager.nim:1620-1680).

The first flush of a graph is lowered and recorded; a later flush with the
same signature replays the recorded launches over its own buffers.  These
tests check that a replay over new inputs equals a fresh lowering of the
same inputs bit for bit (rew_mi355x_clear_cache drops the plans, so the
next flush lowers anew), that it launches the same kernels, and that graphs
differing only in what the lowering reads (which leaves are the same
tensor, the value of a host constant, which results the caller holds, the
execution mode) are not confused.
"""
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import jit as J
from rew_amd import nn
from rew_amd import ops as O
from rew_amd.eager import DType

from test_gpu_composites import _llama_params
from test_gpu_moe import build_moe

ROOT = Path(__file__).resolve().parents[1]


def f32(x):
    return E.fromHost(np.asarray(x, np.float32))


def scalar_like(v, t):
    """A host scalar broadcast to t's shape, as rew's composites build them."""
    return O.broadcastTo(O.scalarF32(float(v)), list(t.shape), [])


def small_layer(oracle):
    B, S, H, nh, nkv, I = 2, 64, 256, 4, 2, 512
    key = oracle.init_key(0x5EED0A01)
    p, m = _llama_params(oracle, key, H, nh, nkv, I)
    hd = H // nh
    rope = nn.RotaryPositionEncoding.init(hd, S, 500000.0)
    layer = nn.LlamaDecoderLayer(
        nn.GroupedQueryAttention(m["q"], m["k"], m["v"], m["o"], nh, nkv, hd, rope),
        nn.GatedFeedForward(m["g"], m["u"], m["d"]),
        nn.RMSNorm(E.fromHost(p["g1"]), 1e-5), nn.RMSNorm(E.fromHost(p["g2"]), 1e-5))
    xs = [oracle.round_bf16(oracle.normal_f32(oracle.fold_in(key, 100 + i), B * S * H)
                            .reshape(B, S, H)) for i in range(3)]
    return layer, xs


def test_layer_replay_equals_fresh_lowering(gpu, oracle):
    layer, xs = small_layer(oracle)
    xt = [E.fromHost(x, DType.BFLOAT16) for x in xs]
    E.clearEagerCache()
    E.resetStats()
    got = [E.toHost(layer.forward(x, causal=True)) for x in xt]
    s = E.stats()
    assert s["flush_plan_hits"] >= 2, s
    assert s["flush_host_ns"] > 0, s
    for x, g in zip(xt, got):
        E.clearEagerCache()
        np.testing.assert_array_equal(g, E.toHost(layer.forward(x, causal=True)))
    # the inputs differ, so a replay reading the recorded flush's buffers
    # would have repeated its output
    assert not np.array_equal(got[1], got[2])


def test_replay_launches_the_recorded_kernels(gpu, oracle):
    layer, xs = small_layer(oracle)
    xt = [E.fromHost(x, DType.BFLOAT16) for x in xs[:2]]
    E.clearEagerCache()
    runs = []
    for x in xt:
        E.resetStats()
        E.profileBegin()
        y = layer.forward(x, causal=True)
        E.flush()
        names = [n for n, _, _ in E.profileEnd()]
        runs.append((names, E.stats()))
        del y
    (rec_names, rec), (rep_names, rep) = runs
    assert rec["flush_plan_hits"] == 0 and rep["flush_plan_hits"] >= 1
    assert rec_names == rep_names
    assert any(n.startswith("flash_attn") for n in rep_names), rep_names
    assert rec["kernels_launched"] == rep["kernels_launched"]
    assert rec["fused_groups"] == rep["fused_groups"]
    print(f"host time per flush: recorded {rec['flush_host_ns'] / 1e3:.0f} us, "
          f"replayed {rep['flush_host_ns'] / 1e3:.0f} us")


def test_lazy_moe_replays(gpu, oracle):
    T, H, I, E_, k, S = 256, 256, 128, 16, 4, 2
    moe, host = build_moe(oracle, T, H, I, E_, k, S, 0x5EED0A02)
    params = nn.moeParams(moe)
    lz = J.lazy(lambda a: [nn.moeFromParams(a[1:], S, E_, k).forward(a[0])], "planCacheMoE")
    x2 = oracle.round_bf16(np.roll(host["x"], 7, axis=0) * np.float32(0.5))
    xt = [E.fromHost(host["x"], DType.BFLOAT16), E.fromHost(x2, DType.BFLOAT16)]
    E.clearEagerCache()
    E.resetStats()
    got = [E.toHost(lz.call([x] + params)[0]) for x in xt]
    assert E.stats()["flush_plan_hits"] >= 1
    for x, g in zip(xt, got):
        E.clearEagerCache()
        np.testing.assert_array_equal(g, E.toHost(lz.call([x] + params)[0]))
        np.testing.assert_array_equal(g, E.toHost(moe.forward(x)))


def test_same_tensor_twice_is_another_graph(gpu):
    rng = np.random.default_rng(5)
    a = rng.standard_normal((64, 128)).astype(np.float32)
    b = rng.standard_normal((64, 128)).astype(np.float32)
    ta, tb = f32(a), f32(b)
    E.clearEagerCache()
    f = lambda x, y: O.add(O.mul(x, y), x)
    for x, y, want in [(ta, tb, a * b + a), (ta, ta, a * a + a), (tb, ta, b * a + b),
                       (tb, tb, b * b + b)]:
        np.testing.assert_array_equal(E.toHost(f(x, y)), want)


def test_host_constants_are_part_of_the_signature(gpu):
    x = np.linspace(-3, 3, 4096, dtype=np.float32).reshape(32, 128)
    tx = f32(x)
    E.clearEagerCache()
    for c in (2.0, 3.0, 2.0, -0.5):
        y = O.add(O.mul(tx, scalar_like(c, tx)), scalar_like(1.0, tx))
        np.testing.assert_array_equal(E.toHost(y), x * np.float32(c) + np.float32(1.0))


def test_held_intermediate_changes_the_plan(gpu):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((128, 256)).astype(np.float32)
    tx = f32(x)
    E.clearEagerCache()
    want_h = np.exp(x * np.float32(0.5))
    for hold in (False, True, False, True):
        h = O.exp(O.mul(tx, scalar_like(0.5, tx)))
        y = O.reduceSum(h, [1])
        if not hold:  # the exp is then only a prologue of the reduction
            del h
        np.testing.assert_allclose(E.toHost(y), want_h.sum(1), rtol=1e-5)
        if hold:
            np.testing.assert_allclose(E.toHost(h), want_h, rtol=1e-6)
            del h


def test_op_by_op_mode_replays(gpu):
    rng = np.random.default_rng(7)
    E.clearEagerCache()
    E.setMode(1)
    try:
        for _ in range(3):
            a = rng.standard_normal((256, 64)).astype(np.float32)
            ta = f32(a)
            y = O.maximum(O.add(ta, ta), scalar_like(0.0, ta))
            np.testing.assert_array_equal(E.toHost(y), np.maximum(a + a, 0))
    finally:
        E.setMode(0)


CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from rew_amd import eager as E, ops as O
E.installEagerBackend(E.mi355x(0))
x = E.fromHost(np.arange(4096, dtype=np.float32).reshape(64, 64))
outs = [E.toHost(O.mul(O.add(x, x), x)) for _ in range(3)]
s = E.stats()
print(json.dumps({"hits": s["flush_plan_hits"], "flushes": s["flushes"],
                  "same": all(np.array_equal(o, outs[0]) for o in outs)}))
"""


def test_plan_cache_switch(gpu):
    res = {}
    for val in ("0", "1"):
        env = dict(os.environ, REW_MI355X_PLAN_CACHE=val)
        r = subprocess.run([sys.executable, "-c", CHILD, str(ROOT)], env=env,
                           capture_output=True, text=True, timeout=300)
        assert r.returncode == 0, r.stderr[-3000:]
        res[val] = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["0"]["hits"] == 0 and res["0"]["same"], res
    assert res["1"]["hits"] == 2 and res["1"]["same"], res
