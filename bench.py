#!/usr/bin/env python3
"""Throughput of rew's eager hot path on one MI355X through the mi355x backend.

Default workload (the headline metric): one Llama-style decoder layer prefill,
bf16, B=4 x S=2048 tokens, hidden 4096, 32 query / 8 KV heads (GQA), head dim
128, RoPE theta 500000, RMSNorm eps 1e-5, SwiGLU intermediate 14336, token
embeddings gathered from a [128256, 4096] table with uniform random ids.
A step is: torchIndexSelect(table, ids) -> LlamaDecoderLayer.forward, driven
through the same eager op sequence rew's nn layers emit (rew_amd.nn), with
every input already resident in HBM.

Other workloads (``--workload``) are the remaining configurations of the
hot path, each measured the same way: ``chain`` (fp32 elementwise +
reductions + softmax + RMSNorm, HBM-bound), ``swiglu`` (the gated FFN,
MFMA-bound), ``mnist`` (MLP inference with argmax, latency-bound), ``moe``
(DeepSeek-style routed MoE layer) and ``copy`` (a plain streaming kernel of
known size, the calibration for the HBM byte counters).

Prints ONE JSON line with the metric (from a timed pass of K steps), a
roofline object for the dominant kernel (its launches timed by HIP events on
the backend's own stream over a second, profiled pass of the same K steps),
a cpu_baseline (the CPU restatement in oracle/ timed on this host's cores on
a bounded sample) and a parity object: after the timed passes, one more step
of the same workload is read back and compared with that cpu_baseline's own
oracle output on the sample (bit-exact for index and byte results, within
the stated tolerance for floating point).  The default llama run also
measures the other configurations (MNIST, the chain, the SwiGLU FFN, the
MoE layer) the same way and carries their records under "configs".
"""
from __future__ import annotations

import argparse
import ctypes as C
import json
import os
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

from rew_amd import eager as E  # noqa: E402
from rew_amd import nn, rng  # noqa: E402
from rew_amd import ops as O  # noqa: E402
from rew_amd.eager import DType  # noqa: E402

HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
BF16_PEAK_TFLOPS = 2516.6      # MI355X dense bf16 MFMA, TFLOP/s
FP32_PEAK_TFLOPS = 157.3       # MI355X fp32 vector, TFLOP/s
TRAFFIC_FILE = ROOT / "profiles" / "traffic.json"

# C4 shape (the reference's LlamaDecoderLayer / GroupedQueryAttention / GatedFeedForward)
C4 = dict(batch=4, seq_len=2048, hidden=4096, heads=32, kv_heads=8, head_dim=128,
          intermediate=14336, vocab=128256, rope_theta=500000.0, eps=1e-5)


def llama_layer_flops(B, S, H, nh, nkv, hd, I, causal=True):
    """Algorithmic FLOPs of one decoder layer (2 per multiply-add)."""
    T = B * S
    proj = 2 * T * H * (nh * hd + 2 * nkv * hd) + 2 * T * nh * hd * H
    ffn = 2 * T * H * I * 3
    # QK^T and PV over the visible (query, key) pairs
    pairs = S * (S + 1) // 2 if causal else S * S
    attn = 2 * 2 * B * nh * pairs * hd
    return proj + attn + ffn


# ---- timing ---------------------------------------------------------------------------------

class HipEvents:
    """HIP events recorded on the backend's stream (not torch's)."""

    def __init__(self, stream):
        self.hip = C.CDLL("libamdhip64.so")
        self.stream = stream

    def event(self):
        ev = C.c_void_p()
        rc = self.hip.hipEventCreate(C.byref(ev))
        if rc != 0:
            raise RuntimeError(f"hipEventCreate failed ({rc})")
        return ev

    def record(self, ev):
        rc = self.hip.hipEventRecord(ev, C.c_void_p(self.stream))
        if rc != 0:
            raise RuntimeError(f"hipEventRecord failed ({rc})")

    def elapsed_ms(self, a, b):
        self.hip.hipEventSynchronize(b)
        ms = C.c_float()
        rc = self.hip.hipEventElapsedTime(C.byref(ms), a, b)
        if rc != 0:
            raise RuntimeError(f"hipEventElapsedTime failed ({rc})")
        return float(ms.value)


def backend_stream():
    s = C.c_void_p()
    rc = E._lib.load().rew_mi355x_stream(E.context(), C.byref(s))
    if rc != 0:
        raise RuntimeError("rew_mi355x_stream failed")
    return s.value


def kernel_symbol(entry_name: str) -> str:
    return entry_name.split("[")[0].split("{")[0].split("+")[0]


def timed_run(step, steps, warmup):
    """First call, warmup, then two passes of `steps` steps, each bracketed by
    sync on both sides:

    1. the profiled pass: every kernel launch bracketed by HIP events on the
       backend stream (rew_mi355x_profile_*), which gives per-kernel
       durations for the roofline and the breakdown.  The per-launch events
       add gaps between kernels, so this pass is not the one timed;
    2. the timed pass: wall clock and HIP events at its two ends only; it
       gives `value` and ms_per_step.

    Returns (wall_s, device_ms, first_ms, profile entries, host counters);
    wall and device time are the timed pass's.  The host counters are the
    timed pass's flush host time per step (lowering or replay of a recorded
    plan, plus enqueueing) and how many of its flushes replayed a plan."""
    t0 = time.perf_counter()
    y = step()
    E.sync()
    first_ms = (time.perf_counter() - t0) * 1e3
    del y
    for _ in range(warmup):
        step()
    E.sync()
    ev = HipEvents(backend_stream())
    e0, e1 = ev.event(), ev.event()

    def run(profiled):
        outs = []
        E.sync()
        if profiled:
            E.profileBegin()
        t0 = time.perf_counter()
        ev.record(e0)
        for _ in range(steps):
            outs.append(step())
            if len(outs) > 2:
                outs.pop(0)
        ev.record(e1)
        E.sync()
        wall = time.perf_counter() - t0
        prof = E.profileEnd() if profiled else None
        outs.clear()
        return wall, ev.elapsed_ms(e0, e1), prof

    pwall, _, prof = run(True)
    s0 = E.stats()
    wall, dev_ms, _ = run(False)
    s1 = E.stats()
    hostc = {"flush_host_us_per_step": round((s1["flush_host_ns"] - s0["flush_host_ns"]) / 1e3 /
                                             steps, 1),
             "flushes": s1["flushes"] - s0["flushes"],
             "flush_plan_hits": s1["flush_plan_hits"] - s0["flush_plan_hits"]}
    for name, n, ms in sorted(prof, key=lambda r: -r[2]):
        print(f"#   {ms * 1e3 / steps:9.1f} us/step  x{n // steps:<3d} {name}", file=sys.stderr)
    print(f"#   timed pass {wall * 1e3 / steps:.3f} ms/step, profiled pass "
          f"{pwall * 1e3 / steps:.3f} ms/step; flush host time "
          f"{hostc['flush_host_us_per_step']} us/step, {hostc['flush_plan_hits']} of "
          f"{hostc['flushes']} flushes replayed a recorded plan", file=sys.stderr)
    return wall, dev_ms, first_ms, prof, hostc


def by_symbol(prof, work_of, by_shape=False):
    """Groups profile entries by kernel symbol: launches, ms and the summed
    algorithmic work (work_of(entry name) -> units, or None if unknown).
    by_shape: one group per entry name (symbol and launch shape), so that
    launches of one symbol over different sizes are not averaged together."""
    out = {}
    for name, n, ms in prof:
        d = out.setdefault(name if by_shape else kernel_symbol(name),
                           {"launches": 0, "ms": 0.0, "work": 0, "known": True,
                            "symbol": kernel_symbol(name)})
        d["launches"] += n
        d["ms"] += ms
        w = work_of(name)
        if w is None:
            d["known"] = False
        else:
            d["work"] += w * n
    return out


def traffic_for(workload, kernel):
    """HBM bytes per launch of `kernel` in `workload` from the committed
    rocprofv3 FETCH_SIZE / WRITE_SIZE runs (profiles/traffic.json), or None."""
    try:
        data = json.loads(TRAFFIC_FILE.read_text())
    except (OSError, ValueError):
        return None
    rec = data.get(f"{workload}:{kernel}")
    return None if rec is None else int(rec["bytes_per_launch"])


def roofline(workload, syms, bound):
    """Roofline object of the kernel with the largest summed duration."""
    _, d = max(syms.items(), key=lambda kv: kv[1]["ms"])
    ksym = d["symbol"]
    avg_ms = d["ms"] / d["launches"]
    peak, unit = (BF16_PEAK_TFLOPS, "TFLOP/s") if bound == "mfma" else (HBM_PEAK_GBS, "GB/s")
    roof = {"bound": bound, "kernel": ksym, "achieved": None, "peak": peak, "unit": unit,
            "frac": None, "traffic": traffic_for(workload, ksym),
            "avg_launch_us": round(avg_ms * 1e3, 2), "launches": d["launches"]}
    if d["known"]:
        per_launch = d["work"] / d["launches"]
        scale = 1e12 if bound == "mfma" else 1e9
        achieved = per_launch / (avg_ms * 1e-3) / scale
        roof["achieved"] = round(achieved, 1)
        roof["frac"] = round(achieved / peak, 4)
        roof["algorithmic_" + ("flops" if bound == "mfma" else "bytes") + "_per_launch"] = \
            int(per_launch)
    return roof


def breakdown(syms, steps):
    return sorted(((k, round(v["ms"] / steps, 3), v["launches"] // steps)
                   for k, v in syms.items()), key=lambda r: -r[1])


def record(args, metric, value, unit, ms_per_step, dtype, config, roof, cpu, parity, extra,
           hib=True, steps=None, warmup=None):
    """One workload's result: the contract's fields plus `parity` (the same
    run's outputs compared with the oracle on a sample) and `extra`."""
    rec = {"metric": metric, "value": round(value, 3 if value < 1000 else 1), "unit": unit,
           "n_gpus": 1, "steps": args.steps if steps is None else steps,
           "warmup": args.warmup if warmup is None else warmup,
           "ms_per_step": round(ms_per_step, 4), "higher_is_better": hib, "scaling": "weak",
           "vs_baseline": None, "dtype": dtype,
           "data": "synthetic (rew Threefry normalF32/uniformF32 inputs, random-init weights)",
           "config": config, "roofline": roof, "cpu_baseline": cpu, "parity": parity}
    rec.update(extra)
    return rec


def normwise(got, want) -> float:
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    return float(np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-300))


def max_rel(got, want) -> float:
    """Largest elementwise |got - want| / |want| (pairs where both are 0 count as 0)."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    den = np.abs(want)
    diff = np.abs(got - want)
    rel = np.where(den > 0, diff / np.where(den > 0, den, 1.0), np.where(diff > 0, np.inf, 0.0))
    return float(rel.max()) if rel.size else 0.0


def parity_obj(checks, sample):
    """`checks`: name -> (error, tolerance, kind).  ok = every error within its
    tolerance; a tolerance of None marks a figure that is reported only."""
    out = {"ok": all(e <= t for e, t, _ in checks.values() if t is not None), "sample": sample}
    for name, (e, t, kind) in checks.items():
        out[name] = {"err": e if isinstance(e, int) else float(f"{e:.3e}"), "tol": t,
                     "kind": kind}
    return out


def oracle_mod():
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc
    orc.build()
    return orc


# ---- C4: Llama decoder layer prefill -------------------------------------------------------

def visible_pairs(Sq: int, Sk: int, cmp: int) -> int:
    """(query, key) pairs a mask predicate cmp(i, j) keeps; -1 = no mask."""
    if cmp == -1:
        return Sq * Sk
    i = np.arange(Sq)[:, None]
    j = np.arange(Sk)[None, :]
    pred = {0: i == j, 1: i != j, 2: i < j, 3: i <= j, 4: i > j, 5: i >= j}[cmp]
    return int(pred.sum())


def entry_flops(entry_name: str) -> int | None:
    """Algorithmic FLOPs of one launch from its profile name:
    "<gemm variant>[b,M,N,K]" -> 2bMNK; "flash_attn[B,H,Hkv,Sq,Sk,D,cmp,skip]"
    -> 4*B*H*D*(visible pairs) (QK^T and PV over the pairs the mask keeps)."""
    if "[" not in entry_name:
        return None
    dims = [int(v) for v in entry_name[entry_name.index("[") + 1:entry_name.index("]")].split(",")]
    if entry_name.startswith("flash_attn"):
        B, H, _, Sq, Sk, D, cmp, _ = dims
        return 4 * B * H * D * visible_pairs(Sq, Sk, cmp)
    if entry_name.startswith("moe_gemm"):
        _, rows, n, k = dims  # [groups, rows (routed, then shared), N, K]
        return (4 if "swiglu" in entry_name else 2) * rows * n * k
    b, m, n, k = dims
    # the SwiGLU kernel runs the gate and up projections over the same A
    return (4 if "swiglu" in entry_name else 2) * b * m * n * k


def build_llama(cfg, seed=0x5EED0004, norm="rms"):
    """Weights ~N(0, 0.02) bf16, zero biases, gammas ~N(1, 0.1) f32, keyed per
    tensor in declaration order from initKey(seed).  norm "rms" gives the
    config's RMSNorm; "layer" gives rew's own LayerNorm (llama.nim:32-33) with
    those gammas and zero betas."""
    H, nh, nkv, hd, I = (cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                         cfg["intermediate"])
    V = cfg["vocab"]
    keys = rng.split(rng.initKey(seed), 12)
    host = {}

    def lin(k, name, fi, fo):
        w = rng.normalF32(k, fi * fo, 0.0, 0.02).reshape(fi, fo)
        wb = E.f32_to_bf16_bits(w)
        host["w" + name] = wb
        host["b" + name] = np.zeros(fo, np.float32)
        return nn.Linear(E.fromHost(wb, DType.BFLOAT16),
                         E.fromHost(np.zeros(fo, np.uint16), DType.BFLOAT16))

    m = {}
    for i, (n, fi, fo) in enumerate([("q", H, nh * hd), ("k", H, nkv * hd),
                                     ("v", H, nkv * hd), ("o", nh * hd, H),
                                     ("g", H, I), ("u", H, I), ("d", I, H)]):
        m[n] = lin(keys[i], n, fi, fo)
    host["g1"] = rng.normalF32(keys[7], H, 1.0, 0.1)
    host["g2"] = rng.normalF32(keys[8], H, 1.0, 0.1)
    table = E.f32_to_bf16_bits(rng.normalF32(keys[9], V * H, 0.0, 0.02)).reshape(V, H)
    S = cfg["seq_len"]
    ids = rng.tokenIds(keys[10], cfg["batch"] * S, V)
    rope = nn.RotaryPositionEncoding.init(hd, S, cfg["rope_theta"])
    if norm == "rms":
        n1 = nn.RMSNorm(E.fromHost(host["g1"]), cfg["eps"])
        n2 = nn.RMSNorm(E.fromHost(host["g2"]), cfg["eps"])
    else:
        zero = np.zeros(H, np.float32)
        n1 = nn.LayerNorm(E.fromHost(host["g1"]), E.fromHost(zero), [H], cfg["eps"])
        n2 = nn.LayerNorm(E.fromHost(host["g2"]), E.fromHost(zero), [H], cfg["eps"])
    layer = nn.LlamaDecoderLayer(
        nn.GroupedQueryAttention(m["q"], m["k"], m["v"], m["o"], nh, nkv, hd, rope),
        nn.GatedFeedForward(m["g"], m["u"], m["d"]), n1, n2)
    emb = nn.Embedding(E.fromHost(table, DType.BFLOAT16))
    return layer, emb, E.fromHost(ids), host, table, ids


def cpu_baseline_llama(cfg, host, table, ids, seqs, norm):
    """The oracle's restatement of the same layer on a bounded sample: the
    first `seqs` of the batch's sequences, each a full S-token causal prefill.
    Returns (cpu_baseline, the oracle's output [seqs, S, H])."""
    orc = oracle_mod()
    nh, nkv, hd, S = cfg["heads"], cfg["kv_heads"], cfg["head_dim"], cfg["seq_len"]
    p = {}
    for n in "qkvogud":
        p["w" + n] = orc.from_bf16(host["w" + n])
        p["b" + n] = host["b" + n]
    p["g1"], p["g2"] = host["g1"], host["g2"]
    c, s = nn.rope_tables(hd, S, cfg["rope_theta"])
    x = orc.from_bf16(table[ids[:seqs * S]]).reshape(seqs, S, cfg["hidden"])
    t0 = time.perf_counter()
    want = orc.llama_layer(x, p, nh, nkv, c, s, cfg["eps"], True, True, norm)
    dt = time.perf_counter() - t0
    return ({"value": round(seqs * S / dt, 2), "unit": "tokens/s",
             "cores": int(orc.lib().orc_num_threads()), "kind": "port",
             "sample": f"{seqs} of the {cfg['batch']} sequences ({seqs * S} tokens, full "
                       f"hidden/FFN/head dims, causal), oracle/ C restatement with OpenMP, "
                       f"{dt:.1f} s"}, want)


def run_llama(args):
    cfg = dict(C4)
    B, S, H = cfg["batch"], cfg["seq_len"], cfg["hidden"]
    t0 = time.perf_counter()
    layer, emb, ids_t, host, table, ids = build_llama(cfg, norm=args.norm)
    E.sync()
    print(f"# inputs ready in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)

    def step():
        x = O.reshape(emb.lookup(ids_t), [B, S, H])
        y = layer.forward(x, causal=True)
        E.flush()
        return y

    wall, dev_ms, first_ms, prof, hostc = timed_run(step, args.steps, args.warmup)
    ms_per_step = wall * 1e3 / args.steps
    flops = llama_layer_flops(B, S, H, cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                              cfg["intermediate"])
    syms = by_symbol(prof, entry_flops)
    roof = roofline("llama" if args.norm == "rms" else "llama_layernorm", syms, "mfma")
    kernel_ms = sum(v["ms"] for v in syms.values()) / args.steps
    # parity, outside the timed region: one more step of the same workload
    # with the gathered embedding held, so both come back to the host
    x_t = O.reshape(emb.lookup(ids_t), [B, S, H])
    y_t = layer.forward(x_t, causal=True)
    x_dev = E.toHost(x_t).reshape(B * S, H)
    y_dev = E.toHostF32(y_t)
    del x_t, y_t
    emb_mismatch = int(np.count_nonzero(np.any(x_dev != table[ids], axis=1)))
    checks = {"embedding_rows": (emb_mismatch, 0, "rows of the gathered [8192,4096] bf16 "
                                 "embedding not bit-equal to table[ids]")}
    cpu = None
    sample = f"embedding: all {B * S} rows"
    if not args.no_cpu_baseline:
        cpu, want = cpu_baseline_llama(cfg, host, table, ids, args.cpu_seqs, args.norm)
        checks["layer_out"] = (normwise(y_dev[:args.cpu_seqs], want), 2e-2,
                               "normwise relative, bf16 layer output vs oracle")
        sample += (f"; layer output: sequences 0..{args.cpu_seqs - 1} ({args.cpu_seqs * S} "
                   f"tokens), the cpu_baseline's own oracle run")
    parity = parity_obj(checks, sample)
    config = {"workload": "llama_decoder_layer_prefill_bf16", "batch": B, "seq_len": S,
              "hidden": H, "heads": cfg["heads"], "kv_heads": cfg["kv_heads"],
              "head_dim": cfg["head_dim"], "intermediate": cfg["intermediate"],
              "vocab": cfg["vocab"], "rope_theta": cfg["rope_theta"], "causal": True,
              "norm": "rmsnorm" if args.norm == "rms" else "layernorm",
              "parallelism": "single-gpu"}
    extra = {"layer": {"algorithmic_tflop": round(flops / 1e12, 4),
                       "achieved_tflops": round(flops / (ms_per_step * 1e-3) / 1e12, 1),
                       "mfma_frac": round(flops / (ms_per_step * 1e-3) / 1e12 /
                                          BF16_PEAK_TFLOPS, 4),
                       "device_ms_per_step": round(dev_ms / args.steps, 3),
                       "kernel_ms_per_step": round(kernel_ms, 3),
                       "first_call_ms": round(first_ms, 1),
                       "host": hostc,
                       "kernels": breakdown(syms, args.steps)[:12]}}
    metric = ("llama_layer_prefill_tokens_per_s" if args.norm == "rms"
              else "llama_layer_layernorm_prefill_tokens_per_s")
    return record(args, metric, B * S * args.steps / wall, "tokens/s", ms_per_step, "bf16",
                  config, roof, cpu, parity, extra)


# ---- C3: SwiGLU gated FFN ------------------------------------------------------------------

def run_swiglu(args, steps=None, warmup=None):
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    T, H, I = 4096, 4096, 14336
    keys = rng.split(rng.initKey(0x5EED0003), 4)
    x = E.f32_to_bf16_bits(rng.normalF32(keys[0], T * H)).reshape(1, T, H)
    ws = [E.f32_to_bf16_bits(rng.normalF32(keys[1 + i], fi * fo, 0.0, 0.02)).reshape(fi, fo)
          for i, (fi, fo) in enumerate([(H, I), (H, I), (I, H)])]
    lins = [nn.Linear(E.fromHost(w, DType.BFLOAT16),
                      E.fromHost(np.zeros(w.shape[1], np.uint16), DType.BFLOAT16)) for w in ws]
    ffn = nn.GatedFeedForward(*lins)
    xt = E.fromHost(x, DType.BFLOAT16)
    E.sync()

    def step():
        y = ffn.forward(xt)
        E.flush()
        return y

    wall, dev_ms, first_ms, prof, hostc = timed_run(step, steps, warmup)
    ms = wall * 1e3 / steps
    flops = 2 * T * H * I * 3
    syms = by_symbol(prof, entry_flops)
    roof = roofline("swiglu", syms, "mfma")
    y_dev = E.toHostF32(step()).reshape(T, H)
    cpu, parity = None, None
    if not args.no_cpu_baseline:
        orc = oracle_mod()
        rows = np.arange(0, T, 16)           # 256 token rows spread over the batch
        xf = orc.from_bf16(x.reshape(T, H)[rows])
        wf = [orc.from_bf16(w) for w in ws]
        z = np.zeros(I, np.float32)
        t0 = time.perf_counter()
        want = orc.gated_ffn(xf, wf[0], z, wf[1], z, wf[2], np.zeros(H, np.float32), True)
        dt = time.perf_counter() - t0
        cpu = {"value": round(2 * len(rows) * H * I * 3 / dt / 1e12, 4), "unit": "TFLOP/s",
               "cores": int(orc.lib().orc_num_threads()), "kind": "port",
               "sample": f"{len(rows)} of the {T} token rows (every 16th) through the same "
                         f"FFN, oracle/ C restatement with OpenMP, {dt:.1f} s"}
        parity = parity_obj({"ffn_out": (normwise(y_dev[rows], want), 2e-2,
                                         "normwise relative, bf16 FFN output vs oracle")},
                            f"{len(rows)} token rows (every 16th of {T}), the cpu_baseline's "
                            f"own oracle run")
    return record(args, "swiglu_ffn_tflops", flops / (ms * 1e-3) / 1e12, "TFLOP/s", ms, "bf16",
                  {"workload": "swiglu_gated_ffn_bf16", "tokens": T, "hidden": H,
                   "intermediate": I},
                  roof, cpu, parity,
                  {"kernels": breakdown(syms, steps), "first_call_ms": round(first_ms, 1),
                   "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)},
                  steps=steps, warmup=warmup)


# ---- C2: elementwise + reduction chain (HBM-bound) ----------------------------------------

def run_chain(args, steps=None, warmup=None):
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    R, Cn = 8192, 4096
    keys = rng.split(rng.initKey(0x5EED0002), 2)
    x = rng.normalF32(keys[0], R * Cn).reshape(R, Cn)
    g = rng.normalF32(keys[1], Cn, 1.0, 0.1)
    xt, gt = E.fromHost(x), E.fromHost(g)
    E.sync()
    nbytes = R * Cn * 4
    # algorithmic bytes of each op group of the chain
    groups = {"relu_chain": 2 * nbytes, "reduceSum": nbytes + R * 4, "reduceMean": nbytes + R * 4,
              "reduceMax": nbytes + R * 4, "softmax": 2 * nbytes, "rmsNorm": 2 * nbytes + Cn * 4}
    total = sum(groups.values())

    def step():
        y = nn.relu(O.add(xt, xt))
        outs = [y, O.reduceSum(y, [1]), O.reduceMean(y, [1]), O.reduceMax(y, [1]),
                nn.softmax(xt, 1), nn.rmsNorm(xt, gt, 1e-5)]
        E.flush()
        return outs

    wall, dev_ms, first_ms, prof, hostc = timed_run(step, steps, warmup)
    ms = wall * 1e3 / steps

    def bytes_of(name):
        if name.startswith("rmsnorm_rows"):
            return groups["rmsNorm"]
        if name.startswith("softmax_rows"):
            return groups["softmax"]
        if name.startswith("ew_"):  # the relu chain, or the [8192] divide of reduceMean
            return groups["relu_chain"] if name.startswith(f"ew_fused{{{R * Cn}x") else 3 * R * 4
        if name.startswith("reduce"):
            # one read of x; one [R] output per op, plus reduceMean's quotient
            ops = int(name.split("ops")[0].rsplit(",", 1)[1]) if "ops" in name else 1
            return nbytes + R * 4 * (ops + (1 if ",mean" in name else 0))
        return None

    syms = by_symbol(prof, bytes_of)
    roof = roofline("chain", by_symbol(prof, bytes_of, by_shape=True), "hbm")
    outs = [E.toHost(t) for t in step()]
    cpu, parity = None, None
    if not args.no_cpu_baseline:
        orc = oracle_mod()
        rows = np.arange(0, R, 4)            # 2048 rows spread over the batch
        xs, t0 = np.ascontiguousarray(x[rows]), time.perf_counter()
        reps = 0
        while True:
            y = orc.binary(orc.MAX, orc.binary(orc.ADD, xs, xs), np.zeros_like(xs))
            s_ = orc.reduce(orc.RSUM, y, [1])
            m_ = orc.binary(orc.DIV, orc.reduce(orc.RSUM, y, [1]),
                            np.full(len(rows), Cn, np.float32))
            mx = orc.reduce(orc.RMAX, y, [1])
            sm = orc.softmax_rows(xs)
            rn = orc.rmsnorm_rows(xs, g, 1e-5)
            reps += 1
            if time.perf_counter() - t0 >= 10.0:
                break
        dt = time.perf_counter() - t0
        cpu = {"value": round(total * len(rows) / R * reps / dt / 1e9, 2), "unit": "GB/s",
               "cores": int(orc.lib().orc_num_threads()), "kind": "port",
               "sample": f"{reps} passes of the chain over {len(rows)} of the {R} rows (every "
                         f"4th), oracle/ C restatement, {dt:.1f} s"}
        ry, rs, rm, rmx, rsm, rrn = (o[rows] for o in outs)
        parity = parity_obj(
            {"relu": (int(np.count_nonzero(ry.view(np.uint32) != y.view(np.uint32))), 0,
                      "elements of relu(x + x) not bit-equal"),
             "reduceSum": (max_rel(rs, s_), 1e-5, "max elementwise relative"),
             "reduceMean": (max_rel(rm, m_), 1e-5, "max elementwise relative"),
             "reduceMax": (int(np.count_nonzero(rmx.view(np.uint32) != mx.view(np.uint32))), 0,
                           "rows not bit-equal"),
             "softmax": (max_rel(rsm, sm), 1e-5, "max elementwise relative"),
             "rmsNorm": (max_rel(rrn, rn), 1e-5, "max elementwise relative")},
            f"{len(rows)} of the {R} rows (every 4th), the cpu_baseline's own oracle run")
    return record(args, "eager_chain_hbm_gbs", total / (ms * 1e-3) / 1e9, "GB/s", ms, "f32",
                  {"workload": "eager_elementwise_reduction_chain_f32", "rows": R, "cols": Cn},
                  roof, cpu, parity,
                  {"kernels": breakdown(syms, steps), "algorithmic_bytes_per_step": total,
                   "hbm_frac": round(total / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)},
                  steps=steps, warmup=warmup)


# ---- copy: the streaming kernel the HBM byte counters are calibrated on --------------------

def run_copy(args):
    n = 256 * 1024 * 1024  # 1 GiB of fp32
    x = E.fromHost(np.ones(n, np.float32))
    E.sync()

    def step():
        y = O.neg(x)
        E.flush()
        return y

    wall, dev_ms, first_ms, prof, hostc = timed_run(step, args.steps, args.warmup)
    ms = wall * 1e3 / args.steps
    syms = by_symbol(prof, lambda name: 2 * n * 4)
    roof = roofline("copy", syms, "hbm")
    y = E.toHost(step())
    parity = parity_obj({"neg": (int(np.count_nonzero(y != -1.0)), 0,
                                 "elements of neg(1) not equal to -1")}, f"all {n} elements")
    return record(args, "stream_copy_gbs", 2 * n * 4 / (ms * 1e-3) / 1e9, "GB/s", ms, "f32",
                  {"workload": "stream_neg_f32", "elements": n}, roof, None, parity,
                  {"bytes_per_launch": 2 * n * 4})


# ---- C5: DeepSeek-style routed MoE layer ---------------------------------------------------

C5 = dict(tokens=8192, hidden=2048, intermediate=1408, routed=64, shared=2, top_k=6)


def moe_flops(T, H, I, E_, S, k):
    """Sparse algorithmic FLOPs: router + the k routed experts of every token
    + the shared experts (each expert 3 GEMMs of 2*H*I per token)."""
    return 2 * T * H * E_ + 2 * 3 * T * k * H * I + 2 * 3 * T * S * H * I


def build_moe(cfg, seed=0x5EED0005):
    T, H, I, E_, S = (cfg["tokens"], cfg["hidden"], cfg["intermediate"], cfg["routed"],
                      cfg["shared"])
    keys = rng.split(rng.initKey(seed), 2 + S + E_)
    x = E.f32_to_bf16_bits(rng.normalF32(keys[0], T * H)).reshape(T, H)
    wr = rng.normalF32(keys[1], H * E_, 0.0, 0.02).reshape(H, E_)
    host = {"x": x, "wr": wr, "experts": []}

    def expert(key):
        ks = rng.split(key, 3)
        ws = [E.f32_to_bf16_bits(rng.normalF32(ks[i], fi * fo, 0.0, 0.02)).reshape(fi, fo)
              for i, (fi, fo) in enumerate([(H, I), (H, I), (I, H)])]
        host["experts"].append(ws)
        return nn.DeepSeekExpert(*[nn.Linear(E.fromHost(w, DType.BFLOAT16),
                                             E.fromHost(np.zeros(w.shape[1], np.uint16),
                                                        DType.BFLOAT16)) for w in ws])

    shared = [expert(keys[2 + i]) for i in range(S)]
    routed = [expert(keys[2 + S + e]) for e in range(E_)]
    moe = nn.DeepSeekMoE(nn.Linear(E.fromHost(wr), E.fromHost(np.zeros(E_, np.float32))),
                         shared, routed, cfg["top_k"])
    return moe, E.fromHost(x, DType.BFLOAT16), host


def run_moe(args, steps=None, warmup=None):
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    cfg = dict(C5)
    T, H, I, E_, S, k = (cfg["tokens"], cfg["hidden"], cfg["intermediate"], cfg["routed"],
                         cfg["shared"], cfg["top_k"])
    t0 = time.perf_counter()
    moe, xt, host = build_moe(cfg)
    E.sync()
    print(f"# inputs ready in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)

    if args.moe_path == "lazy":
        # rew runs DeepSeekMoE.forward only under jit/lazy (its topK is
        # trace-only, src/rew/ops/sort.nim:88-90): the layer is traced once
        # with its parameters as arguments and every step is one
        # rew_mi355x_execute_jit call of the cached module
        from rew_amd import jit as J
        lz = J.lazy(lambda a: [nn.moeFromParams(a[1:], S, E_, k).forward(a[0])],
                    "deepseekMoE")
        call_args = [xt] + nn.moeParams(moe)

        def step():
            y = lz.call(call_args)[0]
            E.flush()
            return y
    else:
        def step():
            y = moe.forward(xt)
            E.flush()
            return y

    wall, dev_ms, first_ms, prof, hostc = timed_run(step, steps, warmup)
    ms = wall * 1e3 / steps
    flops = moe_flops(T, H, I, E_, S, k)
    syms = by_symbol(prof, entry_flops)
    roof = roofline("moe", syms, "mfma")
    y_dev = E.toHostF32(step())
    cpu, parity = None, None
    if not args.no_cpu_baseline:
        orc = oracle_mod()
        rows = np.arange(0, T, T // 256)     # 256 tokens, one in every 32
        xs = orc.from_bf16(host["x"][rows])
        z = lambda n: np.zeros(n, np.float32)
        exps = [(orc.from_bf16(a), z(I), orc.from_bf16(b), z(I), orc.from_bf16(c), z(H))
                for a, b, c in host["experts"]]
        t0 = time.perf_counter()
        want, _, _ = orc.deepseek_moe(xs, exps[:S], exps[S:], host["wr"], z(E_), k)
        dt = time.perf_counter() - t0
        cpu = {"value": round(len(rows) / dt, 2), "unit": "tokens/s",
               "cores": int(orc.lib().orc_num_threads()), "kind": "port",
               "sample": f"{len(rows)} of the {T} tokens (every {T // len(rows)}th) through "
                         f"the reference's dense formulation (every routed expert on every "
                         f"token, deepseek.nim:122-145), oracle/ C restatement, {dt:.1f} s"}
        # router and expert ids of all T tokens.  The logits are an fp32
        # GEMM over K = H whose accumulation order rew leaves to the plugin,
        # so they are held to the bound every summation order meets:
        # |got - exact| <= K * 2^-24 * sum_k |x_k| |w_k| (first order).  The
        # ids must be the oracle's top-k of the device's own probabilities
        # exactly, and a row whose ids differ from the oracle's top-k of the
        # oracle's probabilities must be a near-tie (two candidates closer
        # than twice that row's probability error)
        xf = orc.from_bf16(host["x"])
        logits_dev = E.toHost(moe.gate.forward(O.astype(xt, DType.FLOAT32)))
        probs_dev = E.toHost(nn.softmax(moe.gate.forward(O.astype(xt, DType.FLOAT32)), 1))
        ids_dev = E.toHost(moe.route(xt)[1])
        logits = orc.linear(xf, host["wr"], z(E_), False)
        absdot = np.abs(xf).astype(np.float64) @ np.abs(host["wr"]).astype(np.float64)
        logit_ratio = float(np.max(np.abs(logits_dev.astype(np.float64) - logits) /
                                   (H * 2.0 ** -24 * np.maximum(absdot, 1e-300))))
        probs = orc.softmax_rows(logits)
        _, ids_want = orc.topk_rows(probs, k)
        _, ids_same = orc.topk_rows(probs_dev, k)
        diff = np.where(np.any(ids_dev != ids_want, axis=1))[0]
        not_tie = 0
        for r in diff:
            row_err = np.max(np.abs(probs_dev[r] - probs[r]))
            srt = np.sort(probs[r])[::-1]
            if np.min(srt[:k] - srt[1:k + 1]) > 2 * row_err:
                not_tie += 1
        parity = parity_obj(
            {"moe_out": (normwise(y_dev[rows], want), 2e-2,
                         "normwise relative, bf16 layer output vs the oracle's dense layer"),
             "router_logits": (logit_ratio, 1.0,
                               "max |got - oracle| / (K 2^-24 sum|x||w|), fp32 router GEMM, "
                               "all tokens"),
             "router_probs": (normwise(probs_dev, probs), None,
                              "normwise relative, fp32 router softmax, all tokens "
                              "(reported; bounded through the logits)"),
             "expert_ids_given_probs": (int(np.count_nonzero(np.any(ids_dev != ids_same,
                                                                     axis=1))), 0,
                                        "rows whose device top-k ids differ from the "
                                        "oracle's top-k of the same probabilities"),
             "expert_ids_off_near_ties": (not_tie, 0,
                                          f"rows whose ids differ from the oracle's and are "
                                          f"not a near-tie ({len(diff)} rows differ in all)")},
            f"ids and router: all {T} tokens; layer output: {len(rows)} tokens (every "
            f"{T // len(rows)}th), the cpu_baseline's own oracle run")
    return record(args, "moe_layer_tokens_per_s", T * steps / wall, "tokens/s", ms, "bf16",
                  {"workload": "deepseek_moe_layer_bf16", "tokens": T, "hidden": H,
                   "intermediate": I, "routed_experts": E_, "shared_experts": S, "top_k": k,
                   "path": args.moe_path},
                  roof, cpu, parity,
                  {"kernels": breakdown(syms, steps), "first_call_ms": round(first_ms, 1),
                   "host": hostc,
                   "algorithmic_tflop": round(flops / 1e12, 4),
                   "achieved_tflops": round(flops / (ms * 1e-3) / 1e12, 1),
                   "mfma_frac": round(flops / (ms * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4)},
                  steps=steps, warmup=warmup)


# ---- C1: MNIST-shaped MLP inference (latency-bound) ----------------------------------------

def run_mnist(args, steps=None, warmup=None):
    steps = args.steps if steps is None else steps
    warmup = args.warmup if warmup is None else warmup
    B, D, Hd, C = 128, 784, 128, 10
    keys = rng.split(rng.initKey(0x5EED0001), 3)
    x = rng.uniformF32(keys[0], B * D, 0.0, 1.0).reshape(B, D)
    w1 = rng.xavierUniformF32(keys[1], D, Hd).reshape(D, Hd)
    w2 = rng.xavierUniformF32(keys[2], Hd, C).reshape(Hd, C)
    l1 = nn.Linear(E.fromHost(w1), E.fromHost(np.zeros(Hd, np.float32)))
    l2 = nn.Linear(E.fromHost(w2), E.fromHost(np.zeros(C, np.float32)))
    xt = E.fromHost(x)
    E.sync()

    if args.mnist_path == "lazy":
        # Linear -> relu -> Linear -> softmax as one lazy batch (the traced
        # module, parameters as arguments), then the argmax: rew's argmax
        # raises in both modes (its int32 reduceMin), so it runs as the
        # backend's native op on the batch's output
        from rew_amd import jit as J
        mlp = J.lazy(lambda a: [nn.softmax(nn.Linear(a[3], a[4]).forward(
            nn.relu(nn.Linear(a[1], a[2]).forward(a[0]))), 1)], "mnistMlp")
        call_args = [xt, l1.weight, l1.bias, l2.weight, l2.bias]

        def step():
            ids = O.argmax(mlp.call(call_args)[0], 1)
            E.flush()
            return ids
    else:
        def step():
            ids = O.argmax(nn.softmax(l2.forward(nn.relu(l1.forward(xt))), 1), 1)
            E.flush()
            return ids

    wall, dev_ms, first_ms, prof, hostc = timed_run(step, steps, warmup)
    ms = wall * 1e3 / steps
    flops = 2 * B * D * Hd + 2 * B * Hd * C

    def gemm_flops(name):
        if name.startswith("class_head{"):  # the last Linear, softmax and argmax
            m, k, n = (int(v) for v in name[11:name.index("}")].split("x"))
            return 2 * m * k * n
        f = entry_flops(name)
        return f if f is not None and name.startswith("gemm") else None

    syms = by_symbol(prof, gemm_flops)
    ksym, d = max(syms.items(), key=lambda kv: kv[1]["ms"])
    roof = {"bound": "fp32", "kernel": ksym, "achieved": None, "peak": FP32_PEAK_TFLOPS,
            "unit": "TFLOP/s", "frac": None, "traffic": traffic_for("mnist", ksym),
            "avg_launch_us": round(d["ms"] / d["launches"] * 1e3, 2), "launches": d["launches"]}
    if d["known"] and d["work"]:
        ach = d["work"] / d["launches"] / (d["ms"] / d["launches"] * 1e-3) / 1e12
        roof["achieved"] = round(ach, 3)
        roof["frac"] = round(ach / FP32_PEAK_TFLOPS, 5)
    ids_dev = E.toHost(step())
    cpu, parity = None, None
    if not args.no_cpu_baseline:
        orc = oracle_mod()
        t0, reps = time.perf_counter(), 0
        z1, z2 = np.zeros(Hd, np.float32), np.zeros(C, np.float32)
        while True:
            h = np.maximum(orc.linear(x, w1, z1, False), 0)
            want = orc.argmax_rows(orc.softmax_rows(orc.linear(h, w2, z2, False)))
            reps += 1
            if time.perf_counter() - t0 >= 10.0:
                break
        dt = time.perf_counter() - t0
        cpu = {"value": round(B * reps / dt, 1), "unit": "rows/s",
               "cores": int(orc.lib().orc_num_threads()), "kind": "port",
               "sample": f"{reps} forwards of the full [128,784] batch, oracle/ C restatement, "
                         f"{dt:.1f} s"}
        parity = parity_obj({"argmax": (int(np.count_nonzero(ids_dev != want)), 0,
                                        "rows whose argmax differs (bit-exact)")},
                            f"the full batch of {B} rows, the cpu_baseline's own oracle run")
    return record(args, "mnist_mlp_rows_per_s", B * steps / wall, "rows/s", ms, "f32",
                  {"workload": "mnist_mlp_inference_f32", "batch": B, "layers": [D, Hd, C],
                   "path": args.mnist_path},
                  roof, cpu, parity,
                  {"kernels": breakdown(syms, steps), "first_call_ms": round(first_ms, 2),
                   "host": hostc,
                   "us_per_forward": round(ms * 1e3, 1), "algorithmic_flops": flops,
                   "device_us_per_forward": round(dev_ms * 1e3 / steps, 1)},
                  steps=steps, warmup=warmup)


def compact(rec):
    """The other configurations' records as carried on the headline line."""
    keep = ("metric", "value", "unit", "ms_per_step", "steps", "warmup", "dtype", "config",
            "roofline", "cpu_baseline", "parity", "kernels", "mfma_frac", "hbm_frac",
            "us_per_forward", "device_us_per_forward")
    return {k: rec[k] for k in keep if k in rec}


WORKLOADS = {"llama": run_llama, "swiglu": run_swiglu, "chain": run_chain, "copy": run_copy,
             "moe": run_moe, "mnist": run_mnist}

# the other configurations, run after the headline by default: (key, runner,
# steps, warmup) -- MNIST forwards are ~30 us, so it takes more steps
EXTRAS = [("C1_mnist_mlp", run_mnist, 200, 20), ("C2_eager_chain", run_chain, None, None),
          ("C3_swiglu_ffn", run_swiglu, None, None), ("C5_deepseek_moe", run_moe, None, None)]


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="llama", choices=sorted(WORKLOADS))
    ap.add_argument("--norm", default="rms", choices=["rms", "layer"],
                    help="llama workload: the config's RMSNorm, or rew's own LayerNorm "
                         "(src/rew/models/llama.nim:32-33)")
    ap.add_argument("--no-extras", action="store_true",
                    help="llama workload: skip the other configurations' records")
    ap.add_argument("--cpu-seqs", type=int, default=2,
                    help="sequences of the llama batch in the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--mnist-path", default="lazy", choices=["lazy", "eager"],
                    help="mnist workload: the MLP as a lazy batch then the native argmax, or "
                         "every op dispatched eagerly")
    ap.add_argument("--moe-path", default="lazy", choices=["lazy", "eager"],
                    help="moe workload: rew's lazy batch (its executable form) or the "
                         "eager op stream of the mirror")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X only; the multi-GPU sharding of the "
              "path is a design note, not code. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if E.deviceCount() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    E.installEagerBackend(E.mi355x(0))
    rec = WORKLOADS[args.workload](args)
    if args.workload == "llama" and not args.no_extras:
        extras = {}
        for key, fn, st, wu in EXTRAS:
            print(f"# {key}", file=sys.stderr, flush=True)
            extras[key] = compact(fn(args, st, wu))
            E.sync()
        rec["configs"] = extras
    print(json.dumps(rec), flush=True)


if __name__ == "__main__":
    main()
