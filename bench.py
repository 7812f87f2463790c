#!/usr/bin/env python3
"""Throughput of rew's eager hot path on one MI355X through the mi355x backend.

Default workload (the headline metric): one Llama-style decoder layer prefill,
bf16, B=4 x S=2048 tokens, hidden 4096, 32 query / 8 KV heads (GQA), head dim
128, RoPE theta 500000, RMSNorm eps 1e-5, SwiGLU intermediate 14336, token
embeddings gathered from a [128256, 4096] table with uniform random ids.
A step is: torchIndexSelect(table, ids) -> LlamaDecoderLayer.forward, driven
through the same eager op sequence rew's nn layers emit (rew_amd.nn), with
every input already resident in HBM.

Prints ONE JSON line (rank 0, N=1) with the metric, a roofline object for
the dominant kernel (durations from HIP events recorded on the backend's own
stream), the whole-layer MFMA fraction, and a cpu_baseline: the CPU
restatement in oracle/ timed on this host's cores on a bounded sample.
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


def profile_step(step):
    """Per-kernel totals of one step from the backend's launch events."""
    lib = E._lib.load()
    ctx = E.context()
    if lib.rew_mi355x_profile_begin(ctx) != 0:
        raise RuntimeError(lib.rew_mi355x_last_error().decode())
    step()
    if lib.rew_mi355x_profile_end(ctx) != 0:
        raise RuntimeError(lib.rew_mi355x_last_error().decode())
    out = []
    name = C.create_string_buffer(256)
    n = C.c_int64()
    ms = C.c_double()
    i = 0
    while lib.rew_mi355x_profile_entry(ctx, i, name, 256, C.byref(n), C.byref(ms)) == 0:
        out.append((name.value.decode(), int(n.value), float(ms.value)))
        i += 1
    return out


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
    dims = [int(v) for v in entry_name[entry_name.index("[") + 1:-1].split(",")]
    if entry_name.startswith("flash_attn"):
        B, H, _, Sq, Sk, D, cmp, _ = dims
        return 4 * B * H * D * visible_pairs(Sq, Sk, cmp)
    b, m, n, k = dims
    # the SwiGLU kernel runs the gate and up projections over the same A
    return (4 if "swiglu" in entry_name else 2) * b * m * n * k


def kernel_symbol(entry_name: str) -> str:
    return entry_name.split("[")[0].split("{")[0].split("+")[0]


# ---- C4: Llama decoder layer prefill -------------------------------------------------------

def build_llama(cfg, seed=0x5EED0004, small_vocab=None):
    """Weights ~N(0, 0.02) bf16, zero biases, gammas ~N(1, 0.1) f32, keyed per
    tensor in declaration order from initKey(seed)."""
    H, nh, nkv, hd, I = (cfg["hidden"], cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                         cfg["intermediate"])
    V = small_vocab or cfg["vocab"]
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
    layer = nn.LlamaDecoderLayer(
        nn.GroupedQueryAttention(m["q"], m["k"], m["v"], m["o"], nh, nkv, hd, rope),
        nn.GatedFeedForward(m["g"], m["u"], m["d"]),
        nn.RMSNorm(E.fromHost(host["g1"]), cfg["eps"]),
        nn.RMSNorm(E.fromHost(host["g2"]), cfg["eps"]))
    emb = nn.Embedding(E.fromHost(table, DType.BFLOAT16))
    return layer, emb, E.fromHost(ids), host, table, ids


def cpu_baseline_llama(cfg, host, table, ids, tokens):
    """The oracle's restatement of the same layer on a bounded sample: one
    sequence of `tokens` tokens (the first `tokens` ids of sequence 0)."""
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle as orc
    orc.build()
    nh, nkv, hd = cfg["heads"], cfg["kv_heads"], cfg["head_dim"]
    p = {}
    for n in "qkvogud":
        p["w" + n] = orc.from_bf16(host["w" + n])
        p["b" + n] = host["b" + n]
    p["g1"], p["g2"] = host["g1"], host["g2"]
    c, s = nn.rope_tables(hd, tokens, cfg["rope_theta"])
    x = orc.from_bf16(table[ids[:tokens]]).reshape(1, tokens, cfg["hidden"])
    t0 = time.perf_counter()
    orc.llama_layer(x, p, nh, nkv, c, s, cfg["eps"], True, True, "rms")
    dt = time.perf_counter() - t0
    return {"value": tokens / dt, "unit": "tokens/s", "cores": int(orc.lib().orc_num_threads()),
            "kind": "port",
            "sample": f"1 x {tokens}-token causal prefill of the same layer (full hidden/FFN/"
                      f"head dims), oracle/ C restatement with OpenMP, {dt:.2f} s"}


def run_llama(args):
    cfg = dict(C4)
    B, S, H = cfg["batch"], cfg["seq_len"], cfg["hidden"]
    t0 = time.perf_counter()
    layer, emb, ids_t, host, table, ids = build_llama(cfg)
    E.sync()
    print(f"# inputs ready in {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)

    def step():
        x = O.reshape(emb.lookup(ids_t), [B, S, H])
        y = layer.forward(x, causal=True)
        E.flush()
        return y

    t0 = time.perf_counter()
    y = step()
    E.sync()
    first_ms = (time.perf_counter() - t0) * 1e3
    del y
    for _ in range(args.warmup):
        step()
    E.sync()
    ev = HipEvents(backend_stream())
    e0, e1 = ev.event(), ev.event()
    E.sync()
    t0 = time.perf_counter()
    ev.record(e0)
    outs = []
    for _ in range(args.steps):
        outs.append(step())
        if len(outs) > 2:
            outs.pop(0)
    ev.record(e1)
    E.sync()
    wall = time.perf_counter() - t0
    dev_ms = ev.elapsed_ms(e0, e1)
    outs.clear()
    ms_per_step = wall * 1e3 / args.steps
    tokens = B * S
    value = tokens * args.steps / wall
    flops = llama_layer_flops(B, S, H, cfg["heads"], cfg["kv_heads"], cfg["head_dim"],
                              cfg["intermediate"])

    # per-kernel breakdown of one extra step
    prof = profile_step(step)
    E.sync()
    for name, n, ms in sorted(prof, key=lambda r: -r[2]):
        print(f"#   {ms * 1e3:9.1f} us  x{n:<3d} {name}", file=sys.stderr)
    by_sym = {}
    for name, n, ms in prof:
        sym = kernel_symbol(name)
        d = by_sym.setdefault(sym, {"launches": 0, "ms": 0.0, "flops": 0, "flops_known": True})
        d["launches"] += n
        d["ms"] += ms
        f = entry_flops(name)
        if f is None:
            d["flops_known"] = False
        else:
            d["flops"] += f * n
    dom = max(by_sym.items(), key=lambda kv: kv[1]["ms"])
    dsym, d = dom
    avg_ms = d["ms"] / d["launches"]
    if d["flops_known"]:
        per_launch = d["flops"] / d["launches"]
        achieved = per_launch / (avg_ms * 1e-3) / 1e12
        roof = {"bound": "mfma", "kernel": dsym, "achieved": round(achieved, 1),
                "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                "frac": round(achieved / BF16_PEAK_TFLOPS, 4), "traffic": None,
                "avg_launch_us": round(avg_ms * 1e3, 2), "launches_per_step": d["launches"],
                "algorithmic_flops_per_launch": int(per_launch)}
    else:
        roof = {"bound": "hbm", "kernel": dsym, "achieved": None, "peak": HBM_PEAK_GBS,
                "unit": "GB/s", "frac": None, "traffic": None,
                "avg_launch_us": round(avg_ms * 1e3, 2), "launches_per_step": d["launches"]}
    total_prof_ms = sum(v["ms"] for v in by_sym.values())
    breakdown = sorted(((k, round(v["ms"], 3), v["launches"]) for k, v in by_sym.items()),
                       key=lambda r: -r[1])

    cpu = None
    if not args.no_cpu_baseline:
        cpu = cpu_baseline_llama(cfg, host, table, ids, args.cpu_tokens)

    line = {
        "metric": "llama_layer_prefill_tokens_per_s",
        "value": round(value, 1), "unit": "tokens/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_per_step, 3),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "bf16",
        "data": "synthetic (rew Threefry/normalF32 inputs, random-init weights)",
        "config": {"workload": "llama_decoder_layer_prefill_bf16", "batch": B, "seq_len": S,
                   "hidden": H, "heads": cfg["heads"], "kv_heads": cfg["kv_heads"],
                   "head_dim": cfg["head_dim"], "intermediate": cfg["intermediate"],
                   "vocab": cfg["vocab"], "rope_theta": cfg["rope_theta"], "causal": True,
                   "parallelism": "single-gpu"},
        "roofline": roof,
        "layer": {"algorithmic_tflop": round(flops / 1e12, 4),
                  "achieved_tflops": round(flops / (ms_per_step * 1e-3) / 1e12, 1),
                  "mfma_frac": round(flops / (ms_per_step * 1e-3) / 1e12 / BF16_PEAK_TFLOPS, 4),
                  "device_ms_per_step": round(dev_ms / args.steps, 3),
                  "kernel_ms_per_step": round(total_prof_ms, 3),
                  "first_call_ms": round(first_ms, 1),
                  "kernels": breakdown[:12]},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def main():
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--workload", default="llama", choices=["llama"])
    ap.add_argument("--cpu-tokens", type=int, default=512,
                    help="tokens in the cpu_baseline sample")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py: this build measures one MI355X only (the sharded path is design-only); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if E.deviceCount() < 1:
        print("bench.py: no HIP device visible", file=sys.stderr)
        sys.exit(1)
    E.installEagerBackend(E.mi355x(0))
    run_llama(args)


if __name__ == "__main__":
    main()
