"""Python face of the CPU oracle (TEST INFRASTRUCTURE ONLY).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
import this module, and only as the checker / the timed CPU column.

Floating-point arithmetic runs in oracle/rew_oracle.c (plain C restatement
of rew's op semantics, each function citing the reference).  numpy is used
here only for index/byte work (transposes, broadcasts, slices, gathers).
Composite oracles at the bottom chain the C primitives in exactly the op
order of rew's composites (cited per function).
"""
from __future__ import annotations

import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB = HERE / "librew_oracle.so"

F32, BF16 = 0, 1
ADD, SUB, MUL, DIV, MAX, MIN, POW, REM, ATAN2 = range(9)
NEG, ABS, EXP, LOG, SQRT, RSQRT, TANH, LOGISTIC, SIN, COS, FLOOR, CEIL = range(12)
RSUM, RMAX, RMIN, RPROD = range(4)

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB.exists():
            build()
        _lib = C.CDLL(str(LIB))
    return _lib


def _p(a: np.ndarray) -> C.c_void_p:
    return a.ctypes.data_as(C.c_void_p)


def _i64(xs) -> C.Array:
    xs = list(xs)
    return (C.c_int64 * max(1, len(xs)))(*xs)


# ---- rng -------------------------------------------------------------------------

def threefry(k0: int, k1: int, c0: int, c1: int) -> tuple[int, int]:
    out = (C.c_uint32 * 2)()
    lib().orc_threefry(C.c_uint32(k0), C.c_uint32(k1), C.c_uint32(c0), C.c_uint32(c1), out)
    return out[0], out[1]


def split(key: tuple[int, int], n: int) -> list[tuple[int, int]]:
    out = (C.c_uint32 * (2 * max(1, n)))()
    lib().orc_split(C.c_uint32(key[0]), C.c_uint32(key[1]), C.c_int(n), out)
    return [(out[2 * i], out[2 * i + 1]) for i in range(n)]


def fold_in(key: tuple[int, int], data: int) -> tuple[int, int]:
    out = (C.c_uint32 * 2)()
    lib().orc_fold_in(C.c_uint32(key[0]), C.c_uint32(key[1]), C.c_uint64(data), out)
    return out[0], out[1]


def init_key(seed: int) -> tuple[int, int]:
    """src/rew/rng.nim:57-63: low and high halves of the 64-bit seed."""
    return seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF


def uniform_f32(key, n: int, lo: float, hi: float) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_uniform_f32(C.c_uint32(key[0]), C.c_uint32(key[1]), C.c_int64(n), C.c_float(lo),
                          C.c_float(hi), _p(out))
    return out


def normal_f32(key, n: int, mean: float = 0.0, sd: float = 1.0) -> np.ndarray:
    out = np.empty(n, np.float32)
    lib().orc_normal_f32(C.c_uint32(key[0]), C.c_uint32(key[1]), C.c_int64(n), C.c_float(mean),
                         C.c_float(sd), _p(out))
    return out


# ---- bf16 -------------------------------------------------------------------------

def to_bf16(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16(_p(x), C.c_int64(x.size), _p(out))
    return out


def from_bf16(b: np.ndarray) -> np.ndarray:
    b = np.ascontiguousarray(b, np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().orc_bf16_to_f32(_p(b), C.c_int64(b.size), _p(out))
    return out


def round_bf16(x: np.ndarray) -> np.ndarray:
    return from_bf16(to_bf16(x))


# ---- primitives -----------------------------------------------------------------------

def binary(op: int, a: np.ndarray, b: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().orc_binary_f32(C.c_int(op), _p(a), _p(b), _p(out), C.c_int64(a.size))
    return out


def unary(op: int, a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, np.float32)
    out = np.empty(a.shape, np.float32)
    lib().orc_unary_f32(C.c_int(op), _p(a), _p(out), C.c_int64(a.size))
    return out


def reduce(op: int, x: np.ndarray, dims) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    dims = sorted(int(d) for d in dims)
    oshape = [s for i, s in enumerate(x.shape) if i not in dims]
    out = np.empty(oshape, np.float32)
    lib().orc_reduce_f32(C.c_int(op), _p(x), C.c_int(x.ndim), _i64(x.shape),
                         C.c_int(len(dims)), _i64(dims), _p(out))
    return out


def dot_general(a: np.ndarray, b: np.ndarray, lb, rb, lc, rc, bf16: bool = False) -> np.ndarray:
    """stablehlo.dot_general; bf16 operands given as uint16 bit arrays."""
    dt = BF16 if bf16 else F32
    a = np.ascontiguousarray(a, np.uint16 if bf16 else np.float32)
    b = np.ascontiguousarray(b, np.uint16 if bf16 else np.float32)
    used_a = set(lb) | set(lc)
    used_b = set(rb) | set(rc)
    oshape = [a.shape[d] for d in lb] + [s for i, s in enumerate(a.shape) if i not in used_a] + \
             [s for i, s in enumerate(b.shape) if i not in used_b]
    out = np.empty(oshape, np.uint16 if bf16 else np.float32)
    lib().orc_dot_general(C.c_int(dt), _p(a), C.c_int(a.ndim), _i64(a.shape), _p(b),
                          C.c_int(b.ndim), _i64(b.shape), C.c_int(len(lb)), _i64(lb), _i64(rb),
                          C.c_int(len(lc)), _i64(lc), _i64(rc), _p(out))
    return out


def gemm(a: np.ndarray, b: np.ndarray, round_bf16_out: bool = False) -> np.ndarray:
    """Dense [M,K] x [K,N] with double accumulation (float-valued operands)."""
    a = np.ascontiguousarray(a, np.float32)
    b = np.ascontiguousarray(b, np.float32)
    M, K = a.shape
    N = b.shape[1]
    out = np.empty((M, N), np.float32)
    lib().orc_gemm(_p(a), _p(b), _p(out), C.c_int64(M), C.c_int64(N), C.c_int64(K),
                   C.c_int(1 if round_bf16_out else 0))
    return out


# index / byte work (numpy): broadcast_in_dim, transpose, slice, concat, iota, gather
def broadcast_in_dim(x: np.ndarray, out_shape, dims) -> np.ndarray:
    shp = [1] * len(out_shape)
    for i, d in enumerate(dims):
        shp[d] = x.shape[i]
    return np.broadcast_to(x.reshape(shp), tuple(out_shape)).copy()


def iota(shape, dim: int, dtype=np.int32) -> np.ndarray:
    shp = [1] * len(shape)
    shp[dim] = shape[dim]
    return np.broadcast_to(np.arange(shape[dim]).reshape(shp), tuple(shape)).astype(dtype)


def index_select(x: np.ndarray, idx: np.ndarray, dim: int) -> np.ndarray:
    i = np.clip(idx.astype(np.int64), 0, x.shape[dim] - 1)
    return np.take(x, i, axis=dim)


def _index_vector(idx, ivd, batch):
    """The index vector of start/scatter indices `idx` at batch coordinate
    `batch` (coordinates of every dim except index_vector_dim, in order);
    index_vector_dim == rank means a trailing dim of size 1."""
    idx = np.asarray(idx)
    if ivd == idx.ndim:
        return [int(idx[tuple(batch)])]
    pos = list(batch[:ivd]) + [slice(None)] + list(batch[ivd:])
    return [int(v) for v in idx[tuple(pos)]]


def gather(x, idx, offset_dims, collapsed, start_index_map, ivd, slice_sizes,
           operand_batching=(), start_batching=()):
    """stablehlo.gather (rew builds it at src/rew/stablehlo/ops.nim:1387-1408;
    semantics: the StableHLO spec's gather): for every result index, the
    batch coordinates pick an index vector, whose entries set the starts of
    the operand dims named by start_index_map (operand batching dims start at
    the matching batch coordinate); every start is clamped into
    [0, dim - slice]; offset dims walk the operand's window dims in order.
    Explicit loops: small sizes only."""
    x, idx = np.asarray(x), np.asarray(idx)
    rank_i = idx.ndim
    bdims = [d for d in range(rank_i) if d != ivd]
    win = [d for d in range(x.ndim) if d not in collapsed and d not in operand_batching]
    out_rank = len(offset_dims) + len(bdims)
    shape, bi = [], 0
    for d in range(out_rank):
        if d in offset_dims:
            shape.append(slice_sizes[win[list(offset_dims).index(d)]])
        else:
            shape.append(idx.shape[bdims[bi]])
            bi += 1
    out = np.empty(shape, x.dtype)
    batch_out = [d for d in range(out_rank) if d not in offset_dims]
    for o in np.ndindex(*shape):
        batch = [o[d] for d in batch_out]
        start = [0] * x.ndim
        for j, v in enumerate(_index_vector(idx, ivd, batch)):
            start[start_index_map[j]] = v
        for xd, sd in zip(operand_batching, start_batching):
            start[xd] = batch[bdims.index(sd)]
        full = [min(max(start[d], 0), x.shape[d] - slice_sizes[d]) for d in range(x.ndim)]
        for j, d in enumerate(offset_dims):
            full[win[j]] += o[d]
        out[o] = x[tuple(full)]
    return out


def scatter(x, idx, upd, update_window_dims, inserted, scatter_dims_to_operand, ivd, op,
            input_batching=(), index_batching=()):
    """stablehlo.scatter with one input (rew builds it at
    src/rew/stablehlo/ops.nim:1531-1569; semantics: the StableHLO spec's
    scatter): every update element lands at start + window offset and is
    combined with `op` ("add", "maximum", "minimum", "multiply" or
    "replace"); an update whose index falls outside the input is skipped.
    Updates are applied in row-major order of the updates.  Explicit loops:
    small sizes only."""
    x, idx, upd = np.asarray(x), np.asarray(idx), np.asarray(upd)
    out = x.copy()
    rank_i = idx.ndim
    bdims = [d for d in range(rank_i) if d != ivd]
    win = [d for d in range(x.ndim) if d not in inserted and d not in input_batching]
    scat = [d for d in range(upd.ndim) if d not in update_window_dims]
    fn = {"add": lambda a, b: a + b, "maximum": lambda a, b: np.maximum(a, b),
          "minimum": lambda a, b: np.minimum(a, b), "multiply": lambda a, b: a * b,
          "replace": lambda a, b: b}[op]
    for u in np.ndindex(*upd.shape):
        batch = [u[d] for d in scat]
        start = [0] * x.ndim
        for j, v in enumerate(_index_vector(idx, ivd, batch)):
            start[scatter_dims_to_operand[j]] = v
        for xd, sd in zip(input_batching, index_batching):
            start[xd] = batch[bdims.index(sd)]
        full = list(start)
        for j, d in enumerate(update_window_dims):
            full[win[j]] += u[d]
        if all(0 <= full[d] < x.shape[d] for d in range(x.ndim)):
            out[tuple(full)] = fn(out[tuple(full)], upd[u])
    return out


def sort_order(x, axis: int, descending: bool):
    """The permutation stablehlo.sort applies with a one-compare comparator
    (src/rew/ops/sort.nim:13-33): stable, -0 == +0, NaN after every number
    (numpy's stable argsort keeps NaN last and ties in order)."""
    x = np.asarray(x)
    key = np.where(x == 0, 0, x).astype(np.float64) if x.dtype.kind == "f" else x.astype(np.int64)
    return np.argsort(-key if descending else key, axis=axis, kind="stable")


def pad(x: np.ndarray, value, lo, hi, interior) -> np.ndarray:
    """stablehlo.pad as rew emits it (src/rew/ops/shape.nim:139-172; result
    shape src/rew/stablehlo/ops.nim:807-824): the operand's elements spread
    `interior` apart, `lo` / `hi` elements of padding at the edges (negative
    edges crop).  Built element by element from the output side."""
    x = np.asarray(x)
    shape = [d + l + h + max(d - 1, 0) * i for d, l, h, i in zip(x.shape, lo, hi, interior)]
    out = np.full(shape, value, dtype=x.dtype)
    # every operand element lands at lo + i * (interior + 1), if in range
    for src in np.ndindex(*x.shape):
        dst = tuple(l + s * (i + 1) for l, s, i in zip(lo, src, interior))
        if all(0 <= d < n for d, n in zip(dst, shape)):
            out[dst] = x[src]
    return out


def _clamped_starts(starts, room):
    # stablehlo.dynamic_slice / dynamic_update_slice clamp each start into
    # [0, operand dim - window dim]
    return [min(max(int(s), 0), r) for s, r in zip(starts, room)]


def dynamic_slice(x: np.ndarray, starts, sizes) -> np.ndarray:
    """stablehlo.dynamic_slice (src/rew/ops/shape.nim:213-250)."""
    st = _clamped_starts(starts, [d - s for d, s in zip(x.shape, sizes)])
    return x[tuple(slice(a, a + s) for a, s in zip(st, sizes))].copy()


def dynamic_update_slice(x: np.ndarray, upd: np.ndarray, starts) -> np.ndarray:
    """stablehlo.dynamic_update_slice (src/rew/ops/shape.nim:251-290)."""
    st = _clamped_starts(starts, [d - u for d, u in zip(x.shape, upd.shape)])
    out = x.copy()
    out[tuple(slice(a, a + u) for a, u in zip(st, upd.shape))] = upd
    return out


def cholesky(a: np.ndarray, lower: bool = True) -> np.ndarray:
    """stablehlo.cholesky (src/rew/ops/linalg.nim:177-202) over the last two
    dims, in float64 by the Cholesky-Crout recurrence, from the referenced
    triangle only; the other triangle is zero."""
    a = np.asarray(a, np.float64)
    out = np.zeros_like(a)
    n = a.shape[-1]
    for b in np.ndindex(*a.shape[:-2]):
        m = a[b] if lower else a[b].T
        L = np.zeros((n, n))
        for j in range(n):
            L[j, j] = np.sqrt(m[j, j] - sum(L[j, k] * L[j, k] for k in range(j)))
            for i in range(j + 1, n):
                L[i, j] = (m[i, j] - sum(L[i, k] * L[j, k] for k in range(j))) / L[j, j]
        out[b] = L if lower else L.T
    return out


def _bn_view(x, fi):
    # [outer, C, inner] view with the feature dim in the middle
    x = np.asarray(x, np.float64)
    return x.reshape(int(np.prod(x.shape[:fi], dtype=np.int64)), x.shape[fi], -1)


def batch_norm_inference(x, scale, offset, mean, var, eps, fi):
    """stablehlo.batch_norm_inference (src/rew/ops/normalization.nim:87-118), float64:
    scale (x - mean) / sqrt(var + eps) + offset along feature dim fi."""
    v = _bn_view(x, fi)
    b = lambda t: np.asarray(t, np.float64)[None, :, None]
    return (b(scale) * ((v - b(mean)) / np.sqrt(b(var) + eps)) + b(offset)).reshape(np.shape(x))


def batch_norm_training(x, scale, offset, eps, fi):
    """stablehlo.batch_norm_training (normalization.nim:120-162): the batch mean and
    the (biased) batch variance per feature, then the inference formula."""
    v = _bn_view(x, fi)
    mean = v.mean(axis=(0, 2))
    var = ((v - mean[None, :, None]) ** 2).mean(axis=(0, 2))
    return batch_norm_inference(x, scale, offset, mean, var, eps, fi), mean, var


def batch_norm_grad(x, scale, mean, var, dy, eps, fi):
    """stablehlo.batch_norm_grad (normalization.nim:164-205): the gradient of
    sum(dy * batch_norm_training(x)) with mean and var the batch statistics."""
    v, g = _bn_view(x, fi), _bn_view(dy, fi)
    n = v.shape[0] * v.shape[2]
    b = lambda t: np.asarray(t, np.float64)[None, :, None]
    std = np.sqrt(b(var) + eps)
    xn = (v - b(mean)) / std
    d_off = g.sum(axis=(0, 2))
    d_sc = (g * xn).sum(axis=(0, 2))
    dx = b(scale) / std * (g - b(d_off) / n - xn * b(d_sc) / n)
    return dx.reshape(np.shape(x)), d_sc, d_off


# ---- composites ------------------------------------------------------------------------

def softmax_rows(x: np.ndarray) -> np.ndarray:
    """src/rew/nn/activation.nim:64-77 over the last axis."""
    x = np.ascontiguousarray(x, np.float32)
    cols = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_softmax_rows(_p(x), C.c_int64(x.size // cols), C.c_int64(cols), _p(out))
    return out


def rmsnorm_rows(x: np.ndarray, gamma: np.ndarray, eps: float = 1e-5) -> np.ndarray:
    """src/rew/nn/norm.nim:204-224 over the last axis."""
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(gamma, np.float32)
    cols = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_rmsnorm_rows(_p(x), _p(g), C.c_int64(x.size // cols), C.c_int64(cols),
                           C.c_float(eps), _p(out))
    return out


def layernorm_rows(x: np.ndarray, gamma: np.ndarray, beta: np.ndarray,
                   eps: float = 1e-5) -> np.ndarray:
    """src/rew/nn/norm.nim:41-84 over the last axis."""
    x = np.ascontiguousarray(x, np.float32)
    g = np.ascontiguousarray(gamma, np.float32)
    b = np.ascontiguousarray(beta, np.float32)
    cols = x.shape[-1]
    out = np.empty_like(x)
    lib().orc_layernorm_rows(_p(x), _p(g), _p(b), C.c_int64(x.size // cols), C.c_int64(cols),
                             C.c_float(eps), _p(out))
    return out


def rope(x: np.ndarray, cos_t: np.ndarray, sin_t: np.ndarray, offset: int = 0) -> np.ndarray:
    """src/rew/nn/rope.nim:56-108, 153-179; x [..., S, D]."""
    x = np.ascontiguousarray(x, np.float32)
    S, D = x.shape[-2], x.shape[-1]
    out = np.empty_like(x)
    ct = np.ascontiguousarray(cos_t, np.float32)
    st = np.ascontiguousarray(sin_t, np.float32)
    lib().orc_rope(_p(x), _p(ct), _p(st), C.c_int64(x.size // (S * D)), C.c_int64(S),
                   C.c_int64(D), C.c_int64(offset), _p(out))
    return out


def rope_tables(head_dim: int, max_seq: int, theta: float):
    """initRotaryPositionEncoding (src/rew/nn/rope.nim:112-145) in float32 C-like steps."""
    half = head_dim // 2
    inv = np.array([np.float32(1.0) / np.float32(theta ** (float(2 * i) / float(head_dim)))
                    for i in range(half)], np.float32)
    ang = (np.arange(max_seq, dtype=np.float32)[:, None] * inv[None, :]).astype(np.float32)
    c = unary(COS, ang)
    s = unary(SIN, ang)
    return np.repeat(c, 2, axis=1), np.repeat(s, 2, axis=1)


def sdpa(q, k, v, causal, scale: float | None = None, mixed: bool = False) -> np.ndarray:
    """src/rew/nn/attention.nim:36-81 with GQA sharing (groupedqueryattention.nim:126-133).
    q [B,H,Sq,D], k/v [B,Hkv,Sk,D] as float arrays (bf16-valued when mixed).
    causal: False/0 unmasked, True/1 rew's makeCausalMask (i <= j visible),
    2 the mirrored mask (i >= j visible), 3 / 4 the strict forms (i < j /
    i > j visible); masked scores get -1e9 added."""
    q = np.ascontiguousarray(q, np.float32)
    k = np.ascontiguousarray(k, np.float32)
    v = np.ascontiguousarray(v, np.float32)
    B, H, Sq, D = q.shape
    Hkv, Sk = k.shape[1], k.shape[2]
    sc = np.float32(1.0) / np.sqrt(np.float32(D)) if scale is None else np.float32(scale)
    out = np.empty_like(q)
    lib().orc_sdpa(_p(q), _p(k), _p(v), C.c_int64(B), C.c_int64(H), C.c_int64(Hkv),
                   C.c_int64(Sq), C.c_int64(Sk), C.c_int64(D), C.c_int(int(causal)),
                   C.c_float(sc), C.c_int(1 if mixed else 0), _p(out))
    return out


def argmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    cols = x.shape[-1]
    out = np.empty(x.shape[:-1], np.int32)
    lib().orc_argmax_rows(_p(x), C.c_int64(x.size // cols), C.c_int64(cols), _p(out))
    return out


def topk_rows(x: np.ndarray, k: int):
    x = np.ascontiguousarray(x, np.float32)
    cols = x.shape[-1]
    rows = x.size // cols
    vals = np.empty(x.shape[:-1] + (k,), np.float32)
    idx = np.empty(x.shape[:-1] + (k,), np.int32)
    lib().orc_topk_rows(_p(x), C.c_int64(rows), C.c_int64(cols), C.c_int64(k), _p(vals), _p(idx))
    return vals, idx


# ---- layer oracles (mixed-precision op sequences) ---------------------------------------

def linear(x, w, b, bf16: bool):
    """Linear.forward (src/rew/nn/linear.nim:43-49): matmul then broadcast bias add."""
    xw = gemm(x, w, round_bf16_out=bf16)
    y = binary(ADD, xw, np.broadcast_to(b, xw.shape))
    return round_bf16(y) if bf16 else y


def silu(x):
    """activation.nim:28-38: x * (1 / (1 + exp(-x)))."""
    one = np.ones_like(x)
    return binary(MUL, x, binary(DIV, one, binary(ADD, one, unary(EXP, unary(NEG, x)))))


def gated_ffn(x2d, wg, bg, wu, bu, wd, bd, bf16: bool):
    """GatedFeedForward.forward (src/rew/nn/gated_ffn.nim:46-67), mixed precision."""
    g = linear(x2d, wg, bg, bf16)
    u = linear(x2d, wu, bu, bf16)
    h = binary(MUL, silu(g), u)
    if bf16:
        h = round_bf16(h)
    return linear(h, wd, bd, bf16)


def gqa(x3d, p, nh, nkv, cos_t, sin_t, causal: bool, bf16: bool):
    """GroupedQueryAttention.forward (src/rew/nn/groupedqueryattention.nim:75-144)."""
    B, S, E = x3d.shape
    hd = E // nh
    x2 = x3d.reshape(B * S, E)
    qp = linear(x2, p["wq"], p["bq"], bf16).reshape(B, S, nh, hd).transpose(0, 2, 1, 3)
    kp = linear(x2, p["wk"], p["bk"], bf16).reshape(B, S, nkv, hd).transpose(0, 2, 1, 3)
    vp = linear(x2, p["wv"], p["bv"], bf16).reshape(B, S, nkv, hd).transpose(0, 2, 1, 3)
    qr = rope(qp, cos_t, sin_t)
    kr = rope(kp, cos_t, sin_t)
    if bf16:
        qr, kr = round_bf16(qr), round_bf16(kr)
    att = sdpa(qr, kr, vp, causal, mixed=bf16)
    a2 = np.ascontiguousarray(att.transpose(0, 2, 1, 3)).reshape(B * S, E)
    return linear(a2, p["wo"], p["bo"], bf16).reshape(B, S, E)


def llama_layer(x3d, p, nh, nkv, cos_t, sin_t, eps=1e-5, causal=True, bf16=True,
                norm="rms"):
    """LlamaDecoderLayer.forward (src/rew/models/llama.nim:106-117) as the
    mixed-precision op sequence: fp32 norms, bf16 contractions, bf16 residuals."""
    B, S, E = x3d.shape

    def nrm(h, g):
        h2 = h.reshape(B * S, E)
        if norm == "rms":
            y = rmsnorm_rows(h2, g, eps)
        else:
            y = layernorm_rows(h2, g, np.zeros_like(g), eps)
        y = y.reshape(B, S, E)
        return round_bf16(y) if bf16 else y

    normed = nrm(x3d, p["g1"])
    attn = gqa(normed, p, nh, nkv, cos_t, sin_t, causal, bf16)
    res = binary(ADD, x3d, attn)
    if bf16:
        res = round_bf16(res)
    normed2 = nrm(res, p["g2"])
    mlp = gated_ffn(normed2.reshape(B * S, E), p["wg"], p["bg"], p["wu"], p["bu"], p["wd"],
                    p["bd"], bf16).reshape(B, S, E)
    out = binary(ADD, res, mlp)
    return round_bf16(out) if bf16 else out


def deepseek_moe(x2d, shared, routed, wr, br, k):
    """DeepSeekMoE.forward (src/rew/models/deepseek.nim:114-145) as the
    mixed-precision op sequence rew_amd.nn emits: bf16 expert FFNs, an fp32
    router on astype(x), topK, renormalisation, and the dense expert loop
    out = bf16(out + bf16(f32(E_e(x)) * w_e)) in expert order.
    shared / routed: lists of (wg, bg, wu, bu, wd, bd) float arrays holding
    bf16 values.  Returns (out, topk indices, renormalised weights)."""
    x = np.ascontiguousarray(x2d, np.float32)
    T, H = x.shape
    out = gated_ffn(x, *shared[0], True) if shared else np.zeros((T, H), np.float32)
    for s in shared[1:]:
        out = round_bf16(binary(ADD, out, gated_ffn(x, *s, True)))
    probs = softmax_rows(linear(x, wr, br, False))
    tv, ti = topk_rows(probs, k)
    denom = reduce(RSUM, tv, [1])
    tw = binary(DIV, tv, np.ascontiguousarray(np.broadcast_to(denom[:, None], tv.shape)))
    for e, ex in enumerate(routed):
        w = reduce(RSUM, binary(MUL, tw, (ti == e).astype(np.float32)), [1])
        y = gated_ffn(x, *ex, True)
        contrib = round_bf16(binary(MUL, y, np.ascontiguousarray(np.broadcast_to(w[:, None], y.shape))))
        out = round_bf16(binary(ADD, out, contrib))
    return out, ti, tw
