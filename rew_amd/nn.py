"""Mirror of the rew.nn composites that generate the hot op streams.

Each function emits the same eager op sequence as the cited reference
composite.  The reference layers are fp32-only in places (reductions,
scalar constants, RoPE tables, Linear biases), so bf16 configurations run
them as a *mixed-precision op sequence*: bf16 contractions, with ``astype``
to float32 around the fp32-only composites and back to bf16 before the next
contraction.  For float32 inputs every ``_f32``/``_to`` hop is a no-op and
the sequence is exactly the reference's.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field
from typing import Sequence

import numpy as np

from . import ops as O
from .eager import DType, Tensor, TensorError


def _f32(x: Tensor) -> Tensor:
    return x if x.dtype == DType.FLOAT32 else O.astype(x, DType.FLOAT32)


def _to(x: Tensor, dt: DType) -> Tensor:
    return x if x.dtype == dt else O.astype(x, dt)


# ---- activations (src/rew/nn/activation.nim:21-77) ------------------------------------

def relu(x: Tensor) -> Tensor:
    zero = O.scalarF32(0.0, x.device)
    return O.maximum(x, O.broadcastTo(zero, x.shape, []))


def sigmoid(x: Tensor) -> Tensor:
    one = O.scalarF32(1.0, x.device)
    oneB = O.broadcastTo(one, x.shape, [])
    expNeg = O.exp(O.neg(x))
    return O.divide(oneB, O.add(oneB, expNeg))


def silu(x: Tensor) -> Tensor:
    return O.mul(x, sigmoid(x))


def softmax(x: Tensor, axis: int) -> Tensor:
    maxVal = O.reduceMax(x, [axis])
    bdims = [i for i in range(len(x.shape)) if i != axis]
    maxB = O.broadcastTo(maxVal, x.shape, bdims)
    shifted = O.sub(x, maxB)
    expShifted = O.exp(shifted)
    sumExp = O.reduceSum(expShifted, [axis])
    sumB = O.broadcastTo(sumExp, x.shape, bdims)
    return O.divide(expShifted, sumB)


# ---- normalization (src/rew/nn/norm.nim:41-84, 204-224) ---------------------------------

def rmsNorm(x: Tensor, gamma: Tensor, eps: float = 1e-5) -> Tensor:
    if len(x.shape) == 0:
        raise TensorError("rmsNorm: input must have at least 1 dimension")
    last = len(x.shape) - 1
    sq = O.mul(x, x)
    meanSq = O.reduceMean(sq, [last])
    epsB = O.broadcastTo(O.scalarF32(eps, x.device), meanSq.shape, [])
    rms = O.sqrt(O.add(meanSq, epsB))
    rmsB = O.broadcastTo(rms, x.shape, list(range(last)))
    normed = O.divide(x, rmsB)
    return O.mul(O.broadcastTo(gamma, x.shape, [last]), normed)


@dataclass
class LayerNorm:
    gamma: Tensor
    beta: Tensor
    normalizedShape: Sequence[int]
    eps: float = 1e-5

    @staticmethod
    def init(normalizedShape: Sequence[int], eps: float = 1e-5, device=None) -> "LayerNorm":
        n = int(np.prod(normalizedShape))
        return LayerNorm(O.constantF32(normalizedShape, np.ones(n, np.float32), device),
                         O.constantF32(normalizedShape, np.zeros(n, np.float32), device),
                         list(normalizedShape), eps)

    def forward(self, x: Tensor) -> Tensor:
        nd = len(self.normalizedShape)
        r = len(x.shape)
        if r < nd:
            raise TensorError(
                f"LayerNorm.forward: input rank {r} is less than normalized dims {nd}")
        red = list(range(r - nd, r))
        mean = O.reduceMean(x, red)
        bdims = list(range(r - nd))
        meanB = O.broadcastTo(mean, x.shape, bdims)
        centered = O.sub(x, meanB)
        sq = O.mul(centered, centered)
        variance = O.reduceMean(sq, red)
        epsB = O.broadcastTo(O.scalarF32(self.eps, x.device), variance.shape, [])
        invStd = O.rsqrt(O.add(variance, epsB))
        invStdB = O.broadcastTo(invStd, x.shape, bdims)
        normalized = O.mul(centered, invStdB)
        gammaB = O.broadcastTo(self.gamma, x.shape, red)
        betaB = O.broadcastTo(self.beta, x.shape, red)
        return O.add(O.mul(gammaB, normalized), betaB)


@dataclass
class RMSNorm:
    """rmsNorm with a learnt gamma (the config's RMSNorm, eps 1e-5)."""
    gamma: Tensor
    eps: float = 1e-5

    def forward(self, x: Tensor) -> Tensor:
        return rmsNorm(x, self.gamma, self.eps)


# ---- Linear / gated FFN (src/rew/nn/linear.nim:43-49, gated_ffn.nim:46-67) -------------

@dataclass
class Linear:
    weight: Tensor  # [in, out]
    bias: Tensor    # [out]

    def forward(self, x: Tensor) -> Tensor:
        xw = O.matmul(x, self.weight)
        biasB = O.broadcastTo(self.bias, xw.shape, [1])
        return O.add(xw, biasB)


@dataclass
class GatedFeedForward:
    gateProj: Linear
    upProj: Linear
    downProj: Linear

    def forward(self, x: Tensor) -> Tensor:
        batch, seqLen = x.shape[0], x.shape[1]
        xFlat = O.reshape(x, [batch * seqLen, x.shape[2]])
        gateFlat = self.gateProj.forward(xFlat)
        upFlat = self.upProj.forward(xFlat)
        # mixed precision: SiLU and the gate product run in fp32
        gateAct = silu(_f32(gateFlat))
        hiddenFlat = _to(O.mul(gateAct, _f32(upFlat)), x.dtype)
        outFlat = self.downProj.forward(hiddenFlat)
        return O.reshape(outFlat, [batch, seqLen, outFlat.shape[1]])


# ---- RoPE (src/rew/nn/rope.nim:56-179) ---------------------------------------------------

def rope_tables(headDim: int, maxSeqLen: int, theta: float):
    """cos/sin tables [maxSeqLen, headDim] exactly as initRotaryPositionEncoding
    builds them: f64 pow for invFreq, f32 angles, values duplicated at 2i, 2i+1."""
    half = headDim // 2
    invFreq = np.array([np.float32(1.0) / np.float32(theta ** (float(2 * i) / float(headDim)))
                        for i in range(half)], dtype=np.float32)
    pos = np.arange(maxSeqLen, dtype=np.float32)[:, None]
    angle = (pos * invFreq[None, :]).astype(np.float32)
    c = np.cos(angle).astype(np.float32)
    s = np.sin(angle).astype(np.float32)
    return np.repeat(c, 2, axis=1), np.repeat(s, 2, axis=1)


def applyRotate(x: Tensor, cosTbl: Tensor, sinTbl: Tensor) -> Tensor:
    rank = len(x.shape)
    headDim = x.shape[-1]
    half = headDim // 2
    leading = list(x.shape[:rank - 1])
    pairShape = leading + [half, 2]
    xPairs = O.reshape(x, pairShape)
    pr = len(pairShape)
    starts0 = [0] * pr
    limits0 = list(pairShape[:pr - 2]) + [half, 1]
    strides = [1] * pr
    starts1 = [0] * (pr - 1) + [1]
    limits1 = list(pairShape[:pr - 2]) + [half, 2]
    x0 = O.slice_(xPairs, starts0, limits0, strides)
    x1 = O.slice_(xPairs, starts1, limits1, strides)
    flatShape = list(x0.shape[:-1])
    x0Flat = O.reshape(x0, flatShape)
    x1Flat = O.reshape(x1, flatShape)
    cosPairs = O.reshape(cosTbl, pairShape)
    sinPairs = O.reshape(sinTbl, pairShape)
    cos0 = O.reshape(O.slice_(cosPairs, starts0, limits0, strides), flatShape)
    sin0 = O.reshape(O.slice_(sinPairs, starts0, limits0, strides), flatShape)
    x0Rot = O.sub(O.mul(cos0, x0Flat), O.mul(sin0, x1Flat))
    x1Rot = O.add(O.mul(sin0, x0Flat), O.mul(cos0, x1Flat))
    x0r = O.reshape(x0Rot, flatShape + [1])
    x1r = O.reshape(x1Rot, flatShape + [1])
    xRotated = O.concat([x0r, x1r], len(x0r.shape) - 1)
    return O.reshape(xRotated, list(x.shape))


@dataclass
class RotaryPositionEncoding:
    cosCached: Tensor
    sinCached: Tensor
    theta: float
    headDim: int
    maxSeqLen: int

    @staticmethod
    def init(headDim: int, maxSeqLen: int = 2048, theta: float = 10000.0,
             device=None) -> "RotaryPositionEncoding":
        if headDim <= 0 or headDim % 2:
            raise TensorError(
                f"initRotaryPositionEncoding: headDim must be positive and even, got {headDim}")
        c, s = rope_tables(headDim, maxSeqLen, theta)
        return RotaryPositionEncoding(O.constantF32([maxSeqLen, headDim], c, device),
                                      O.constantF32([maxSeqLen, headDim], s, device),
                                      theta, headDim, maxSeqLen)

    def forward(self, x: Tensor, offset: int = 0) -> Tensor:
        if len(x.shape) < 2:
            raise TensorError("RotaryPositionEncoding.forward: input rank must be at least 2")
        seqLen, headDim = x.shape[-2], x.shape[-1]
        if headDim != self.headDim:
            raise TensorError("RotaryPositionEncoding.forward: headDim mismatch")
        total = offset + seqLen
        if total > self.maxSeqLen:
            raise TensorError(
                f"RotaryPositionEncoding.forward: position {total} exceeds maxSeqLen "
                f"{self.maxSeqLen}")
        rank = len(x.shape)
        cosS = O.slice_(self.cosCached, [offset, 0], [total, headDim], [1, 1])
        sinS = O.slice_(self.sinCached, [offset, 0], [total, headDim], [1, 1])
        cosB = O.broadcastTo(cosS, x.shape, [rank - 2, rank - 1])
        sinB = O.broadcastTo(sinS, x.shape, [rank - 2, rank - 1])
        # mixed precision: the tables are fp32, so the rotation runs in fp32
        return _to(applyRotate(_f32(x), cosB, sinB), x.dtype)


# ---- attention (src/rew/nn/attention.nim:18-81) ------------------------------------------

def makeCausalMask(shape: Sequence[int], device=None) -> Tensor:
    """0 where row <= col, -1e9 where row > col (src/rew/nn/attention.nim:18-34).

    Note the orientation: applied to scores[query, key] it lets query i see
    keys j >= i.  This is the reference's behaviour and is reproduced as is.
    """
    if len(shape) != 2:
        raise TensorError(f"makeCausalMask: shape must be rank-2 (seqLen, kvLen), got {shape}")
    rows = O.iota(DType.INT32, shape, 0, device)
    cols = O.iota(DType.INT32, shape, 1, device)
    upper = O.compare(rows, cols, "LE")
    negInfB = O.broadcastTo(O.scalarF32(-1e9, device), shape, [])
    zeroB = O.broadcastTo(O.scalarF32(0.0, device), shape, [])
    return O.select(upper, zeroB, negInfB)


def scaledDotProductAttention(q: Tensor, k: Tensor, v: Tensor, causal: bool = False,
                              scale: float = 0.0) -> Tensor:
    if len(q.shape) < 2 or len(k.shape) < 2 or len(v.shape) < 2:
        raise TensorError("scaledDotProductAttention: operands must have rank >= 2")
    rank = len(q.shape)
    batchDims = list(range(rank - 2))
    sc = scale if scale != 0.0 else float(np.float32(1.0) / np.sqrt(np.float32(q.shape[-1])))
    scores = O.dotGeneral(q, k, batchDims, batchDims, [rank - 1], [rank - 1])
    scores = _f32(scores)  # mixed precision: scale/mask/softmax in fp32
    scores = O.mul(scores, O.broadcastTo(O.scalarF32(sc, q.device), scores.shape, []))
    if causal:
        seqLen, kvLen = scores.shape[-2], scores.shape[-1]
        mask = makeCausalMask([seqLen, kvLen], q.device)
        maskB = O.broadcastTo(mask, scores.shape, [len(scores.shape) - 2, len(scores.shape) - 1])
        scores = O.add(scores, maskB)
    attn = softmax(scores, len(scores.shape) - 1)
    attn = _to(attn, v.dtype)
    return O.dotGeneral(attn, v, batchDims, batchDims, [rank - 1], [rank - 2])


@dataclass
class GroupedQueryAttention:
    qProj: Linear
    kProj: Linear
    vProj: Linear
    outProj: Linear
    numHeads: int
    numKVHeads: int
    headDim: int
    rope: RotaryPositionEncoding | None = None

    def forward(self, q: Tensor, k: Tensor, v: Tensor, causal: bool = False,
                offset: int = 0) -> Tensor:
        batch, seqLen, kvLen = q.shape[0], q.shape[1], k.shape[1]
        kvh, nh, hd = self.numKVHeads, self.numHeads, self.headDim
        groupSize = nh // kvh
        qFlat = O.reshape(q, [batch * seqLen, q.shape[2]])
        kFlat = O.reshape(k, [batch * kvLen, k.shape[2]])
        vFlat = O.reshape(v, [batch * kvLen, v.shape[2]])
        qpFlat = self.qProj.forward(qFlat)
        kpFlat = self.kProj.forward(kFlat)
        vpFlat = self.vProj.forward(vFlat)
        qp = O.reshape(qpFlat, [batch, seqLen, qpFlat.shape[1]])
        kp = O.reshape(kpFlat, [batch, kvLen, kpFlat.shape[1]])
        vp = O.reshape(vpFlat, [batch, kvLen, vpFlat.shape[1]])
        qr = O.transpose(O.reshape(qp, [batch, seqLen, nh, hd]), [0, 2, 1, 3])
        kr = O.transpose(O.reshape(kp, [batch, kvLen, kvh, hd]), [0, 2, 1, 3])
        vr = O.transpose(O.reshape(vp, [batch, kvLen, kvh, hd]), [0, 2, 1, 3])
        qrRoped = self.rope.forward(qr, offset) if self.rope else qr
        krRoped = self.rope.forward(kr, offset) if self.rope else kr
        kExpand = O.reshape(krRoped, [batch, kvh, 1, kvLen, hd])
        kVExp = O.broadcastTo(kExpand, [batch, kvh, groupSize, kvLen, hd], [0, 1, 2, 3, 4])
        kFull = O.reshape(kVExp, [batch, nh, kvLen, hd])
        vExpand = O.reshape(vr, [batch, kvh, 1, kvLen, hd])
        vVExp = O.broadcastTo(vExpand, [batch, kvh, groupSize, kvLen, hd], [0, 1, 2, 3, 4])
        vFull = O.reshape(vVExp, [batch, nh, kvLen, hd])
        attnOut = scaledDotProductAttention(qrRoped, kFull, vFull, causal=causal)
        attnT = O.transpose(attnOut, [0, 2, 1, 3])
        attnFlat = O.reshape(attnT, [batch, seqLen, nh * hd])
        attnFlat2d = O.reshape(attnFlat, [batch * seqLen, attnFlat.shape[2]])
        outFlat = self.outProj.forward(attnFlat2d)
        return O.reshape(outFlat, [batch, seqLen, outFlat.shape[1]])


# ---- models (src/rew/models/llama.nim:106-117, deepseek.nim:74-145) -----------------------

@dataclass
class LlamaDecoderLayer:
    selfAttn: GroupedQueryAttention
    mlp: GatedFeedForward
    inputLayernorm: object      # LayerNorm (reference) or RMSNorm (config)
    postAttentionLayernorm: object

    def forward(self, x: Tensor, causal: bool = True, offset: int = 0) -> Tensor:
        normed = _to(self.inputLayernorm.forward(_f32(x)), x.dtype)
        attn = self.selfAttn.forward(normed, normed, normed, causal=causal, offset=offset)
        res = O.add(x, attn)
        normed2 = _to(self.postAttentionLayernorm.forward(_f32(res)), x.dtype)
        mlp = self.mlp.forward(normed2)
        return O.add(res, mlp)


@dataclass
class Embedding:
    weight: Tensor  # [vocab, embed]

    def forward(self, indices: Tensor) -> Tensor:
        """One-hot [..., vocab] x weight (src/rew/nn/embedding.nim:39-62)."""
        vocab = self.weight.shape[0]
        if len(indices.shape) < 2 or indices.shape[-1] != vocab:
            raise TensorError("Embedding.forward: indices must be [..., vocabSize] one-hot")
        lead = int(np.prod(indices.shape[:-1]))
        emb2d = O.matmul(O.reshape(indices, [lead, vocab]), self.weight)
        return O.reshape(emb2d, list(indices.shape[:-1]) + [self.weight.shape[1]])

    def lookup(self, ids: Tensor) -> Tensor:
        """Row gather; equal to ``forward(one_hot(ids))`` (one nonzero product per sum)."""
        return O.torchIndexSelect(self.weight, ids, 0, 0)


@dataclass
class DeepSeekExpert:
    gateProj: Linear
    upProj: Linear
    downProj: Linear

    def forward(self, x: Tensor) -> Tensor:
        gate = silu(_f32(self.gateProj.forward(x)))
        up = _f32(self.upProj.forward(x))
        hidden = _to(O.mul(gate, up), x.dtype)
        return self.downProj.forward(hidden)


def routedWeightForExpert(topWeights: Tensor, topIndices: Tensor, expertIdx: int) -> Tensor:
    idB = O.broadcastTo(O.scalarI32(expertIdx, topIndices.device), topIndices.shape, [])
    mask = O.astype(O.compare(topIndices, idB, "EQ"), DType.FLOAT32)
    return O.reduceSum(O.mul(topWeights, mask), [1])


@dataclass
class DeepSeekMoE:
    gate: Linear                 # router, fp32 [hidden, numRouted]
    sharedExperts: list
    routedExperts: list
    numExpertsPerTok: int

    def route(self, hiddenFlat: Tensor):
        """softmax(L_r(x)) -> top-k -> renormalised weights (deepseek.nim:132-137)."""
        logits = self.gate.forward(_f32(hiddenFlat))
        probs = softmax(logits, 1)
        topW, topI = O.topK(probs, self.numExpertsPerTok, 1, True)
        denom = O.reduceSum(topW, [1])
        topWeights = O.divide(topW, O.broadcastTo(denom, topW.shape, [0]))
        return topWeights, topI

    def forward(self, hiddenFlat: Tensor) -> Tensor:
        """DeepSeekMoE.forward (deepseek.nim:122-145): shared experts, then every
        routed expert on every token weighted by its (mostly zero) routing
        weight, added in expert order.  The backend recognises the chain and
        evaluates each expert only on its routed tokens (exactly the same sum:
        every skipped term is an exact zero)."""
        out = (self.sharedExperts[0].forward(hiddenFlat) if self.sharedExperts
               else O.zerosLike(hiddenFlat))
        for e in self.sharedExperts[1:]:
            out = O.add(out, e.forward(hiddenFlat))
        topWeights, topI = self.route(hiddenFlat)
        for idx, e in enumerate(self.routedExperts):
            w = routedWeightForExpert(topWeights, topI, idx)
            wB = O.broadcastTo(O.unsqueeze(w, 1), list(hiddenFlat.shape), [0, 1])
            y = _f32(e.forward(hiddenFlat))
            contrib = _to(O.mul(y, wB), hiddenFlat.dtype)
            out = O.add(out, contrib)
        return out

    forward_dense = forward


# ---- parameter lists for jit / lazy ----------------------------------------------------
# rew's jit traces a function of tensors only (an eager tensor closed over by
# a traced function is a mode error, src/rew/tensor.nim:177-186), so a layer
# runs under jit/lazy with its parameters passed as arguments and rebuilt
# from the argument list inside the traced function.

def moeParams(moe: "DeepSeekMoE") -> list:
    """The router's weight and bias, then every expert's gate/up/down
    weight and bias (shared experts first)."""
    out = [moe.gate.weight, moe.gate.bias]
    for e in list(moe.sharedExperts) + list(moe.routedExperts):
        for lin in (e.gateProj, e.upProj, e.downProj):
            out += [lin.weight, lin.bias]
    return out


def moeFromParams(params, numShared: int, numRouted: int, numExpertsPerTok: int) -> "DeepSeekMoE":
    """Inverse of moeParams."""
    p = list(params)
    gate = Linear(p[0], p[1])
    experts = []
    for i in range(numShared + numRouted):
        q = p[2 + 6 * i: 8 + 6 * i]
        experts.append(DeepSeekExpert(Linear(q[0], q[1]), Linear(q[2], q[3]), Linear(q[4], q[5])))
    return DeepSeekMoE(gate, experts[:numShared], experts[numShared:], numExpertsPerTok)
