"""GPU parity of the bf16 MFMA GEMM kernels behind dot_general / matmul
(src/rew/ops/linalg.nim:204-256; result dtype = operand dtype).

Both tile kernels (256x256 and 128x128) are forced on ragged shapes through
REW_MI355X_GEMM_TILE in a child process, and compared with the oracle's
fp64-accumulated GEMM on the same bf16 operands rounded once to bf16:
normwise relative error <= 2e-2 and every element within 2 bf16 ulps of the
reference plus the fp32 accumulation bound.
"""
import json
import os
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1]); sys.path.insert(0, sys.argv[1] + "/oracle")
import oracle as orc
from rew_amd import eager as E, ops as O
from rew_amd.eager import DType
E.installEagerBackend(E.mi355x(0))
out = []
for (M, K, N, bt, seed) in json.loads(sys.argv[2]):
    key = orc.init_key(seed)
    a = orc.round_bf16(orc.normal_f32(orc.fold_in(key, 0), M * K).reshape(M, K))
    b = orc.round_bf16(orc.normal_f32(orc.fold_in(key, 1), K * N).reshape(K, N))
    E.profileBegin()
    if bt:   # B given as [N, K] (K-contiguous): dot_general contracting dim 1 of both
        c = O.dotGeneral(E.fromHost(a, DType.BFLOAT16), E.fromHost(np.ascontiguousarray(b.T), DType.BFLOAT16), [], [], [1], [1])
    else:
        c = O.matmul(E.fromHost(a, DType.BFLOAT16), E.fromHost(b, DType.BFLOAT16))
    got = E.toHostF32(c)
    names = [n for n, _, _ in E.profileEnd()]
    want = orc.gemm(a, b, round_bf16_out=True)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    err = float(np.linalg.norm(got - want) / np.linalg.norm(want))
    # per element: |got - exact| <= 2 bf16 ulps of |exact| + fp32 accumulation bound
    bound = 2 * 2.0 ** -8 * np.abs(exact) + K * 2.0 ** -23 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))
    worst = float(np.max(np.abs(got - exact) - bound))
    out.append({"shape": [M, K, N, bt], "err": err, "worst": worst, "kernels": names})
print(json.dumps(out))
"""

SHAPES = [  # M, K, N, B given transposed
    (512, 256, 768, 0),
    (300, 200, 520, 0),
    (257, 72, 264, 1),
    (1024, 1000, 256, 0),
    (256, 64, 256, 1),
    (40, 136, 1032, 0),
    (300, 1000, 520, 1),   # K tail (1000 % 64) with B K-contiguous
    (513, 4104, 1024, 0),  # K tail, M tail, several k-tiles
    (333, 192, 264, 0),    # K % 64 == 0 with 6 k-tiles: a ring turn plus a two-step remainder
    (200, 320, 512, 1),    # the same with B K-contiguous, 10 k-tiles
    (64, 128, 64, 0),      # exactly one ring turn, M and N far below a tile
]


@pytest.mark.parametrize("tile", ["lds", "256", "128"])
def test_gemm_tiles_match_oracle(gpu, oracle, tile):
    env = dict(os.environ, REW_MI355X_GEMM_TILE=tile)
    r = subprocess.run([sys.executable, "-c", CHILD, str(ROOT),
                        json.dumps([list(s) + [31 + i] for i, s in enumerate(SHAPES)])],
                       env=env, capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    for item in res:
        prefix = {"lds": "gemm_lds", "256": "gemm_bf16_256", "128": "gemm_bf16_mfma"}[tile]
        assert any(k.startswith(prefix) for k in item["kernels"]), item
        assert item["err"] <= 2e-2, item
        assert item["worst"] <= 0.0, item
