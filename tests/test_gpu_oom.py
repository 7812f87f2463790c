"""A device allocation that fails surfaces as rew's EagerError and leaves the
context usable.

rew reports a failed backend call as an EagerError carrying the message
(src/rew/eager.nim:1751-1754).  The backend fails an allocation with
REW_MI355X_ERR_OOM after trimming its cache and retrying.  To reach that path
deterministically, a child process creates its context under
REW_MI355X_MAX_DEVICE_BYTES (the most device memory the allocator may hold),
then:

* uploads a tensor larger than the limit (fails at fromHost);
* builds a deferred result larger than what is left (fails at its flush);
* keeps computing afterwards: earlier tensors still read back, new work gives
  the right values, and memory freed after the failures can be allocated
  again up to the limit.
"""
import json
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]
CAP = 64 << 20

CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from rew_amd import eager as E, ops as O
E.installEagerBackend(E.mi355x(0))
out = {}
a = E.fromHost(np.arange(1024, dtype=np.float32))
out["small_ok"] = bool(np.array_equal(E.toHost(O.add(a, a)), 2 * np.arange(1024, dtype=np.float32)))
try:
    E.fromHost(np.zeros(20 << 20, np.float32))            # 80 MiB > the limit
    out["upload_err"] = None
except E.EagerError as e:
    out["upload_err"] = str(e)
x = E.fromHost(np.ones((4096, 2048), np.float32))          # 32 MiB resident
z = O.concat([x, x, x], 0)                                 # 96 MiB at its flush
try:
    E.toHost(z)
    out["flush_err"] = None
except E.EagerError as e:
    out["flush_err"] = str(e)
del z
out["x_ok"] = bool(np.all(E.toHost(O.reduceSum(x, [1])) == 2048.0))
b = E.fromHost(np.full(4096, 3.0, np.float32))
out["after_ok"] = bool(np.all(E.toHost(O.mul(b, b)) == 9.0))
del x
y = E.fromHost(np.ones((3 << 20,), np.float32))            # 12 MiB
w = O.concat([y, y, y, y], 0)                              # 48 MiB: fits once x is gone
out["refill_ok"] = bool(np.all(E.toHost(w) == 1.0))
print(json.dumps(out))
"""


def test_allocation_failure_is_eager_error(gpu):
    env = dict(__import__("os").environ, REW_MI355X_MAX_DEVICE_BYTES=str(CAP))
    r = subprocess.run([sys.executable, "-c", CHILD, str(ROOT)], env=env,
                       capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    assert res["small_ok"], res
    for key in ("upload_err", "flush_err"):
        msg = res[key]
        assert msg is not None, res
        assert "device allocation of" in msg and "failed on mi355x:0" in msg, msg
        assert f"REW_MI355X_MAX_DEVICE_BYTES = {CAP}" in msg, msg
    assert res["x_ok"] and res["after_ok"] and res["refill_ok"], res
