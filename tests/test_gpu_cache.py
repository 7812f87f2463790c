"""GPU check of the persistent compiled-program cache (the counterpart of
rew's compileWithPersistentCache, src/rew/eager.nim:1557-1618, laid out as
<REW_CACHE_DIR>/<version>/executables, src/rew/binaries/cache.nim:16-54):
a first process compiles its fused programs and stores them; a second
process with the same cache directory loads every one of them and computes
the same bits; REW_EXECUTABLE_CACHE=off stores nothing."""
import json
import os
import subprocess
import sys
from pathlib import Path

import pytest

pytestmark = pytest.mark.gpu

ROOT = Path(__file__).resolve().parents[1]

CHILD = r"""
import json, sys
import numpy as np
sys.path.insert(0, sys.argv[1])
from rew_amd import eager as E, ops as O, nn
E.installEagerBackend(E.mi355x(0))
x = E.fromHost(np.linspace(-2, 2, 8192, dtype=np.float32).reshape(64, 128))
a = nn.silu(O.add(O.mul(x, x), x))                       # fused elementwise program
b = O.reduceSum(nn.relu(O.sub(x, O.mul(x, x))), [1])      # fused reduction program
out = [E.toHost(a).view(np.uint32).tolist(), E.toHost(b).view(np.uint32).tolist()]
s = E.stats()
print(json.dumps({"compiled": s["programs_compiled"], "loaded": s["programs_loaded"],
                  "out": out}))
"""


def run_child(env):
    r = subprocess.run([sys.executable, "-c", CHILD, str(ROOT)], env=env, capture_output=True,
                       text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-3000:]
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_second_process_loads_every_program(gpu, tmp_path):
    env = dict(os.environ, REW_CACHE_DIR=str(tmp_path))
    env.pop("REW_EXECUTABLE_CACHE", None)
    env.pop("REW_MI355X_JIT", None)
    first = run_child(env)
    assert first["compiled"] >= 2 and first["loaded"] == 0, first
    files = sorted((tmp_path / "0.2.0" / "executables").glob("*.hsaco"))
    assert len(files) == first["compiled"]
    second = run_child(env)
    assert second["compiled"] == 0 and second["loaded"] == first["compiled"], second
    assert second["out"] == first["out"]


def test_cache_switch_off_stores_nothing(gpu, tmp_path):
    env = dict(os.environ, REW_CACHE_DIR=str(tmp_path), REW_EXECUTABLE_CACHE="off")
    env.pop("REW_MI355X_JIT", None)
    r = run_child(env)
    assert r["compiled"] >= 2 and r["loaded"] == 0
    assert not list(tmp_path.rglob("*.hsaco"))


def test_damaged_entry_is_recompiled(gpu, tmp_path):
    env = dict(os.environ, REW_CACHE_DIR=str(tmp_path))
    env.pop("REW_EXECUTABLE_CACHE", None)
    env.pop("REW_MI355X_JIT", None)
    first = run_child(env)
    files = sorted((tmp_path / "0.2.0" / "executables").glob("*.hsaco"))
    files[0].write_bytes(b"not a code object")
    again = run_child(env)
    assert again["compiled"] == 1 and again["loaded"] == first["compiled"] - 1, again
    assert again["out"] == first["out"]
