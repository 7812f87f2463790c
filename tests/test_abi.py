"""CPU checks of librew_mi355x: it loads, exports every symbol the header
declares, its host-side generators match the oracle bit for bit, and its
error paths behave without a GPU (no compute is launched here)."""
import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]


def _declared_symbols():
    text = (ROOT / "include" / "rew_mi355x.h").read_text()
    return sorted(set(re.findall(r"\b(rew_mi355x_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from rew_amd import _lib
    lib = _lib.load()
    names = _declared_symbols()
    assert len(names) >= 25
    for n in names:
        assert hasattr(lib, n), f"librew_mi355x.so does not export {n}"
    assert set(names) == set(_lib.SIGNATURES), "ctypes table out of sync with the header"
    assert lib.rew_mi355x_abi_version() == 3


def test_stats_struct_matches_header():
    from rew_amd import _lib
    text = (ROOT / "include" / "rew_mi355x.h").read_text()
    body = re.search(r"typedef struct rew_mi355x_stats \{(.*?)\} rew_mi355x_stats;", text, re.S)
    fields = re.findall(r"int64_t\s+([a-z_0-9]+);", body.group(1))
    assert [n for n, _ in _lib.Stats._fields_] == fields


def test_rng_matches_oracle(oracle):
    from rew_amd import _lib
    lib = _lib.load()
    key = oracle.init_key(0x5EED0002)
    for n in (1, 7, 100003):
        u = np.empty(n, np.float32)
        lib.rew_mi355x_rng_uniform_f32(key[0], key[1], n, -0.5, 0.25,
                                       u.ctypes.data_as(C.c_void_p))
        np.testing.assert_array_equal(u, oracle.uniform_f32(key, n, -0.5, 0.25))
        z = np.empty(n, np.float32)
        lib.rew_mi355x_rng_normal_f32(key[0], key[1], n, 0.0, 0.02,
                                      z.ctypes.data_as(C.c_void_p))
        np.testing.assert_array_equal(z, oracle.normal_f32(key, n, 0.0, 0.02))
    out = (C.c_uint32 * 8)()
    lib.rew_mi355x_rng_split(key[0], key[1], 4, out)
    assert [(out[2 * i], out[2 * i + 1]) for i in range(4)] == oracle.split(key, 4)
    lib.rew_mi355x_rng_fold_in(key[0], key[1], 123456789012, out)
    assert (out[0], out[1]) == oracle.fold_in(key, 123456789012)


def test_error_paths_without_device():
    from rew_amd import _lib
    lib = _lib.load()
    n = C.c_int(-1)
    assert lib.rew_mi355x_device_count(C.byref(n)) == 0
    if n.value > 0:
        pytest.skip("a HIP device is visible; the no-device path is not reachable")
    ctx = C.c_void_p()
    rc = lib.rew_mi355x_init(0, C.byref(ctx))
    assert rc == 3  # REW_MI355X_ERR_DEVICE
    assert b"not present" in lib.rew_mi355x_last_error()
    # null / released handles never crash
    lib.rew_mi355x_release(None)
    rc = lib.rew_mi355x_to_host(C.c_void_p(0x1234), None, 0)
    assert rc == 5  # REW_MI355X_ERR_RELEASED
    assert b"released" in lib.rew_mi355x_last_error()
    rc = lib.rew_mi355x_execute(None, b"add", None, 0, None, None, 0, None, 0, None)
    assert rc == 1 and b"null context" in lib.rew_mi355x_last_error()
    rc = lib.rew_mi355x_alloc(None, 11, None, 0, C.byref(C.c_void_p()))
    assert rc == 1 and b"null context" in lib.rew_mi355x_last_error()
    rc = lib.rew_mi355x_buf_device_ptr(C.c_void_p(0x1234), C.byref(C.c_void_p()))
    assert rc == 5 and b"released" in lib.rew_mi355x_last_error()
    rc = lib.rew_mi355x_moe_routed_ffn(None, None)
    assert rc == 1 and b"null context" in lib.rew_mi355x_last_error()


@pytest.mark.parametrize("ordinal", [-1, 64, 1 << 30])
def test_bad_device_ordinal(ordinal):
    """An ordinal outside the device table is refused before any HIP call,
    as rew's selectDevice refuses an ordinal past the client's devices
    (src/rew/eager.nim:160-172)."""
    from rew_amd import _lib
    lib = _lib.load()
    ctx = C.c_void_p()
    assert lib.rew_mi355x_init(ordinal, C.byref(ctx)) == 1  # REW_MI355X_ERR_INVALID
    assert b"ordinal" in lib.rew_mi355x_last_error()
    assert not ctx.value


def test_plugin_path_resolution(tmp_path, monkeypatch):
    """The library is resolved like rew's resolvePluginPath
    (src/rew/binaries/resolver.nim:22-78): REW_PJRT_PLUGIN_PATH directories
    in order, then REW_BUILD, then the in-tree build."""
    import shutil
    from rew_amd import _lib
    a, b = tmp_path / "a", tmp_path / "b"
    a.mkdir()
    b.mkdir()
    shutil.copy(_lib.LIB_PATH, b / _lib.LIB_NAME)
    monkeypatch.setenv("REW_PJRT_PLUGIN_PATH", f"{a}:{b}")
    assert _lib.resolve_plugin_path() == b / _lib.LIB_NAME
    monkeypatch.setenv("REW_PJRT_PLUGIN_PATH", str(a))
    assert _lib.resolve_plugin_path() == _lib.LIB_PATH
    monkeypatch.setenv("REW_BUILD", "true")
    assert _lib.resolve_plugin_path() == _lib.LIB_PATH
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "missing" / _lib.LIB_NAME)
    with pytest.raises(_lib.ResolveError, match="REW_BUILD=true"):
        _lib.resolve_plugin_path()
    monkeypatch.delenv("REW_BUILD")
    with pytest.raises(_lib.ResolveError, match="not found"):
        _lib.resolve_plugin_path()


def test_library_carries_its_run_time_headers():
    """The headers the run-time compiled kernels include are in the library
    itself, so a lone copy of the .so needs no source tree."""
    data = (ROOT / "rew_amd" / "librew_mi355x.so").read_bytes()
    for name in ("vm_device.h", "rtc_prelude.h", "vm.h", "rew_mi355x.h"):
        assert name.encode() in data
    assert b"namespace vm" in data and b"Fused elementwise programs" in data
