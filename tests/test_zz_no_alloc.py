"""GPU check of rew_mi355x_moe_routed_ffn_noalloc, the allocation-free form
of rew_mi355x_moe_routed_ffn: its working memory is a static device array
instead of caching-allocator blocks, and the caller passes every input and
the output.  Checked bit for bit against the allocating entry point on two
calls in a row, the second with a smaller input (fewer tokens, a shorter
expert chain), since the array keeps the previous call's contents; and a
call needing more working memory than the array holds is refused on the
host with ERR_INVALID before anything is launched."""
import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import _lib
from rew_amd import eager as E
from rew_amd import ops as O
from rew_amd.eager import DType

from test_gpu_moe import build_moe

SCRATCH_BYTES = 64 << 20


def _noalloc(x, start, topW, topI, experts, ids, width):
    lib = _lib.load()
    fn = lib.rew_mi355x_moe_routed_ffn_noalloc
    fn.restype = C.c_int
    fn.argtypes = [C.c_void_p, C.c_void_p]
    out = E.empty(DType.BFLOAT16, x.shape)
    a, keep = E._moe_args(x, start, topW, topI, experts, ids, width, out)
    rc = fn(E.context(), C.byref(a))
    return rc, out


def _case(oracle, T, chain, seed):
    moe, host = build_moe(oracle, T, 256, 128, 16, 4, 1, seed)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    start = moe.sharedExperts[0].forward(xt)
    topW, topI = moe.route(xt)
    experts = [moe.routedExperts[e] for e in chain]
    ref = E.toHost(E.moeRoutedFfn(xt, start, topW, topI, experts, chain, 16))
    rc, out = _noalloc(xt, start, topW, topI, experts, chain, 16)
    assert rc == 0, _lib.load().rew_mi355x_last_error()
    return ref, E.toHost(out)


def test_noalloc_matches_allocating_entry_point(gpu, oracle):
    ref1, got1 = _case(oracle, 256, list(range(16)), 0x5EED0605)
    np.testing.assert_array_equal(got1, ref1)
    # second call: fewer tokens and a shorter chain reuse the same array
    ref2, got2 = _case(oracle, 100, [2, 5, 9, 14], 0x5EED0606)
    np.testing.assert_array_equal(got2, ref2)
    assert not np.array_equal(got2, ref1[:100])


def test_noalloc_refuses_more_than_its_scratch(gpu, oracle):
    moe, host = build_moe(oracle, 16, 256, 128, 16, 4, 1, 0x5EED0607)
    xt = E.fromHost(host["x"], DType.BFLOAT16)
    start = moe.sharedExperts[0].forward(xt)
    topW, topI = moe.route(xt)
    out = E.empty(DType.BFLOAT16, xt.shape)
    a, keep = E._moe_args(xt, start, topW, topI, moe.routedExperts, list(range(16)), 16, out)
    # 100000 tokens x 4 slots of (256 + 128) bf16 columns: about 307 MB of
    # working memory, far above the array; refused before any launch
    a.tokens = 100000
    need = 100000 * 4 * (256 + 128) * 2
    assert need > SCRATCH_BYTES
    lib = _lib.load()
    fn = lib.rew_mi355x_moe_routed_ffn_noalloc
    fn.restype = C.c_int
    fn.argtypes = [C.c_void_p, C.c_void_p]
    assert fn(E.context(), C.byref(a)) == 1
    msg = lib.rew_mi355x_last_error()
    assert b"static scratch holds" in msg, msg
    # the context keeps working
    x = np.arange(8, dtype=np.float32)
    np.testing.assert_array_equal(E.toHost(O.add(E.fromHost(x), E.fromHost(x))), x + x)
