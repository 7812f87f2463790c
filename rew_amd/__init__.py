"""rew_amd: MI355X-native eager backend for rew (bitstormFA/rew).

The product is ``librew_mi355x.so`` (C ABI in include/rew_mi355x.h, HIP
kernels for gfx950 under csrc/).  The Python modules mirror rew's host
surface over that ABI: ``eager`` (dispatcher, tensors, transfers), ``ops``
(the ``{.rewOp.}`` procs) and ``nn`` (the layer composites).
"""
from . import eager, nn, ops  # noqa: F401
from .eager import (DType, Device, Tensor, dispatchEager, fromHost,  # noqa: F401
                    installEagerBackend, mi355x, toHost)
