"""GPU checks of complex / real / imag (src/rew/ops/arith.nim:86-106,
unary.nim:184-224) and fft (src/rew/ops/linalg.nim:328-348) against numpy:
the parts bit for bit, the transforms within 1e-5 normwise for complex64
(each axis an exact-length DFT summed in double)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

from rew_amd import eager as E
from rew_amd import ops as O
from rew_amd.eager import DType, EagerError


def crnd(shape, seed, dt=np.complex64):
    g = np.random.default_rng(seed)
    return (g.standard_normal(shape) + 1j * g.standard_normal(shape)).astype(dt)


def close(got, want, tol=1e-5):
    assert got.shape == want.shape and got.dtype == want.dtype, (got.shape, got.dtype, want.dtype)
    err = np.linalg.norm(got - want) / max(np.linalg.norm(want), 1e-30)
    assert err <= tol, err


@pytest.mark.parametrize("dt,cdt", [(np.float32, np.complex64), (np.float64, np.complex128)])
def test_complex_real_imag(gpu, dt, cdt):
    g = np.random.default_rng(1)
    re, im = g.standard_normal((3, 5)).astype(dt), g.standard_normal((3, 5)).astype(dt)
    z = O.complex(E.fromHost(re), E.fromHost(im))
    assert z.dtype == (DType.COMPLEX64 if dt == np.float32 else DType.COMPLEX128)
    assert E.toHost(z).tolist() == (re + 1j * im).astype(cdt).tolist()
    assert E.toHost(O.real(z)).tolist() == re.tolist()
    assert E.toHost(O.imag(z)).tolist() == im.tolist()
    # of a real tensor: itself and zeros
    assert E.toHost(O.real(E.fromHost(re))).tolist() == re.tolist()
    assert E.toHost(O.imag(E.fromHost(re))).tolist() == np.zeros_like(re).tolist()


@pytest.mark.parametrize("shape,k", [((3, 16), 1), ((2, 15), 1), ((2, 8, 6), 2), ((2, 4, 5, 6), 3)])
def test_fft_ifft(gpu, shape, k):
    x = crnd(shape, 2)
    axes = tuple(range(len(shape) - k, len(shape)))
    fl = list(shape[-k:])
    close(E.toHost(O.fft(E.fromHost(x), "FFT", fl)), np.fft.fftn(x, axes=axes).astype(np.complex64))
    close(E.toHost(O.fft(E.fromHost(x), "IFFT", fl)), np.fft.ifftn(x, axes=axes).astype(np.complex64))


@pytest.mark.parametrize("shape,k", [((4, 16), 1), ((3, 15), 1), ((2, 8, 6), 2), ((2, 6, 7), 2)])
def test_rfft_irfft(gpu, shape, k):
    x = np.random.default_rng(3).standard_normal(shape).astype(np.float32)
    axes = tuple(range(len(shape) - k, len(shape)))
    fl = list(shape[-k:])
    spec = E.toHost(O.fft(E.fromHost(x), "RFFT", fl))
    close(spec, np.fft.rfftn(x, axes=axes).astype(np.complex64))
    back = E.toHost(O.fft(E.fromHost(spec), "IRFFT", fl))
    close(back, np.fft.irfftn(spec.astype(np.complex128), s=fl, axes=axes).astype(np.float32))
    close(back, x, 1e-5)


def test_fft_under_jit_equals_eager(gpu):
    from rew_amd import jit as J
    x = np.random.default_rng(6).standard_normal((3, 8, 6)).astype(np.float32)

    def f(a):
        s = O.fft(a[0], "RFFT", [8, 6])
        return [s, O.fft(s, "IRFFT", [8, 6]), O.real(s), O.imag(s)]
    j = J.jit(f, "fftJit")
    assert '"stablehlo.fft"' in j.text([E.fromHost(x)])
    got = [E.toHost(o) for o in j.call([E.fromHost(x)])]
    want = [E.toHost(o) for o in f([E.fromHost(x)])]
    for g_, w_ in zip(got, want):
        assert g_.shape == w_.shape and g_.tolist() == w_.tolist()


def test_fft_f64_and_errors(gpu):
    x = crnd((5, 12), 4, np.complex128)
    close(E.toHost(O.fft(E.fromHost(x), "FFT", [12])), np.fft.fft(x), 1e-12)
    with pytest.raises(EagerError, match="complex"):
        O.fft(E.fromHost(np.ones((4, 8), np.float32)), "FFT", [8])
    with pytest.raises(EagerError, match="fftLength"):
        O.fft(E.fromHost(crnd((4, 8), 5)), "FFT", [6])
