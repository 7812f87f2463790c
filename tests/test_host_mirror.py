"""The host mirror of rew's dispatcher and ops, checked through a fake
backend (the reference's own drop-in seam, tests/tdispatch_arith.nim:65-88):
op names and attrs reach the backend in rew's wire format, validation
errors fire before dispatch, and a missing backend raises."""
import pytest

from rew_amd import eager, nn
from rew_amd import ops as O
from rew_amd.eager import DType, Tensor, TensorError


class FakeBackend:
    def __init__(self):
        self.calls = []

    def __call__(self, op, operands, attrs):
        self.calls.append((op, [t.shape for t in operands], list(attrs)))
        # shape rules of the ops this test drives
        a = dict(attrs)
        if op == "reshape":
            shape = [int(x) for x in a["shape"].strip("@[]").split(",")]
        elif op == "transpose":
            perm = [int(x) for x in a["permutation"].strip("@[]").split(",")]
            shape = [operands[0].shape[p] for p in perm]
        elif op == "broadcastTo":
            shape = [int(x) for x in a["output_shape"].strip("[]").split(",") if x]
        elif op in ("reduceSum", "reduceMax"):
            dims = [int(x) for x in a["dims"].strip("[]").split(",") if x]
            shape = [s for i, s in enumerate(operands[0].shape) if i not in dims]
        elif op == "dotGeneral":
            shape = [operands[0].shape[0], operands[1].shape[1]]
        else:
            shape = list(operands[0].shape) if operands else []
        dt = DType.BOOL if op == "compare" else (operands[0].dtype if operands else DType.FLOAT32)
        return [Tensor(None, dt, shape, eager.mi355x(0))]


def fake_tensor(shape, dt=DType.FLOAT32):
    return Tensor(None, dt, shape, eager.mi355x(0))


@pytest.fixture
def fake():
    be = FakeBackend()
    eager.setEagerBackend(be)
    yield be
    eager.clearEagerBackend()


def test_no_backend_raises():
    eager.clearEagerBackend()
    with pytest.raises(eager.NoEagerBackendError, match="no PJRT execution backend"):
        O.add(fake_tensor([2]), fake_tensor([2]))


def test_attr_wire_format(fake):
    x = fake_tensor([2, 3])
    O.reshape(x, [3, 2])
    O.transpose(x, [1, 0])
    O.broadcastTo(fake_tensor([3]), [2, 3], [1])
    O.reduceSum(x, [1])
    O.matmul(x, fake_tensor([3, 4]))
    O.astype(x, DType.BFLOAT16)
    ops = {c[0]: dict(c[2]) for c in fake.calls}
    assert ops["reshape"] == {"shape": "@[3, 2]"}                    # shape.nim:41
    assert ops["transpose"] == {"permutation": "@[1, 0]"}            # shape.nim:73
    assert ops["broadcastTo"] == {"output_shape": "[2,3]", "broadcast_dimensions": "[1]"}
    assert ops["reduceSum"] == {"dims": "[1]"}                       # reduce.nim:112-113
    assert ops["dotGeneral"] == {"lhs_batching": "[]", "rhs_batching": "[]",
                                 "lhs_contracting": "[1]", "rhs_contracting": "[0]"}
    assert ops["astype"] == {"dtype": "bfloat16"}                    # unary.nim:125


def test_validation_before_dispatch(fake):
    with pytest.raises(TensorError, match="shape mismatch"):
        O.add(fake_tensor([2]), fake_tensor([3]))
    with pytest.raises(TensorError, match="dtype mismatch"):
        O.mul(fake_tensor([2]), fake_tensor([2], DType.BFLOAT16))
    with pytest.raises(TensorError, match="v1 supports only float32"):
        O.reduceSum(fake_tensor([2], DType.BFLOAT16), [0])
    with pytest.raises(TensorError, match="inner dim mismatch"):
        O.matmul(fake_tensor([2, 3]), fake_tensor([4, 5]))
    with pytest.raises(TensorError, match="element count mismatch"):
        O.reshape(fake_tensor([2, 3]), [5])
    assert fake.calls == []


def test_softmax_op_sequence(fake):
    nn.softmax(fake_tensor([4, 8]), 1)
    assert [c[0] for c in fake.calls] == [
        "reduceMax", "broadcastTo", "sub", "exp", "reduceSum", "broadcastTo", "divide"]


def test_causal_mask_orientation_ops(fake):
    """makeCausalMask (attention.nim:18-34): iota rows/cols, compare LE,
    select(upper, 0, -1e9) -- rows <= cols keep their score."""
    eager.setEagerBackend(fake)
    try:
        nn.makeCausalMask([4, 4])
    except Exception:
        pass  # scalarF32 needs a device; the op stream up to it is what we check
    names = [c[0] for c in fake.calls]
    assert names[:3] == ["iota", "iota", "compare"]
    assert dict(fake.calls[2][2]) == {"comparison_direction": "LE"}
    assert dict(fake.calls[0][2])["dtype"] == "dtInt32"
