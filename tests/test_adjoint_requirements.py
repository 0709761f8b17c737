"""required_gradients (reference ictc_o3/autograd/adjoint_requirements.py:12-26) on CPU:
which adjoints a custom Function's backward is asked for under autograd.grad / backward()."""
import torch

from ictc_o3.autograd.adjoint_requirements import required_gradients
from ictc_o3.backends.hip.species import validate_species


class _Probe(torch.autograd.Function):
    seen = []

    @staticmethod
    def forward(ctx, a, b):
        ctx.save_for_backward(a, b)
        return a * b

    @staticmethod
    def backward(ctx, g):
        a, b = ctx.saved_tensors
        _Probe.seen.append(required_gradients((a, b), ctx.needs_input_grad))
        return g * b, g * a


def _run(target, nonleaf=False):
    _Probe.seen.clear()
    a = torch.randn(3, requires_grad=True)
    b = torch.randn(3, requires_grad=True)
    left = a * 1 if nonleaf else a
    y = _Probe.apply(left, b).sum()
    if target == "backward":
        y.backward()
    else:
        torch.autograd.grad(y, [a] if target == "a" else [a, b])
    return _Probe.seen[-1]


def test_untargeted_leaf_adjoint_is_skipped():
    assert _run("a") == (True, False)
    assert _run("a", nonleaf=True) == (True, False)


def test_targeted_and_backward_keep_every_adjoint():
    assert _run("both") == (True, True)
    assert _run("backward") == (True, True)


def test_functorch_transform_keeps_declared():
    seen = []

    class Probe(torch.autograd.Function):
        @staticmethod
        def forward(a, b):
            return a * b

        @staticmethod
        def setup_context(ctx, inputs, output):
            ctx.save_for_backward(*inputs)

        @staticmethod
        def backward(ctx, g):
            a, b = ctx.saved_tensors
            seen.append(required_gradients((a, b), (True, True)))
            return g * b, g * a

    torch.func.grad(lambda a, b: Probe.apply(a, b).sum())(torch.randn(3), torch.randn(3))
    assert seen == [(True, True)]


def test_species_validation_is_tied_to_the_tensor():
    good = torch.tensor([0, 2, 1])
    validate_species(good, 3)
    assert good._ictc_hip_valid_species == (3, good._version)
    bad = torch.tensor([0, 3, 1])
    try:
        validate_species(bad, 3)
    except ValueError:
        pass
    else:
        raise AssertionError("out-of-range species accepted")
    good[1] = 5                                      # in-place change bumps the version: re-checked
    try:
        validate_species(good, 3)
    except ValueError:
        pass
    else:
        raise AssertionError("in-place out-of-range species accepted")
