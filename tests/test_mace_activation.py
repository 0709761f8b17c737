"""mace_hip.activation.silu: derivatives of every order match torch's silu (float64 on the CPU,
gradcheck / gradgradcheck through the composed formula), and on the GPU the one-pass double
backward (ictc_hip_silu_second, used when no further graph is recorded) matches torch's own
silu double backward on fp32 activations."""
import ctypes

import pytest
import torch
import torch.nn.functional as F

from mace_hip.activation import silu


def test_matches_torch_silu_to_second_order_cpu():
    g = torch.Generator().manual_seed(0)
    x = (4 * torch.randn(300, generator=g, dtype=torch.float64)).requires_grad_()
    assert torch.allclose(silu(x), F.silu(x), atol=1e-15)
    assert torch.autograd.gradcheck(silu, (x,))
    assert torch.autograd.gradgradcheck(silu, (x,))
    go = torch.randn(300, generator=g, dtype=torch.float64)
    h = torch.randn(300, generator=g, dtype=torch.float64)
    ours = torch.autograd.grad((torch.autograd.grad(silu(x), x, go, create_graph=True)[0] * h).sum(), x)[0]
    ref = torch.autograd.grad((torch.autograd.grad(F.silu(x), x, go, create_graph=True)[0] * h).sum(), x)[0]
    assert torch.allclose(ours, ref, atol=1e-12)


@pytest.mark.gpu
def test_fused_double_backward_matches_torch_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    dev = torch.device("cuda", 0)
    g = torch.Generator().manual_seed(1)
    n = 105634 * 64 + 7                               # a radial-MLP activation, not a multiple of 4
    x0 = 3 * torch.randn(n, generator=g)
    x0[:8] = torch.tensor([-120.0, -88.0, -30.0, -1e-7, 0.0, 1e-7, 30.0, 120.0])   # exp over/underflow
    x0 = x0.to(dev)
    go0 = torch.randn(n, generator=g).to(dev)
    h0 = torch.randn(n, generator=g).to(dev)

    def second(fn):
        x = x0.clone().requires_grad_()
        go = go0.clone().requires_grad_()
        first, = torch.autograd.grad(fn(x), x, go, create_graph=True)
        return torch.autograd.grad((first * h0).sum(), (x, go))   # last backward: fused path for silu

    for ours, ref, name in zip(second(silu), second(F.silu), ("x", "grad_output")):
        assert torch.isfinite(ours).all(), f"non-finite silu double backward wrt {name}"
        err = (ours - ref).abs().max() / ref.abs().max()
        assert err < 1e-6, f"silu double backward wrt {name}: relative error {err:.2e}"
    from ictc_o3 import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation or launches nothing
    assert lib.ictc_hip_silu_second(fake, fake, fake, fake, fake, -1, None) == 1
    assert lib.ictc_hip_silu_second(None, fake, fake, fake, fake, 8, None) == 1
    assert lib.ictc_hip_silu_second(fake, None, fake, None, fake, 8, None) == 1   # grad_x needs grad
    assert lib.ictc_hip_silu_second(fake, None, fake, None, None, 8, None) == 0   # nothing requested
