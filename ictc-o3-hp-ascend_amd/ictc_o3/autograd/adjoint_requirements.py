"""Prune adjoints the autograd engine will not execute.

Same contract as the reference's ``required_gradients``
(``ictc_o3/autograd/adjoint_requirements.py:12-26``): ``ctx.needs_input_grad``
reflects requires_grad at graph construction, but a ``torch.autograd.grad`` call
that targets only some leaves (e.g. positions for forces) will not run the
gradient nodes of the others.  When the engine can be queried, only adjoints
whose gradient edge will execute are requested; otherwise (tracing, functorch
transforms, proxy modes, or an engine that refuses the query) every declared
gradient is kept.

The gradient edge of a non-leaf is its ``grad_fn``; that of a leaf is its
``AccumulateGrad`` node.  Under ``autograd.grad`` the engine answers False for a
leaf that is not a target and raises for one that is (kept); under
``backward()`` it answers True for every leaf.
"""
import torch
from torch.fx.experimental.proxy_tensor import get_proxy_mode


_QUERY = getattr(torch._C, "_will_engine_execute_node", None)


def required_gradients(inputs, declared):
    query = _QUERY
    if (query is None or torch.compiler.is_compiling() or get_proxy_mode() is not None
            or torch._C._are_functorch_transforms_active()):
        return tuple(bool(d) for d in declared)
    result = []
    for tensor, needed in zip(inputs, declared):
        if not needed or tensor is None:
            result.append(False)
            continue
        try:
            node = tensor.grad_fn if tensor.grad_fn is not None else \
                torch.autograd.graph.get_gradient_edge(tensor).node
            result.append(bool(query(node)))
        except (RuntimeError, AttributeError, AssertionError):
            result.append(True)
    return tuple(result)
