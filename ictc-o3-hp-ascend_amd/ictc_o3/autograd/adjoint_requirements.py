"""Prune adjoints the autograd engine will not execute.

Same contract as the reference's ``required_gradients``
(``ictc_o3/autograd/adjoint_requirements.py:12-26``): ``ctx.needs_input_grad``
reflects requires_grad at graph construction, but a ``torch.autograd.grad`` call
that targets only some leaves (e.g. positions for forces) will not run the
gradient nodes of the others.  When the engine can be queried, only adjoints
whose gradient edge will execute are requested; otherwise every declared
gradient is kept.
"""
import torch


_QUERY = getattr(torch._C, "_will_engine_execute_node", None)


def required_gradients(inputs, declared):
    query = _QUERY
    if query is None or torch.compiler.is_compiling():
        return tuple(bool(d) for d in declared)
    result = []
    for tensor, needed in zip(inputs, declared):
        if not needed or tensor is None:
            result.append(False)
            continue
        if tensor.grad_fn is None:
            # a leaf: backward() accumulates into every leaf, and the engine cannot be queried about
            # leaves under autograd.grad() (it raises, which costs far more than the answer)
            result.append(True)
            continue
        try:
            result.append(bool(query(tensor.grad_fn)))       # a non-leaf's gradient edge is its grad_fn
        except (RuntimeError, AttributeError, AssertionError):
            result.append(True)
    return tuple(result)
