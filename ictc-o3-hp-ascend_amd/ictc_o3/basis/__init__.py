"""Host-side constants: frozen basis, CG tensors, path plans, owner modules."""
