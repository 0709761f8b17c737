"""CPU oracle for the ictc_o3 equivariant hot path -- TEST INFRASTRUCTURE ONLY.

This package restates, in plain PyTorch on the CPU (float64 for pinning,
float32 for the CPU baseline), the reference's own CPU ("reference backend")
algorithms for the operators the HIP library implements:

* ``ictc_basis``            -- frozen ICTC harmonic basis, Clebsch-Gordan (CG)
                               construction and normalisation, direction
                               harmonics (``ictc_o3/basis/ictd_irreps.py``);
* ``tensor_product``        -- path-preserving channelwise TP
                               (``_forward_index_add``) and the gather -> TP ->
                               ``index_add`` graph message;
* ``symmetric_contraction`` -- correlation-<=3 symmetric contraction
                               (``_forward_selected_elements``) on U tensors
                               built in the ICTC basis;
* ``mace``                  -- the MACE-ICTC energy/force model used by the
                               full-step configuration.

Every function cites the reference file:line it follows.  Derivatives of any
order come from torch autograd through these eager restatements, exactly as
the reference's CPU path obtains them.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s CPU-baseline
leg may import this package, and only as the checker / CPU baseline.  The
product (``ictc-o3-hp-ascend_amd/``) never imports it.
"""
