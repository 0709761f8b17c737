"""C-ABI checks that need no GPU: the library loads, exports every entry point the
public headers declare, and rejects invalid descriptors before any launch."""
import ctypes
import os
import re

import pytest

from conftest import ROOT


def _declared_symbols():
    names = set()
    inc = os.path.join(ROOT, "include")
    for fn in os.listdir(inc):
        if fn.endswith(".h"):
            text = open(os.path.join(inc, fn)).read()
            names.update(re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\**\s*(ictc_hip_[A-Za-z0-9_]+)\s*\(",
                                    text, flags=re.M))
    return names


def test_library_exports_every_declared_symbol():
    from ictc_o3 import _lib
    lib = _lib.lib()
    declared = _declared_symbols()
    assert declared, "no declarations parsed"
    for name in declared:
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"
    assert set(_lib.exported_symbols()) == declared


def test_status_strings_and_slot_counts():
    from ictc_o3 import _lib
    lib = _lib.lib()
    assert lib.ictc_hip_status_string(0) == b"ok"
    assert lib.ictc_hip_status_string(2) == b"unsupported degree combination"
    assert lib.ictc_hip_tp_slot_count(2, 2, 2) == 11
    assert lib.ictc_hip_tp_slot_count(3, 3, 3) == 23
    assert lib.ictc_hip_tp_slot_count(0, 3, 3) == 4
    assert lib.ictc_hip_tp_slot_count(4, 4, 4) == 42      # degree-generic kernels
    assert lib.ictc_hip_tp_slot_count(5, 5, 5) == 69
    assert lib.ictc_hip_tp_slot_count(6, 6, 6) == 106
    assert lib.ictc_hip_tp_slot_count(7, 3, 3) == -1


def _desc(c=64, lmax=2):
    from ictc_o3.backends.hip.tensor_product import TensorProductPlan
    from ictc_o3.basis.ictd_irreps import triangle_paths
    return TensorProductPlan(triangle_paths(lmax, lmax, lmax), c, lmax, lmax).desc


def test_descriptor_validation_rejects_before_launch():
    from ictc_o3 import _lib
    lib = _lib.lib()
    fwd = lib.ictc_hip_tp_forward
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation
    d = _desc()
    assert fwd(None, fake, fake, fake, fake, 4, None) == 1
    bad = _desc()
    bad.channels = 0
    assert fwd(ctypes.byref(bad), fake, fake, fake, fake, 4, None) == 1
    bad = _desc()
    bad.gate_index[3] = bad.gate_index[4]          # duplicate gate block
    assert fwd(ctypes.byref(bad), fake, fake, fake, fake, 4, None) == 1
    bad = _desc()
    bad.out_offset[0] = bad.out_components          # output block past the end
    assert fwd(ctypes.byref(bad), fake, fake, fake, fake, 4, None) == 1
    bad = _desc()
    bad.input_lmax = 4                              # path count no longer matches
    assert fwd(ctypes.byref(bad), fake, fake, fake, fake, 4, None) == 1
    bad = _desc()
    bad.input_lmax = 7                              # above every kernel
    assert fwd(ctypes.byref(bad), fake, fake, fake, fake, 4, None) == 2
    assert fwd(ctypes.byref(d), fake, fake, fake, fake, -1, None) == 1
    assert fwd(ctypes.byref(d), None, fake, fake, fake, 4, None) == 1
    # zero rows: valid, nothing launched
    assert fwd(ctypes.byref(d), None, None, None, None, 0, None) == 0
    bwd = lib.ictc_hip_tp_backward
    # gradients to harmonics need the features operand
    assert bwd(ctypes.byref(d), None, fake, fake, fake, None, fake, None, 4, None) == 1


def test_generic_degree_validation_before_launch():
    """Degree sets above 3 pass descriptor validation; the message tangent entry points, which have
    no degree-generic kernels, report UNSUPPORTED before any launch; bond rows are built in-kernel."""
    from ictc_o3 import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced
    d = _desc(16, 4)
    assert lib.ictc_hip_tp_forward(ctypes.byref(d), None, fake, fake, fake, 4, None) == 1
    assert lib.ictc_hip_message_bond_width(ctypes.byref(d)) == 0
    f = fake
    assert lib.ictc_hip_message_forward_tangent(ctypes.byref(d), f, f, f, f, f, f, f, f, None, f, 1, 1, 1, None) == 2
    assert lib.ictc_hip_message_edge_grad_tangent(ctypes.byref(d), f, f, f, f, f, f, f, f, f, None, f, None, None,
                                                  1, 1, 1, None) == 2


def test_python_guards_reject_cpu_tensors():
    import torch
    from ictc_o3.backends.hip.runtime import require_gpu_fp32
    with pytest.raises(ValueError):
        require_gpu_fp32(torch.zeros(3))
    from ictc_o3 import EdgeTensorProduct
    with pytest.raises(ValueError):
        EdgeTensorProduct.create(channels=8, device="cpu")


def test_radius_graph_validation_rejects_before_launch():
    from ictc_o3 import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation or launches nothing
    grid = _lib.CellGrid()
    for i in range(3):
        grid.cell[4 * i] = 10.0
        grid.bins[i], grid.reach[i], grid.periodic[i] = 2, 1, 1
    grid.cutoff_sq = 9.0
    count = lib.ictc_hip_radius_graph_count
    assert count(None, fake, fake, fake, fake, 4, fake, None) == 1
    assert count(ctypes.byref(grid), None, fake, fake, fake, 4, fake, None) == 1
    assert count(ctypes.byref(grid), fake, fake, fake, fake, -1, fake, None) == 1
    assert count(ctypes.byref(grid), None, None, None, None, 0, None, None) == 0
    bad = _lib.CellGrid.from_buffer_copy(grid)
    bad.bins[1] = 0
    assert count(ctypes.byref(bad), fake, fake, fake, fake, 4, fake, None) == 1
    bad = _lib.CellGrid.from_buffer_copy(grid)
    bad.reach[2] = 65
    assert count(ctypes.byref(bad), fake, fake, fake, fake, 4, fake, None) == 1
    bad = _lib.CellGrid.from_buffer_copy(grid)
    bad.cutoff_sq = 0.0
    assert count(ctypes.byref(bad), fake, fake, fake, fake, 4, fake, None) == 1
    fill = lib.ictc_hip_radius_graph_fill
    assert fill(ctypes.byref(grid), fake, fake, fake, fake, 4, None, fake, fake, None) == 1


def test_message_bond_width_and_tangent_validation():
    """Bond width 0 marks degree sets whose kernels form the bond rows in-kernel (then
    ictc_hip_message_bonds launches nothing); the tangent entry points require every
    primal and tangent operand and reject before any launch."""
    from ictc_o3 import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation or launches nothing
    d2, d3 = _desc(64, 2), _desc(128, 3)
    assert lib.ictc_hip_message_bond_width(ctypes.byref(d2)) == 0       # lmax 2: 2 entries/lane x 9 harmonics
    assert lib.ictc_hip_message_bond_width(ctypes.byref(d3)) == 439     # lmax 3 keeps the bond buffer
    assert lib.ictc_hip_message_bonds(ctypes.byref(d2), fake, None, 8, None) == 0
    fwd_t = lib.ictc_hip_message_forward_tangent
    args = [fake] * 10                                       # x, bonds, g, tx, tb, tg, src, rowptr, perm, out
    for i in (0, 1, 2, 3, 4, 5, 6, 7, 9):                    # perm (index 8) may be null
        bad = list(args)
        bad[i] = None
        assert fwd_t(ctypes.byref(d3), *bad, 4, 4, 8, None) == 1, f"forward_tangent accepted null arg {i}"
    assert fwd_t(ctypes.byref(d3), *args, 4, 4, -1, None) == 1
    edge_t = lib.ictc_hip_message_edge_grad_tangent
    args = [fake] * 13                 # x, y, g, tx, ty, tg, dout, src, rowptr, perm, dyp, dg, dxe
    for i in (0, 1, 2, 3, 4, 5, 6, 7, 8):
        bad = list(args)
        bad[i] = None
        assert edge_t(ctypes.byref(d3), *bad, 4, 4, 8, None) == 1, f"edge_grad_tangent accepted null arg {i}"
    none_out = list(args)
    none_out[10] = none_out[11] = none_out[12] = None         # nothing requested: no launch, ok
    assert edge_t(ctypes.byref(d3), *none_out, 4, 4, 8, None) == 0


def test_message_rejects_node_tensors_beyond_32bit_offsets():
    """Node tensors are gathered through 32-bit buffer offsets: sizes at or beyond 4 GiB are
    refused (ICTC_ERR_UNSUPPORTED) before any launch, for the primal and tangent entry points."""
    from ictc_o3 import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation
    d3 = _desc(128, 3)                       # 16 * 128 floats = 8 KiB per node row
    too_many = (1 << 32) // (16 * 128 * 4)   # exactly 4 GiB of node features
    assert lib.ictc_hip_message_forward(ctypes.byref(d3), fake, fake, fake, fake, fake, None, fake,
                                        too_many, 4, 8, None) == 2
    assert lib.ictc_hip_message_forward(ctypes.byref(d3), fake, fake, fake, fake, fake, None, fake,
                                        4, too_many, 8, None) == 2   # output rows are 99 * 128 floats
    assert lib.ictc_hip_message_forward_tangent(ctypes.byref(d3), *([fake] * 8), None, fake,
                                                too_many, 4, 8, None) == 2
    assert lib.ictc_hip_message_edge_grad(ctypes.byref(d3), fake, fake, fake, fake, fake, fake, None,
                                          fake, fake, fake, too_many, 4, 8, 0, None) == 2


def test_degree_linear_weight_grad_workspace_and_validation():
    """Workspace size of the weight adjoint ([ranges][O][k] floats per degree, the ranges sized so
    that the launch's 128 x 64 tiles fit three blocks per CU of 256 CUs, the device count this
    GPU-less host falls back to) and its argument checks, all before any launch."""
    from ictc_o3 import _lib
    from ictc_o3.backends.hip.degree_linear import DegreeLinearPlan
    lib = _lib.lib()
    plan = DegreeLinearPlan((4, 6, 7, 6), 128, 128)
    n = 2048
    jt = [-(-k * 128 // 64) for k in plan.counts]
    work = sum(n * (2 * l + 1) * j for l, j in enumerate(jt))
    room = 3 * 256 - sum(jt)
    rows = max(256, -(-(-(-work // room)) // 32) * 32)
    assert rows == 576
    ranges = [-(-(n * (2 * l + 1)) // rows) for l in range(4)]
    assert sum(r * j for r, j in zip(ranges, jt)) <= 3 * 256
    want = sum(r * 128 * k * 128 for r, k in zip(ranges, plan.counts))
    assert lib.ictc_hip_degree_linear_weight_grad_workspace(ctypes.byref(plan.desc), 0, n) == want
    assert lib.ictc_hip_degree_linear_weight_grad_workspace(ctypes.byref(plan.desc), 0, 0) == 0
    # the mul_ir layout takes one channel block per degree; an unknown layout is rejected
    assert lib.ictc_hip_degree_linear_weight_grad_workspace(ctypes.byref(plan.desc), 1, n) == -1
    assert lib.ictc_hip_degree_linear_weight_grad_workspace(ctypes.byref(plan.desc), 2, n) == -1
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation
    ptrs = (ctypes.c_void_p * 4)(fake, fake, fake, fake)
    wg = lib.ictc_hip_degree_linear_weight_grad
    assert wg(ctypes.byref(plan.desc), 0, fake, fake, 1.0, fake, want - 1, ptrs, n, None) == 1   # workspace too small
    assert wg(ctypes.byref(plan.desc), 0, None, fake, 1.0, fake, want, ptrs, n, None) == 1       # no grad_y
    assert wg(ctypes.byref(plan.desc), 0, fake, fake, 1.0, fake, want, None, n, None) == 1       # no outputs
    assert wg(ctypes.byref(plan.desc), 0, fake, fake, 1.0, fake, want, ptrs, -1, None) == 1      # negative rows
    # x beyond 2 GiB of 32-bit buffer offsets
    assert wg(ctypes.byref(plan.desc), 0, fake, fake, 1.0, fake, 1 << 40, ptrs, 1 << 20, None) == 2


def test_radial_mlp_workspace_and_validation():
    """Workspace of the radial-MLP weight gradients (one [64 x 16 + 2 x 64 x 64] partial per block,
    blocks of four 16-edge tiles, at most two per CU: 256 CUs on this GPU-less host) and the
    argument checks, all before any launch."""
    from ictc_o3 import _lib
    lib = _lib.lib()
    part = 64 * 16 + 2 * 64 * 64
    assert lib.ictc_hip_radial_mlp_workspace(0) == 0
    assert lib.ictc_hip_radial_mlp_workspace(1) == part
    assert lib.ictc_hip_radial_mlp_workspace(64 * 5) == 5 * part
    assert lib.ictc_hip_radial_mlp_workspace(105_634) == 512 * part
    assert lib.ictc_hip_radial_mlp_workspace(-1) == -1
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation or does nothing
    rm = lib.ictc_hip_radial_mlp

    def call(mode=0, basis=8, edges=100, out=fake, w=fake, gw=(None, None, None), ws=None, wsf=0, g=fake, u=fake,
             gf=None, gg=None):
        return rm(mode, fake, w, fake, fake, 1.0, g, u, out, gf, gg, ws, wsf, *gw, basis, edges, None)

    assert call(mode=3) == 2 and call(mode=-1) == 2                 # unknown mode
    assert call(basis=0) == 2 and call(basis=17) == 2               # basis beyond the kernel's 16
    assert call(edges=-1) == 1 and call(w=None) == 1                # negative rows, missing weight
    assert call(out=None) == 1                                      # VALUE without an output
    assert call(mode=1, out=None) == 0                              # VJP asked for nothing: no launch
    assert call(mode=1, g=None, gf=fake) == 1                       # VJP without the adjoint
    assert call(mode=2, u=None, gg=fake) == 1                       # VJP_VJP without the cotangent
    assert call(mode=1, gw=(fake, None, None), ws=fake, wsf=part - 1, edges=1) == 1   # workspace too small
    assert call(mode=1, gw=(None, fake, None), ws=None, wsf=part, edges=1) == 1       # no workspace


def test_species_linear_validation():
    """ictc_hip_species_linear rejects bad modes, channel counts and missing tensors before any
    launch, and an empty node set does nothing."""
    from ictc_o3 import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation or does nothing
    sl = lib.ictc_hip_species_linear

    def call(mode=0, w=fake, x=fake, s=fake, out=fake, c=128, ns=10, nodes=100):
        return sl(mode, w, x, s, out, c, ns, nodes, None)

    assert call(mode=2) == 1 and call(mode=-1) == 1                 # unknown mode
    assert call(c=0) == 1 and call(c=4097) == 1                     # channels outside 1..4096
    assert call(ns=0) == 1 and call(nodes=-1) == 1                  # no species, negative rows
    assert call(w=None) == 1 and call(x=None) == 1 and call(s=None) == 1 and call(out=None) == 1
    assert call(nodes=0, w=None) == 0                               # nothing to do: no launch


def test_readout_validation():
    """ictc_hip_readout rejects bad modes, sizes and missing tensors before any launch, and a VJP
    asked for nothing or an empty node set does nothing."""
    from ictc_o3 import _lib
    lib = _lib.lib()
    fake = ctypes.c_void_p(16)  # never dereferenced: every call below fails validation or does nothing
    ro = lib.ictc_hip_readout

    def call(mode=0, y=fake, wl=fake, x=fake, w1=fake, w2=fake, g=fake, out=fake, gy=None, gx=None, c=128, h=16,
             nodes=100):
        return ro(mode, y, wl, x, w1, w2, 1.0, g, out, gy, gx, c, h, nodes, None)

    assert call(mode=2) == 1 and call(mode=-1) == 1                 # unknown mode
    assert call(c=0) == 1 and call(c=1025) == 1                     # channels outside 1..1024
    assert call(h=0) == 1 and call(h=257) == 1 and call(nodes=-1) == 1
    assert call(x=None) == 1 and call(w1=None) == 1 and call(w2=None) == 1 and call(wl=None) == 1
    assert call(out=None) == 1                                      # VALUE without an output
    assert call(mode=1, g=None, gx=fake) == 1                       # VJP without the adjoint
    assert call(mode=1, y=None, gy=fake) == 1                       # grad_y without y
    assert call(mode=1) == 0                                        # VJP asked for nothing: no launch
    assert call(nodes=0, x=None) == 0                               # nothing to do
