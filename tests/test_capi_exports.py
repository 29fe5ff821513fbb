"""CPU checks of the C-ABI boundary (no compute calls, no GPU needed).

* libnsa_hip.so loads and exports every function declared in include/nsa_hip.h;
* the ctypes signature table covers exactly those declarations;
* size queries that touch no device memory return sane values.
"""

import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "nsa_hip.h")


def _declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"^\s*(?:int|size_t)\s+(nsa_\w+)\s*\(", text, flags=re.M)))


def _lib():
    import _nsa_lib
    if not os.path.exists(_nsa_lib.LIB_PATH):
        pytest.skip("libnsa_hip.so not built")
    return _nsa_lib, _nsa_lib.load()


def test_header_declares_the_entry_points():
    names = _declared()
    for must in ("nsa_sel_fwd", "nsa_sel_dq", "nsa_sel_dkdv", "nsa_range_fwd", "nsa_range_dq",
                 "nsa_range_dkdv", "nsa_pool_fwd", "nsa_pool_bwd", "nsa_importance_topn", "nsa_csr_build",
                 "nsa_gate_fwd", "nsa_bwd_prep"):
        assert must in names


def test_library_exports_every_declared_symbol():
    mod, lib = _lib()
    for name in _declared():
        assert hasattr(lib, name), f"{name} not exported"
    assert sorted(mod.SIGNATURES) == _declared()


def _declared_arity():
    """Parameter count of every declaration in the header."""
    text = re.sub(r"/\*.*?\*/", "", open(HEADER).read(), flags=re.S)
    out = {}
    for m in re.finditer(r"^\s*(?:int|size_t)\s+(nsa_\w+)\s*\(([^)]*)\)", text, flags=re.M):
        params = m.group(2).strip()
        out[m.group(1)] = 0 if params in ("", "void") else params.count(",") + 1
    return out


def test_ctypes_signatures_match_the_header_arity():
    """A wrong argument count in the ctypes table would only surface as a
    TypeError on the first call on a GPU box."""
    import _nsa_lib
    arity = _declared_arity()
    for name, (_, args) in _nsa_lib.SIGNATURES.items():
        assert len(args) == arity[name], f"{name}: ctypes has {len(args)} arguments, the header {arity[name]}"


def test_size_queries():
    _, lib = _lib()
    assert lib.nsa_version() >= 100
    assert lib.nsa_padded_len(32768) >= 32768 + 32
    assert lib.nsa_padded_len(1) % 64 == 0
    assert lib.nsa_sel_dkdv_workspace(1, 4, 32768, 16, 64, 256) > 0
    assert lib.nsa_csr_workspace(1, 4, 32768, 16, 512) > 4 * 32768 * 16 * 4
    # the deterministic selection dK/dV: one 64-key float row pair per work item
    cap_items = 4 * 512 + (4 * 32768 * 16 + 1023) // 1024 + 1
    assert lib.nsa_sel_dkdv_partial_bytes(1, 4, 32768, 16, 128, 64, 1024) == cap_items * 64 * 128 * 2 * 4
    # the window dK/dV has one writer per key: no partial buffer (answered
    # before any device query)
    assert lib.nsa_range_dkdv_partial_bytes(0, 1, 4, 32768, 32768, 128, 1, 1, None) == 0
    assert lib.nsa_range_dkdv_partial_bytes(1, 1, 4, 0, 2047, 128, 32, 16, None) == 0
    # phi's parameter gradients: float partials of dW1, dW2 and the biases per
    # token range; unsupported shapes answer 0
    one = 4 * (128 * 32 * 128 + 128 * 128 + 128 + 128)
    ws = lib.nsa_phi_wgrad_workspace(4, 2047, 128, 128, 32)
    assert ws >= one and ws % one == 0
    assert lib.nsa_phi_wgrad_workspace(4, 2047, 96, 128, 32) == 0
    assert lib.nsa_phi_wgrad_workspace(4, 0, 128, 128, 32) == 0


def test_bad_shapes_are_rejected_without_launching():
    _, lib = _lib()
    # D = 48 is not a supported head dim; block 8 is below 16: both fail the checks
    assert lib.nsa_sel_fwd(None, None, None, None, None, None, 1, 4, 1, 64, 48, 2, 16, 1, None) == -1
    assert lib.nsa_sel_fwd(None, None, None, None, None, None, 1, 4, 1, 64, 64, 2, 8, 1, None) == -1
    assert lib.nsa_range_fwd(7, None, None, None, None, None, 1, 4, 1, 64, 64, 64, 16, 16, 16, None, 1, 1, None) == -3
    # branch outputs are the input type, float32, or NSA_F16S with bf16 inputs
    assert lib.nsa_range_fwd(0, None, None, None, None, None, 1, 4, 1, 64, 64, 64, 16, 16, 16, None, 0, 1, None) == -2
    assert lib.nsa_range_fwd(0, None, None, None, None, None, 1, 4, 1, 64, 64, 64, 16, 16, 16, None, 0, 2, None) == -2
    assert lib.nsa_bwd_prep(*([None] * 12), None, 1, 64, 256, 64, 3, 0, 2, 0, None) == -2
    # the selection chunk is capped at 1024 queries (staged in LDS)
    assert lib.nsa_sel_dkdv(*([None] * 8), 1, *([None] * 5), 0, None, None, 1 << 30, 1, 4, 1, 64, 64, 2, 16, 2048,
                            1, None) == -1
    assert lib.nsa_pool_fwd(None, None, 1, 1, 64, 64, 16, 16, 5, None) == -2


def test_noalloc_entry_point_rejects_oversize_without_a_device():
    mod, lib = _lib()
    # the work items of this call exceed NSA_SEL_NOALLOC_SCRATCH_BYTES: the size
    # check runs before any device call, so it answers here without a GPU
    need = lib.nsa_sel_dkdv_workspace(1, 1, 65536, 16, 64, 2)
    assert need > (1 << 20)
    rc = lib.nsa_sel_dkdv_noalloc(*([None] * 8), 1, *([None] * 5), 1, 16, 1, 65536, 64, 16, 64, 2, 1, None)
    assert rc == mod.NSA_ERR_WORKSPACE
    # bad arguments are shape errors, also before any device call
    assert lib.nsa_sel_dkdv_noalloc(*([None] * 8), 1, *([None] * 5), 0, 16, 1, 64, 64, 16, 64, 2, 1, None) == -1


def test_decode_entry_points_check_before_launching():
    mod, lib = _lib()
    # c3 heads, 32K capacity: partials + scores fit in a few tens of MB
    n = lib.nsa_decode_workspace(16, 64, 4, 128, 32768, 2047, 32, 16, 64, 16, 512)
    assert 0 < n < 64 << 20
    # unsupported: head dim 48, a pooled cache too short for the capacity,
    # more than 4096 candidate blocks
    assert lib.nsa_decode_workspace(1, 16, 1, 48, 4096, 255, 32, 16, 64, 16, 512) == 0
    assert lib.nsa_decode_workspace(1, 16, 1, 128, 4096, 100, 32, 16, 64, 16, 512) == 0
    assert lib.nsa_decode_workspace(1, 16, 1, 128, 64 * 4096 + 1, 1 << 16, 32, 16, 64, 16, 512) == 0
    fake = 1 << 20   # a non-null, 256-byte aligned address that is never dereferenced
    args = [fake] * 9 + [fake, fake, None, None, None]
    # workspace smaller than required: rejected before any launch
    assert lib.nsa_decode_fwd(*args, fake, 16, 1, 16, 1, 128, 4096, 255, 32, 16, 64, 16, 512, 0, 0, 1,
                              None) == mod.NSA_ERR_WORKSPACE
    assert lib.nsa_decode_fwd(*args, fake, 1 << 30, 1, 16, 1, 128, 4096, 255, 32, 16, 64, 16, 512, 0, 0, 7,
                              None) == mod.NSA_ERR_DTYPE
    # lens_in and lens_out must differ (the update of one sequence's length
    # would race with the other KV heads' reads)
    assert lib.nsa_decode_append(*([fake] * 14), fake, fake, 1, 1, 64, 128, 7, 32, 16, 1, None) == mod.NSA_ERR_ARG


def test_f16s_buffers_carry_their_row_scales():
    """NSA_F16S branch outputs: the float16 view of the rows must have the
    float32 row scales after it in the same storage; a plain float16 tensor
    is refused before any call."""
    import torch
    mod, _ = _lib()
    import nsa_hip_ops as ops
    o = ops.f16s_empty((2, 3, 5, 64), "cpu")
    assert o.shape == (2, 3, 5, 64) and o.dtype == torch.float16
    assert o.untyped_storage().nbytes() == 2 * 3 * 5 * (64 * 2 + 4)
    assert mod.dtype_code(o) == mod.NSA_F16S
    assert ops.kept_output((2, 3, 5, 64), torch.empty(0, dtype=torch.float32)).dtype == torch.float32
    with pytest.raises(AssertionError):
        mod.dtype_code(torch.empty(2, 3, 5, 64, dtype=torch.float16))
