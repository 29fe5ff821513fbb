"""The host wrappers that hand a selection partial buffer to a kernel check
its element type and size before the launch: the library takes the buffer
as a plain pointer and reads it with the element type of the dtype code it is
given, so a buffer of another type or size would be read past its end.
(Regression: ``sel_dq_reduce`` asked for a float32 result on bf16 partials
passed NSA_F32 for the bf16 buffer, and the reduce read twice its bytes.)
These run on the CPU: every case raises before anything is launched."""

import pytest
import torch

import nsa_hip_ops as ops

B, Hq, Hkv, T, D, BS, S = 1, 4, 1, 256, 64, 64, 2
G = Hq // Hkv


def _slots():
    return int(ops._lib().nsa_sel_partial_slots(S, BS))


def _idx():
    return torch.zeros(B, Hkv, T, S, dtype=torch.int32)


def _part(dtype, extra=0):
    return torch.zeros(B * Hkv * T * _slots() * G * D + extra, dtype=dtype).view(-1)


def test_sel_dq_reduce_rejects_other_partial_types_and_sizes():
    with pytest.raises(TypeError):
        ops.sel_dq_reduce(_idx(), _part(torch.float16).view(B, Hkv, T, _slots(), G, D), None, BS, torch.float32)
    bad = torch.zeros(B, Hkv, T, _slots() - 1, G, D, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        ops.sel_dq_reduce(_idx(), bad, None, BS, torch.bfloat16)
    ok = _part(torch.bfloat16).view(B, Hkv, T, _slots(), G, D)
    with pytest.raises(TypeError):   # the accumulator is float32 [B, Hq, T, D]
        ops.sel_dq_reduce(_idx(), ok, torch.zeros(B, Hq, T, D, dtype=torch.bfloat16), BS, torch.bfloat16)


def test_dq_finishers_take_partials_of_the_input_dtype():
    q = torch.zeros(B, Hq, T, D, dtype=torch.bfloat16)
    kc = torch.zeros(B, Hkv, 15, D, dtype=torch.bfloat16)
    geom = ops.NSAGeometry(32, 16, BS, S, 128, False, 0)
    for wrong in (torch.float32, torch.float16):
        with pytest.raises(TypeError):
            ops.range_dq_cw(q, q, kc, kc, kc, None, None, None, q, q, q, None, None, None, geom,
                            _part(wrong), _idx())
        with pytest.raises(TypeError):
            ops.range_dq(ops.MODE_COMPRESS, q, kc, kc, kc, q, None, None, None, None, False, 0, 32, 16,
                         sel_part=_part(wrong), sel_idx=_idx(), sel_block=BS)
    with pytest.raises(ValueError):   # one slot's rows short
        ops.range_dq_cw(q, q, kc, kc, kc, None, None, None, q, q, q, None, None, None, geom,
                        _part(torch.bfloat16, extra=-G * D), _idx())


def test_forward_merges_take_partials_of_the_partial_dtype():
    q = torch.zeros(B, Hq, T, D, dtype=torch.bfloat16)
    ml = torch.zeros(B, Hkv, T, _slots(), G, 2, dtype=torch.float32)
    bf = _part(torch.bfloat16).view(B, Hkv, T, _slots(), G, D)
    with pytest.raises(TypeError):   # bf16 inputs keep fp16 partials
        ops.sel_merge(_idx(), (bf, ml), q.shape, Hkv, BS)
    f16 = _part(torch.float16).view(B, Hkv, T, _slots(), G, D)
    with pytest.raises(ValueError):
        ops.sel_merge(_idx(), (f16, ml[..., :1].contiguous()), q.shape, Hkv, BS)
    gate = torch.zeros(B, Hq, T, 3, dtype=torch.bfloat16)
    kv = torch.zeros(B, Hkv, T, D, dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        ops.range_fwd_finish(q, kv, kv, 128, (bf, ml), _idx(), BS, q, gate, vt=kv)
