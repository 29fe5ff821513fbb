"""ctypes binding of libnsa_hip.so (the C-ABI declared in include/nsa_hip.h).

torch is imported first so that its HIP runtime (soname libamdhip64.so.7) is
the one the library binds to: streams and device pointers handed over from
torch are then valid inside the library.  There is no fallback: a missing or
unloadable library raises.
"""

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
# NSA_LIB_PATH: another build of the same library (e.g. for A/B timing)
LIB_PATH = os.environ.get("NSA_LIB_PATH") or os.path.join(_HERE, "libnsa_hip.so")

NSA_OK = 0
NSA_ERR_SHAPE = -1
NSA_ERR_DTYPE = -2
NSA_ERR_ARG = -3
NSA_ERR_LAUNCH = -4
NSA_ERR_WORKSPACE = -5

NSA_F32 = 0
NSA_BF16 = 1
NSA_F16S = 2
MODE_WINDOW = 0
MODE_COMPRESS = 1

_P = ctypes.c_void_p
_I = ctypes.c_int
_L = ctypes.c_int64
_Z = ctypes.c_size_t

# name -> (restype, argtypes); mirrors include/nsa_hip.h
SIGNATURES = {
    "nsa_version": (_I, []),
    "nsa_padded_len": (_I, [_I]),
    "nsa_transpose_kv": (_I, [_P, _P, _I, _I, _I, _I, _I, _P]),
    "nsa_pool_fwd": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_wpool_fwd": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_wpool_bwd": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_wpool_dw": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_heads_split": (_I, [_P, _P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P]),
    "nsa_heads_merge_grad": (_I, [_P, _P, _P, _P, _P, _I, _P, _P, _I, _I, _I, _I, _P]),
    "nsa_pool_bwd": (_I, [_P, _I, _P, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_gate_fwd": (_I, [_P, _P, _P, _P, _P, _L, _I, _I, _P]),
    "nsa_bwd_prep": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _L, _I, _I, _I, _I, _I, _P]),
    "nsa_cast_f32": (_I, [_P, _P, _L, _I, _P]),
    "nsa_pack_heads": (_I, [_P, _P, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_sel_fwd": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_sel_dq": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                        _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_csr_workspace": (_Z, [_I, _I, _I, _I, _I]),
    "nsa_csr_build": (_I, [_P, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_sel_dkdv_workspace": (_Z, [_I, _I, _I, _I, _I, _I]),
    "nsa_sel_dkdv_partial_bytes": (_Z, [_I, _I, _I, _I, _I, _I, _I]),
    "nsa_sel_dkdv": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P, _Z, _P, _P, _Z,
                          _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_sel_dkdv_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _P, _P, _P, _P, _P,
                                  _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_sel_partial_slots": (_I, [_I, _I]),
    "nsa_sel_fwd_bo_workspace": (_Z, [_I, _I, _I, _I, _I, _I]),
    "nsa_sel_fwd_bo": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _Z, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_sel_merge": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_sel_dq_reduce": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_range_fwd": (_I, [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _I, _I, _P]),
    "nsa_range_fwd_finish": (_I, [_I, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I, _I,
                                  _P, _P, _P, _I, _I, _P, _P, _P, _P, _P, _I, _I, _I, _P]),
    "nsa_range_dq": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _I,
                          _I, _I, _I, _I, _I, _I, _I, _I, _I, _P, _P, _I, _I, _P, _I, _I, _P]),
    "nsa_range_dq_cw": (_I, [_P, _P, _P, _P, _P, _P, _P, _P, _I, _I, _I, _P, _P, _P, _P, _P, _P, _I,
                             _I, _I, _I, _I, _I, _P, _P, _I, _I, _P, _I, _I, _P]),
    "nsa_range_dkdv_partial_bytes": (_Z, [_I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_range_dkdv": (_I, [_I, _P, _P, _P, _P, _P, _P, _P, _P, _P, _Z,
                            _I, _I, _I, _I, _I, _I, _I, _I, _I, _I, _P]),
    "nsa_fused_ctx_bytes": (_Z, [_I] * 12),
    "nsa_fused_scratch_bytes": (_Z, [_I] * 12 + [_P]),
    "nsa_fused_fwd": (_I, [_P] * 8 + [_P, _I, _P, _P, _Z, _P, _Z] + [_I] * 14 + [_P]),
    "nsa_fused_bwd": (_I, [_P] * 11 + [_Z, _P, _Z] + [_P] * 8 + [_I] * 12 + [_P]),
    "nsa_importance_topn": (_I, [_P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I, _I, _I,
                                 _I, _I, _I, _I, _I, _P]),
    "nsa_phi_fwd": (_I, [_P] * 7 + [_I] * 7 + [_P]),
    "nsa_phi_dpre": (_I, [_P] * 4 + [_I] * 5 + [_P]),
    "nsa_phi_fold": (_I, [_P, _I, _P] + [_I] * 6 + [_P]),
    "nsa_phi_wgrad_workspace": (_Z, [_I] * 5),
    "nsa_phi_wgrad": (_I, [_P] * 12 + [_Z] + [_I] * 7 + [_P]),
    "nsa_decode_workspace": (_Z, [_I] * 11),
    "nsa_decode_fwd": (_I, [_P] * 15 + [_Z] + [_I] * 14 + [_P]),
    "nsa_decode_append": (_I, [_P] * 16 + [_I] * 8 + [_P]),
}

_lib = None


def load():
    """Load (once) and return the bound library; raises if it is missing."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is not built: run `make -C openbox-llm_amd` or "
            "`python -c 'import __graft_entry__ as g; g.build()'` first")
    lib = ctypes.CDLL(LIB_PATH, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc, what):
    """Map a C status code onto the reference's exception types."""
    if rc == NSA_OK:
        return
    if rc in (NSA_ERR_SHAPE, NSA_ERR_DTYPE):
        raise AssertionError(f"{what}: unsupported shape or dtype (code {rc})")
    raise RuntimeError(f"{what}: HIP library error code {rc}")


def dtype_code(t):
    if t.dtype == torch.float32:
        return NSA_F32
    if t.dtype == torch.bfloat16:
        return NSA_BF16
    if t.dtype == torch.float16:
        # only as branch outputs in the NSA_F16S form: the rows' halves, then a
        # float32 scale per row (of D elements) in the same storage
        rows = t.numel() // t.shape[-1]
        room = t.untyped_storage().nbytes() - t.storage_offset() * 2
        assert t.is_contiguous() and room >= rows * (2 * t.shape[-1] + 4), \
            "float16 tensors are accepted only as NSA_F16S branch outputs (rows followed by their scales)"
        return NSA_F16S
    raise AssertionError(f"dtype {t.dtype} is not supported (float32 or bfloat16)")


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)
