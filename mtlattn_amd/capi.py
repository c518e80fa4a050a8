"""ctypes binding of the C ABI in include/mtlattn_capi.h (libmtlattn_hip.so).

This is the torch-free way to reach the kernels: every function takes device
pointers (ints), sizes and a hipStream_t handle, exactly as the header
declares them. The torch extension `_C` binds the same library from C++; this
module is what a non-torch host (or a test that wants the raw boundary) uses.

`problem_for(...)` fills the argument block from torch tensors for callers
that have them; nothing else here touches torch.
"""

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmtlattn_hip.so")

DTYPE_F32, DTYPE_F16, DTYPE_BF16 = 0, 1, 2
OK, ERR_INVALID, ERR_UNSUPPORTED, ERR_WORKSPACE, ERR_LAUNCH = 0, -1, -2, -3, -4
ABI_VERSION = 2


class Problem(ctypes.Structure):
    """struct mtlattn_problem (field order and widths as in the header)."""
    _fields_ = [
        ("dtype", ctypes.c_int32), ("num_seqs", ctypes.c_int32),
        ("total_q", ctypes.c_int64), ("total_kv", ctypes.c_int64),
        ("num_heads_q", ctypes.c_int32), ("num_heads_kv", ctypes.c_int32),
        ("head_dim", ctypes.c_int32), ("max_seqlen_q", ctypes.c_int32),
        ("scale", ctypes.c_float), ("causal", ctypes.c_int32), ("window", ctypes.c_int32),
        ("cu_seqlens_q", ctypes.c_void_p), ("cu_seqlens_kv", ctypes.c_void_p),
        ("bias", ctypes.c_void_p), ("bias_q_stride", ctypes.c_int64),
        ("bias_h_stride", ctypes.c_int64), ("bias_kv_cols", ctypes.c_int64),
        ("bias_seq_local", ctypes.c_int32), ("bias_seq_stride", ctypes.c_int64),
        ("bias_seq_rows", ctypes.c_int64),
    ]


class MtlattnError(RuntimeError):
    def __init__(self, fn, rc, msg):
        super().__init__(f"{fn} failed ({rc}): {msg}")
        self.rc = rc


_P = ctypes.POINTER(Problem)
_vp, _i64, _i32, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t

# name -> (restype, argtypes); checked against the header by the CPU tests
SIGNATURES = {
    "mtlattn_abi_version": (ctypes.c_int, []),
    "mtlattn_last_error": (ctypes.c_char_p, []),
    "mtlattn_gpu_core_count": (ctypes.c_int, [ctypes.c_int]),
    "mtlattn_varlen_fwd_workspace_size": (_sz, [_P]),
    "mtlattn_varlen_fwd": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _sz, _vp]),
    "mtlattn_varlen_fwd_noalloc": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp]),
    "mtlattn_varlen_bwd_workspace_size": (_sz, [_P]),
    "mtlattn_varlen_bwd": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp,
                                          _vp, _vp, _vp, _vp, _sz, _vp]),
    "mtlattn_bwd_preprocess": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _vp]),
    "mtlattn_bwd_dq": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _i32, _vp]),
    "mtlattn_bwd_dkv": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _vp, _vp, _i32,
                                       _vp]),
    "mtlattn_attn_splitkv_workspace_size": (_sz, [_P, _i32]),
    "mtlattn_attn_splitkv": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _i64, _vp, _vp, _i32, _vp, _sz, _vp]),
    "mtlattn_decode_num_splits": (_i32, [_P]),
    "mtlattn_paged_decode_workspace_size": (_sz, [_P, _i64]),
    "mtlattn_paged_decode": (ctypes.c_int, [_P, _vp, _i64, _vp, _i64, _vp, _i64, _i32, _i64, _vp, _i64, _i64, _vp,
                                            _vp, _vp, _sz, _vp]),
    "mtlattn_pack_padded": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32, _vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "mtlattn_unpack_padded": (ctypes.c_int, [_i32, _i32, _i32, _i32, _i32, _vp, _vp, _vp, _vp, _i64, _i64, _i64,
                                             _vp]),
}

_lib = None


def lib():
    """Loads libmtlattn_hip.so once and declares every signature. Raises if
    the library is not built: there is no other implementation to fall back to."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"mtlattn: {LIB_PATH} is not built (run __graft_entry__.build())")
        L = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        if L.mtlattn_abi_version() != ABI_VERSION:
            raise ImportError(f"mtlattn: library ABI {L.mtlattn_abi_version()} != binding ABI {ABI_VERSION}")
        _lib = L
    return _lib


def call(name, *args):
    """Calls an entry point returning a status; raises MtlattnError with the
    library's message on failure."""
    L = lib()
    rc = getattr(L, name)(*args)
    if rc != OK:
        raise MtlattnError(name, rc, L.mtlattn_last_error().decode())
    return rc


def problem_for(q, k, cu_q, cu_kv, max_seqlen_q, scale, causal=False, window=0, bias=None):
    """Argument block for torch tensors q [total_q,Hq,D], k [total_kv,Hkv,D]
    and device int32 cu_seqlens; `bias` is an fp32 [total_q, H|1, cols]
    tensor with a contiguous last dim, or None."""
    import torch
    dt = {torch.float32: DTYPE_F32, torch.float16: DTYPE_F16, torch.bfloat16: DTYPE_BF16}[q.dtype]
    p = Problem(dtype=dt, num_seqs=cu_q.numel() - 1, total_q=q.shape[0], total_kv=k.shape[0],
                num_heads_q=q.shape[1], num_heads_kv=k.shape[1], head_dim=q.shape[2],
                max_seqlen_q=int(max_seqlen_q), scale=float(scale), causal=int(bool(causal)),
                window=int(window), cu_seqlens_q=cu_q.data_ptr(), cu_seqlens_kv=cu_kv.data_ptr(),
                bias=None, bias_q_stride=0, bias_h_stride=0, bias_kv_cols=0)
    if bias is not None:
        p.bias = bias.data_ptr()
        p.bias_q_stride = bias.stride(0)
        p.bias_h_stride = 0 if bias.shape[1] == 1 else bias.stride(1)
        p.bias_kv_cols = bias.shape[2]
    return p
