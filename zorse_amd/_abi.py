"""ctypes binding of libzorse_amd.so (declared in include/zorse_amd.h).

The library is loaded lazily, always after ``import torch`` so that it binds
to the HIP runtime torch has already mapped.  Every entry point returns an
int status; :func:`check` turns a non-zero status into ``RuntimeError``
carrying the library's thread-local message.  A missing library raises --
there is no fallback path.
"""
from __future__ import annotations

import ctypes
import os
import threading

import torch  # noqa: F401  (must precede the library load: shared HIP runtime)

LIB_NAME = "libzorse_amd.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

ZK_F32, ZK_F16, ZK_BF16 = 0, 1, 2
ZK_ROPE_HALF, ZK_ROPE_INTERLEAVED = 0, 1

STATUS_NAMES = {
    -1: "ZK_EINVAL",
    -2: "ZK_EDTYPE",
    -3: "ZK_EALIGN",
    -4: "ZK_EUNSUPPORTED",
    -5: "ZK_EWORKSPACE",
}

_i64 = ctypes.c_int64
_int = ctypes.c_int
_ptr = ctypes.c_void_p
_f32 = ctypes.c_float
_f64 = ctypes.c_double


class AttnDesc(ctypes.Structure):
    """Mirror of ``zk_attn_desc``."""

    _fields_ = [
        (name, _i64)
        for name in (
            "B", "Sq", "Skv", "Hq", "Hkv", "d",
            "q_sb", "q_ss", "q_sh",
            "k_sb", "k_ss", "k_sh",
            "v_sb", "v_ss", "v_sh",
            "o_sb", "o_ss", "o_sh",
            "dq_sb", "dq_ss", "dq_sh",
            "dk_sb", "dk_ss", "dk_sh",
            "dv_sb", "dv_ss", "dv_sh",
        )
    ] + [
        ("scale", _f32),
        ("causal", _int),
        ("window", _i64),
        ("dtype", _int),
    ]


class AdamwRegion(ctypes.Structure):
    """Mirror of ``zk_adamw_region``."""

    _fields_ = [("offset", _i64), ("rows", _i64), ("cols", _i64), ("ld_t", _i64),
                ("lowp_t", _ptr)]


# name -> (restype, argtypes)
SIGNATURES = {
    "zk_last_error": (ctypes.c_char_p, []),
    "zk_abi_version": (_int, []),
    "zk_device_info": (_int, [_int, ctypes.c_char_p, _int, ctypes.POINTER(_int),
                              ctypes.POINTER(_int), ctypes.POINTER(_i64)]),
    "zk_rmsnorm_fwd": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _i64,
                              _f32, _int, _int, _ptr]),
    "zk_rmsnorm_bwd_workspace": (_i64, [_i64, _i64]),
    "zk_rmsnorm_bwd": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _int,
                              _ptr, _i64, _i64, _i64, _int, _int, _ptr]),
    "zk_rmsnorm_bwd_noalloc": (_int, [_ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _int,
                                      _i64, _i64, _int, _int, _ptr]),
    "zk_swiglu_fwd": (_int, [_ptr, _ptr, _i64, _ptr, _i64, _i64, _i64, _int, _ptr]),
    "zk_swiglu_bwd": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _ptr, _ptr, _i64,
                             _i64, _i64, _int, _ptr]),
    "zk_gemm_nt_supported": (_int, [_i64, _i64, _i64]),
    "zk_gemm": (_int, [_ptr, _i64, _int, _ptr, _i64, _int, _ptr, _i64, _ptr, _i64, _i64, _i64,
                       _i64, _int, _ptr]),
    "zk_gemm_path": (_int, [_i64, _i64, _i64, _i64, _int, _i64, _int, _i64, _i64, _int]),
    "zk_gemm_nt": (_int, [_ptr, _i64, _ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _i64, _i64,
                          _int, _ptr]),
    "zk_gemm_swiglu": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _ptr, _ptr, _i64, _ptr, _i64, _ptr,
                               _i64, _i64, _i64, _i64, _int, _ptr]),
    "zk_swiglu_fwd_t": (_int, [_ptr, _ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _i64, _int,
                                _ptr]),
    "zk_swiglu_bwd_t": (_int, [_ptr, _i64, _ptr, _ptr, _i64, _ptr, _ptr, _i64, _ptr, _ptr,
                                _i64, _i64, _i64, _int, _ptr]),
    "zk_gemm_rope": (_int, [_ptr, _i64, _ptr, _i64, _ptr, _i64, _i64, _i64, _i64, _i64,
                            _i64, _i64, _ptr, _ptr, _i64, _ptr, _int, _int, _ptr]),
    "zk_rope": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _i64, _i64, _i64,
                       _i64, _i64, _i64, _i64, _ptr, _ptr, _i64, _ptr, _int,
                       _int, _int, _ptr]),
    "zk_attn_fwd": (_int, [ctypes.POINTER(AttnDesc), _ptr, _ptr, _ptr, _ptr,
                           _ptr, _ptr]),
    "zk_attn_fwd_t": (_int, [ctypes.POINTER(AttnDesc), _ptr, _ptr, _ptr, _ptr,
                             _ptr, _ptr, _i64, _ptr]),
    "zk_attn_bwd_workspace": (_i64, [ctypes.POINTER(AttnDesc)]),
    "zk_attn_bwd": (_int, [ctypes.POINTER(AttnDesc), _ptr, _ptr, _ptr, _ptr,
                           _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr]),
    "zk_attn_bwd_rope": (_int, [ctypes.POINTER(AttnDesc), _ptr, _ptr, _ptr, _ptr,
                                _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr, _ptr, _i64,
                                _ptr, _int, _ptr]),
    "zk_attn_bwd_rope_t": (_int, [ctypes.POINTER(AttnDesc), _ptr, _ptr, _ptr, _ptr,
                                  _ptr, _ptr, _ptr, _ptr, _ptr, _ptr, _i64, _ptr, _ptr, _i64,
                                  _ptr, _int, _ptr, _ptr, _ptr, _i64, _ptr]),
    "zk_adamw_step": (_int, [_ptr, _ptr, _int, _ptr, _ptr, _ptr, _int, _i64,
                             _f64, _f64, _f64, _f64, _f64, _i64, _ptr]),
    "zk_adamw_step_t": (_int, [_ptr, _ptr, _int, _ptr, _ptr, _ptr, _int, _ptr, _int, _i64,
                                _f64, _f64, _f64, _f64, _f64, _i64, _ptr]),
    "zk_cast": (_int, [_ptr, _int, _ptr, _int, _i64, _int, _ptr]),
    "zk_ce_fwd_chunk": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _ptr, _ptr, _int,
                               _ptr]),
    "zk_ce_bwd_chunk": (_int, [_ptr, _i64, _i64, _i64, _ptr, _i64, _ptr, _f32, _int, _ptr]),
    "zk_transpose": (_int, [_ptr, _i64, _ptr, _i64, _i64, _i64, _int, _ptr]),
    "zk_copy_to_host": (_int, [_ptr, _ptr, _i64, _int, _ptr]),
    "zk_copy_from_host": (_int, [_ptr, _ptr, _i64, _int, _ptr]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """Load (once) and return the library with typed signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise RuntimeError(
                    f"{LIB_PATH} is missing: build it with "
                    "`python -m zorse_amd.build` (or __graft_entry__.build())"
                )
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def exported_symbols() -> list[str]:
    return list(SIGNATURES)


def last_error() -> str:
    msg = lib().zk_last_error()
    return msg.decode() if msg else ""


def check(status: int, what: str) -> None:
    if status != 0:
        code = STATUS_NAMES.get(status, f"hipError {status}")
        raise RuntimeError(f"{what} failed with {code}: {last_error()}")


def dtype_code(dtype: torch.dtype) -> int:
    if dtype == torch.float32:
        return ZK_F32
    if dtype == torch.float16:
        return ZK_F16
    if dtype == torch.bfloat16:
        return ZK_BF16
    raise TypeError(f"unsupported dtype {dtype} (float32, float16, bfloat16)")


def stream_handle(device: torch.device | None = None) -> int:
    """hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
