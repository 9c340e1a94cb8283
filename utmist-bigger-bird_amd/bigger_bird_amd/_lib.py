"""ctypes binding of libbb_attn.so (the C ABI declared in include/bb_attn.h).

The library is loaded lazily from this package directory. There is no fallback: if it is missing or the tensors are
not on a ROCm device, calls raise, so a run can never silently take another code path.
"""
import ctypes
from pathlib import Path

import torch

_PATH = Path(__file__).with_name("libbb_attn.so")
_LIB = None

c_i64p = ctypes.POINTER(ctypes.c_int64)
_vp, _i32, _i64, _f32, _sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_float, ctypes.c_size_t

# name -> (restype, argtypes)
SIGNATURES = {
    "bb_version": (_i32, []),
    "bb_last_error": (ctypes.c_char_p, []),
    "bb_init": (_i32, []),
    "bb_sparse_flash": (_i32, [_vp, c_i64p, _vp, c_i64p, _vp, c_i64p, _vp, _vp, c_i64p, _i32, _i32, _vp, _i64,
                               _vp, c_i64p, _i32, _i64, _i64, _i32, _i32, _i32, _i32, _i64, _i64, _i64, _f32, _i64,
                               _vp, _sz, _vp]),
    "bb_sparse_flash_workspace": (_sz, [_i32, _i64, _i64, _i32, _i32, _i32, _i64, _i64, _i32, _i32, _i64, _i32,
                                        _i32]),
    "bb_exact_attention": (_i32, [_vp, c_i64p, _vp, c_i64p, _vp, c_i64p, _vp, _vp, c_i64p, _i32, _i64, _i64, _i32, _i32,
                                  _i32, _i32, _f32, _vp, _sz, _vp]),
    "bb_exact_attention_workspace": (_sz, [_i32, _i64, _i64, _i32, _i32, _i32, _i32]),
    "bb_transpose_v": (_i32, [_vp, c_i64p, _i32, _i64, _i32, _vp, _vp]),
    "bb_transpose_v_cols": (_i64, [_i64]),
    "bb_routes": (_i32, [_vp, c_i64p, _vp, c_i64p, _vp, _i32, _i32, _i32, _i32, _i64, _i32, _i32, _i64, _i64, _i32,
                         _f32, _i32, _vp, _vp, _vp, _sz, _vp]),
    "bb_routes_workspace": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "bb_int8_quantize": (_i32, [_vp, _i32, _i64, _i64, _i32, _i64, _i32, _f32, _vp, _vp, _i32, _vp]),
    "bb_int8_dequantize": (_i32, [_vp, _vp, _i32, _i64, _i32, _vp, _i32, _vp]),
    "bb_decode": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _i32, _vp, c_i64p, _vp, c_i64p, _i64, _i32, _i32, _i32, _f32,
                         _vp, _i64, _vp, _sz, _vp]),
    "bb_decode_workspace": (_sz, [_i64, _i32, _i32, _i32]),
    "bb_decode_append": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _i32, _vp, _i64, _vp, _i64, _f32, _i64, _i32, _i32, _i32,
                                _f32, _vp, _i64, _vp, _sz, _vp]),
    "bb_decode_noalloc": (_i32, [_vp, _i64, _vp, _vp, _vp, _vp, _i32, _vp, c_i64p, _vp, c_i64p, _i64, _i32, _i32, _i32,
                                 _f32, _vp, _i64, _vp]),
    "bb_decode_noalloc_max_bytes": (_sz, []),
    "bb_rope_inplace": (_i32, [_vp, c_i64p, _i32, _i32, _i64, _i32, _vp, _vp, c_i64p, _i32, _vp]),
    "bb_sparse_decode": (_i32, [_vp, _i64, _vp, c_i64p, _vp, c_i64p, _vp, c_i64p, _i32, _i32, _i64, _vp, _i64, _i32,
                                _i32, _i32, _i32, _i32, _f32, _i32, _i32, _vp, _i64, _vp, _sz, _vp]),
    "bb_sparse_decode_workspace": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "bb_decode_route": (_i32, [_vp, _i64, _vp, c_i64p, _i64, _vp, _i64, _i32, _i32, _i32, _i32, _i32, _f32, _i32, _i32,
                               _vp, _i32, _vp, _vp, _sz, _vp]),
    "bb_decode_route_workspace": (_sz, [_i64, _i32, _i32, _i32, _i32]),
    "bb_gather_rows": (_i32, [_vp, c_i64p, _i64, _i32, _vp, _i64, _i32, _i32, _vp, c_i64p, _vp]),
    "bb_kv_append": (_i32, [_vp, c_i64p, _vp, c_i64p, _vp, _i64, _vp, _i64, _i32, _i32, _i64, _vp, _i64, _vp]),
    "bb_decode_step": (_i32, [_vp, _i64, _vp, c_i64p, _vp, c_i64p, _vp, _i64, _vp, _i64, _vp, _i64, _i64, _i32, _i32,
                              _i32, _i32, _i32, _i32, _f32, _i32, _vp, _vp, _i64, _vp, _sz, _vp]),
    "bb_decode_step_workspace": (_sz, [_i64, _i32, _i32, _i32, _i32, _i32, _i32]),
    "bb_topk_f32": (_i32, [_vp, _i64, _i32, _i64, _i32, _i32, _i32, _vp, _vp, _sz, _vp]),
    "bb_topk_f32_workspace": (_sz, [_i32, _i64]),
    "bb_argmax": (_i32, [_vp, _i64, _i32, _vp, _vp]),
    "bb_rms_norm": (_i32, [_vp, _i64, _i32, _i32, _vp, _f32, _i32, _vp, _i64, _vp]),
    "bb_add_rms_norm": (_i32, [_vp, _i64, _vp, _i64, _i32, _i32, _vp, _f32, _i32, _vp, _i64, _vp, _i64, _vp]),
    "bb_silu_mul": (_i32, [_vp, _vp, _i64, _i32, _vp, _vp]),
    "bb_gemv": (_i32, [_vp, _i64, _i32, _i32, _vp, _i32, _i32, _vp, _vp]),
    "bb_gemv_norm": (_i32, [_vp, _i64, _i32, _i32, _vp, _vp, _vp, _f32, _i32, _i32, _vp, _vp, _vp]),
    "bb_stream_read": (_i32, [_vp, _sz, _vp, _i32, _vp]),
    "bb_int8_quantize_pair": (_i32, [_vp, _vp, _i32, _i64, _i64, _i32, _i64, _i32, _f32, _vp, _vp, _vp, _vp, _i32, _vp]),
}


def lib():
    """The loaded library (raises RuntimeError when it has not been built)."""
    global _LIB
    if _LIB is None:
        if not _PATH.exists():
            raise RuntimeError(f"{_PATH} is missing: build it with `python utmist-bigger-bird_amd/bigger_bird_amd/build.py`")
        handle = ctypes.CDLL(str(_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype, fn.argtypes = res, args
        if torch.cuda.is_available():
            # per-device set-up of the current device ahead of any graph capture (bb_decode_noalloc's scratch)
            rc = handle.bb_init()
            if rc != 0:
                raise RuntimeError(handle.bb_last_error().decode(errors="replace"))
        _LIB = handle
    return _LIB


def library_path() -> Path:
    return _PATH


def check(rc: int) -> None:
    """Map a C ABI status to the reference's exception types (ValueError for argument errors)."""
    if rc == 0:
        return
    msg = lib().bb_last_error().decode(errors="replace")
    if rc == -1:
        raise ValueError(msg)
    raise RuntimeError(msg)


def i64s(*vals):
    return (ctypes.c_int64 * len(vals))(*[int(v) for v in vals])


def ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def stream_of(t: torch.Tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def require_gpu(*tensors, what="bigger_bird_amd"):
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError(f"{what} runs on the ROCm device only (got a {t.device} tensor)")


def workspace(nbytes: int, device) -> torch.Tensor:
    """Workspace from PyTorch's caching allocator (the library never allocates)."""
    return torch.empty(max(int(nbytes), 1), dtype=torch.uint8, device=device)
