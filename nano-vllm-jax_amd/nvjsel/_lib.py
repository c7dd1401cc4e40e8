"""ctypes binding of libnvjsel.so (the C ABI declared in include/nvjsel.h).

Loading is lazy, once per process, under a lock -- the pattern of the
reference's native bindings (nanovllm_jax/kernels/cuda_fp32_ffi.py:181-188,
nanovllm_jax/kernels/flashinfer_ffi.py:139-166).  There is no fallback: if the
library is missing the call raises, so a GPU run can never silently pass on a
non-native path.
"""
from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libnvjsel.so"
ABI_VERSION = 2

F32, BF16, F16 = 0, 1, 2
W_VH, W_HV = 0, 1

STATUS = {0: "OK", -1: "EINVAL", -2: "EUNSUPPORTED", -3: "EWORKSPACE", -4: "EHIP"}

# name -> (restype, argtypes); mirrors include/nvjsel.h
_vp, _i, _sz, _i64, _f = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t, ctypes.c_int64, ctypes.c_float
SIGNATURES = {
    "nvjsel_abi_version": (_i, []),
    "nvjsel_last_error": (ctypes.c_char_p, []),
    "nvjsel_lm_head_workspace_size": (_sz, [_i]),
    "nvjsel_lm_head_top1": (_i, [_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _sz, _vp]),
    "nvjsel_lm_head_top1_noalloc": (_i, [_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp]),
    "nvjsel_lm_head_sample": (_i, [_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp, _vp, _vp, _sz, _vp]),
    "nvjsel_lm_head_logits": (_i, [_vp, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _i, _i64, _vp]),
    "nvjsel_lm_head_prenorm_workspace_size": (_sz, [_i, _i]),
    "nvjsel_rms_norm": (_i, [_vp, _i, _vp, _i, _f, _i, _i, _i, _vp, _vp]),
    "nvjsel_lm_head_top1_prenorm": (_i, [_vp, _i, _vp, _i, _f, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp,
                                         _vp, _sz, _vp]),
    "nvjsel_lm_head_sample_prenorm": (_i, [_vp, _i, _vp, _i, _f, _i, _vp, _i, _i, _i, _i, _i, _i, _vp, _vp,
                                           _vp, _vp, _sz, _vp]),
    "nvjsel_sample_workspace_size": (_sz, [_i, _i]),
    "nvjsel_sample": (_i, [_vp, _i, _i, _i, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
    "nvjsel_derive_keys": (_i, [_vp, _vp, _i, _vp, _vp, _vp]),
    "nvjsel_derive_keys_table": (_i, [_vp, _i, _vp, _i, _vp, _vp]),
    "nvjsel_topk_workspace_size": (_sz, [_i, _i]),
    "nvjsel_topk": (_i, [_vp, _i, _i, _i, _i64, _i, _vp, _vp, _vp, _sz, _vp]),
    "nvjsel_debug_gumbel_draws": (_i, [ctypes.c_uint32, _i, _vp, _vp, _vp]),
    "nvjsel_debug_sample_topp": (_i, [_vp, _i, _i, _i, _i64, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _vp, _sz, _vp]),
}


class NvjselError(RuntimeError):
    """A libnvjsel entry point returned a non-zero status."""

    def __init__(self, fn: str, code: int, message: str):
        super().__init__(f"{fn} -> {STATUS.get(code, code)}: {message}")
        self.code = code


class NativeLibraryMissing(ImportError):
    pass


_lock = threading.Lock()
_lib = None


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise NativeLibraryMissing(
                f"{LIB_PATH} is not built; run __graft_entry__.build() "
                "(or python nano-vllm-jax_amd/nvjsel/build.py)")
        lib = ctypes.CDLL(str(LIB_PATH), mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.nvjsel_abi_version()
        if ver != ABI_VERSION:
            raise NativeLibraryMissing(f"libnvjsel ABI {ver} != expected {ABI_VERSION}; rebuild")
        _lib = lib
        return lib


def call(name: str, *args) -> None:
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        msg = lib.nvjsel_last_error().decode(errors="replace")
        raise NvjselError(name, rc, msg)


def exported_symbols() -> list[str]:
    return list(SIGNATURES)
