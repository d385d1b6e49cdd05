"""ctypes binding of libnanovllm_amd.so (the C ABI in include/nanovllm_amd.h).

The library is built in-tree by extend-nano-vllm_amd/csrc/Makefile into
nanovllm_amd/lib/.  There is no fallback: if the library is missing every
kernel call raises ``NativeLibraryError``.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "lib", "libnanovllm_amd.so")
CSRC_DIR = os.path.join(os.path.dirname(_PKG), "csrc")

NVA_OK = 0
NVA_ERR_ARG = 1
NVA_ERR_WORKSPACE = 2
NVA_ERR_UNSUPPORTED = 3
NVA_ERR_LAUNCH = 4
NVA_ERR_CAPACITY = 5
ARGMAX_STATIC_KEYS = 65536      # NVA_ARGMAX_STATIC_KEYS of the header

KV_BF16 = 0
KV_FP8_E4M3 = 1

# Every symbol the header declares, with (restype, argtypes).
_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_INT = ctypes.c_int
_F32 = ctypes.c_float
_SZ = ctypes.c_size_t

SIGNATURES = {
    "nva_status_string": (ctypes.c_char_p, [_INT]),
    "nva_version": (ctypes.c_char_p, []),
    "nva_store_kvcache": (_INT, [_P, _I64, _P, _I64, _P, _P, _INT, _P, _I32, _I32, _I32, _I64,
                                 _P, _P, _P]),
    "nva_store_kvcache_paged": (_INT, [_P, _I64, _P, _I64, _P, _P, _INT, _I64, _I64, _I64, _I32,
                                       _I32, _P, _I32, _I32, _I32, _P, _P, _P]),
    "nva_rollback": (_INT, [_P, _P, _I32, _P, _P, _P, _P, _INT, _I32, _I64, _I32, _I64, _INT, _P]),
    "nva_aux_gather": (_INT, [_P, _P, _I32, _I64, _I32, _I32, _P, _I32, _P, _I64, _P]),
    "nva_argmax_workspace_size": (_SZ, [_I32, _I32, _I32]),
    "nva_argmax_accept": (_INT, [_P, _I64, _I32, _P, _I32, _I32, _P, _P, _P, _P, _P, _SZ, _P]),
    "nva_argmax_accept_static": (_INT, [_P, _I64, _I32, _P, _I32, _I32, _P, _P, _P, _P, _P]),
    "nva_argmax_rows": (_INT, [_P, _I64, _I32, _I32, _P, _P, _P, _SZ, _P]),
    "nva_paged_attention_workspace_size": (_SZ, [_I32, _I32, _I32, _I32, _I32, _I32, _I32]),
    "nva_paged_attention_varlen": (_INT, [_P, _I64, _I64, _P, _P, _INT, _I64, _I64, _I64, _I32,
                                          _I32, _P, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32,
                                          _I32, _I32, _I32, _F32, _P, _P, _P, _I64, _I64, _P, _SZ, _P]),
    "nva_paged_attention_decode": (_INT, [_P, _I64, _I64, _P, _P, _INT, _I64, _I64, _I64, _I32,
                                          _I32, _P, _P, _I64, _I32, _I32, _I32, _I32, _I32, _I32, _F32,
                                          _P, _P, _P, _I64, _I64, _P, _SZ, _P]),
    "nva_rms_norm": (_INT, [_P, _I64, _P, _P, _I64, _I32, _I32, _F32, _P]),
    "nva_add_rms_norm": (_INT, [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I32, _I32, _F32, _P]),
    "nva_add_then_rms_norm": (_INT, [_P, _I64, _P, _I64, _P, _P, _I64, _P, _I64, _I32, _I32, _F32,
                                     _P]),
    "nva_qk_norm_rope": (_INT, [_P, _I64, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _F32, _P,
                                _P, _P]),
    "nva_qk_norm_rope_store": (_INT, [_P, _I64, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32,
                                      _F32, _P, _P, _P, _INT, _I64, _I64, _I64, _I32, _I32, _P,
                                      _P, _P, _P]),
    "nva_silu_mul": (_INT, [_P, _I64, _P, _I64, _I32, _I32, _P]),
    "nva_verify_metadata": (_INT, [_P, _P, _I32, _P, _I64, _I32, _I32, _P, _P, _P, _P, _I32, _P]),
    "nva_draft_metadata": (_INT, [_P, _P, _P, _I32, _I32, _I32, _P, _I64, _I32, _I32, _I32, _P,
                                  _P, _P, _P]),
    "nva_verify_input_ids": (_INT, [_P, _P, _P, _P, _I64, _I32, _I32, _P, _P]),
    "nva_commit_metadata": (_INT, [_P, _P, _I32, _I32, _P, _I32, _P, _I64, _I32, _I32, _I32, _P,
                                   _P, _P, _P, _P, _P, _P, _I32, _P]),
}


class NativeLibraryError(RuntimeError):
    """The HIP library is missing or could not be loaded."""


class KernelError(RuntimeError):
    """A kernel entry point returned a non-OK status."""


_lib: ctypes.CDLL | None = None


def build(verbose: bool = False) -> str:
    """Compile libnanovllm_amd.so for gfx950 with the committed Makefile."""
    cmd = ["make", "-C", CSRC_DIR, "-j8"]
    if not verbose:
        cmd.insert(1, "-s")
    subprocess.run(cmd, check=True)
    return LIB_PATH


def load() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryError(
            f"{LIB_PATH} is missing: build it with `make -C {CSRC_DIR}` "
            "(or __graft_entry__.build()); there is no non-HIP fallback")
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as exc:  # pragma: no cover - depends on the machine
        raise NativeLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status == NVA_OK:
        return
    msg = load().nva_status_string(status).decode()
    if status in (NVA_ERR_ARG, NVA_ERR_UNSUPPORTED, NVA_ERR_CAPACITY):
        raise ValueError(f"{what}: {msg} (status {status})")
    raise KernelError(f"{what}: {msg} (status {status})")
