"""ctypes binding of libyllm_hip.so (the C ABI in include/yllm_hip.h).

The library is loaded from the package directory.  There is no fallback: if
it is missing, importing any op raises with the build command to run.
"""
from __future__ import annotations

import ctypes
from ctypes import POINTER, c_char_p, c_float, c_int, c_size_t, c_uint16, c_uint32, c_uint64, c_void_p
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libyllm_hip.so"

F16, F32, BF16 = 0, 1, 2
OK, EINVAL, ENOSPC, EDEVICE = 0, -22, -28, -5

# name -> (restype, argtypes); every symbol declared in include/yllm_hip.h
SIGNATURES = {
    "yhip_last_error": (c_char_p, []),
    "yhip_version": (c_char_p, []),
    "yhip_kv_layer_elems": (c_uint64, [c_uint32, c_uint32, c_uint32]),
    "yhip_kv_store": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                              c_uint32, c_uint32, c_uint32, c_void_p]),
    "yhip_kv_from_engine": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                    c_uint32, c_uint32, c_void_p]),
    "yhip_kv_to_engine": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                  c_uint32, c_uint32, c_void_p]),
    "yhip_attn_decode": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32,
                                 c_uint32, c_uint32, c_void_p, c_void_p, c_size_t, c_void_p]),
    "yhip_attn_decode_rope": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32,
                                      c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_float, c_void_p, c_void_p,
                                      c_size_t, c_void_p]),
    "yhip_attn_decode_batch": (c_int, [c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_void_p,
                                       c_void_p, c_uint32, c_uint32, c_uint64, c_uint32, c_uint32,
                                       c_uint32, c_uint32, c_void_p, c_uint32, c_void_p, c_size_t,
                                       c_void_p]),
    "yhip_attn_decode_batch_noalloc": (c_int, [c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_void_p,
                                               c_void_p, c_uint32, c_uint32, c_uint64, c_uint32, c_uint32,
                                               c_uint32, c_uint32, c_void_p, c_uint32, c_void_p]),
    "yhip_attn_decode_workspace": (c_size_t, [c_uint32, c_uint32, c_uint64, c_uint32, c_uint32, c_uint32]),
    "yhip_attn_prefill": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_uint32, c_uint32, c_void_p,
                                  c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                  c_void_p, c_uint32, c_void_p, c_size_t, c_void_p]),
    "yhip_attn_prefill_workspace": (c_size_t, [c_uint32, c_uint32, c_uint32, c_uint32, c_uint32]),
    "yhip_gdn_step": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32,
                              c_uint32, c_uint32, c_float, c_void_p]),
    "yhip_gdn_chunk": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_uint32, c_void_p,
                               c_uint32, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_float,
                               c_void_p, c_size_t, c_void_p]),
    "yhip_gdn_chunk_workspace": (c_size_t, [c_uint32, c_uint32, c_uint32]),
    "yhip_gdn_gates": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_uint32, c_void_p]),
    "yhip_rope_kv_store": (c_int, [c_void_p, c_uint32, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p,
                                   c_uint32, c_void_p, c_void_p, c_uint32, c_uint32, c_uint32, c_uint32, c_uint32,
                                   c_uint32, c_uint32, c_uint32, c_float, c_void_p]),
    "yhip_o_proj_workspace": (c_size_t, [c_uint32, c_uint32, c_uint32, c_uint32, c_uint32]),
    "yhip_o_proj": (c_int, [c_void_p, c_uint32, c_void_p, c_uint32, c_uint32, c_void_p, c_uint32, c_uint32, c_uint32,
                            c_uint32, c_void_p, c_size_t, c_void_p]),
    "yhip_gdn_decode": (c_int, [c_void_p] * 13 + [c_uint32] * 5 + [c_float, c_float, c_void_p]),
    "yhip_gdn_conv": (c_int, [c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32,
                              c_uint32, c_uint32, c_int, c_void_p]),
    "yhip_gdn_gated_norm": (c_int, [c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32, c_void_p, c_uint32,
                                    c_uint32, c_uint32, c_uint32, c_float, c_void_p]),
    "yhip_synth_normal": (None, [c_uint64, c_uint64, c_float, POINTER(c_float), c_uint64]),
    "yhip_synth_round_f16": (None, [POINTER(c_float), c_uint64]),
    "yhip_synth_round_bf16": (None, [POINTER(c_float), c_uint64]),
    "yhip_host_f32_to_f16": (None, [POINTER(c_float), POINTER(c_uint16), c_uint64]),
    "yhip_host_f16_to_f32": (None, [POINTER(c_uint16), POINTER(c_float), c_uint64]),
    "yhip_host_f32_to_bf16": (None, [POINTER(c_float), POINTER(c_uint16), c_uint64]),
}

_lib = None


class YhipError(RuntimeError):
    def __init__(self, code: int, msg: str):
        super().__init__(f"{msg} (code {code})")
        self.code = code


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with `python -m yllm_amd.build` "
                "(there is no CPU fallback for the attention ops)")
        handle = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(rc: int) -> None:
    if rc != OK:
        msg = lib().yhip_last_error().decode(errors="replace")
        raise YhipError(rc, msg)
