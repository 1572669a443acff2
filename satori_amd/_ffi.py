"""ctypes binding of libsatori_hip.so (the C ABI in include/satori_hip.h).

The library is loaded from this package directory only; there is no fallback implementation, so a missing
or unbuildable library is an error at import of the binding.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "libsatori_hip.so")

P = ctypes.c_void_p
I = ctypes.c_int
SZ = ctypes.c_size_t
PP = ctypes.POINTER(ctypes.c_void_p)

# name -> argument types; every entry point returns int (status) except the two noted.
SIGNATURES = {
    "satori_hip_abi_version": (I, []),
    "satori_hip_last_error": (ctypes.c_char_p, []),
    "satori_hip_device_count": (I, [ctypes.POINTER(I)]),
    "satori_hip_context_create": (I, [I, PP]),
    "satori_hip_context_destroy": (I, [P]),
    "satori_hip_context_stream": (I, [P, PP]),
    "satori_hip_ternary2_create": (I, [P, I, I, I, P, SZ, PP]),
    "satori_hip_quantized_create": (I, [P, I, I, I, P, SZ, PP]),
    "satori_hip_ternary2_open": (I, [P, ctypes.c_char_p, PP]),
    "satori_hip_matrix_clone": (I, [P, PP]),
    "satori_hip_matrix_destroy": (I, [P]),
    "satori_hip_matrix_shape": (I, [P, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I),
                                    ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_matvec": (I, [P, P, SZ, P, SZ]),
    "satori_hip_matvec_batch": (I, [P, P, SZ, I, P, SZ]),
    "satori_hip_quantize_q8k": (I, [P, P, I, P, SZ]),
    "satori_hip_matvec_device": (I, [P, P, P, P]),
    "satori_hip_matvec_batch_device": (I, [P, P, I, P, P]),
    "satori_hip_group_create": (I, [P, P, I, P, P, I, PP]),
    "satori_hip_group_execute": (I, [P, P]),
    "satori_hip_group_execute_batch": (I, [P, I, P]),
    "satori_hip_group_set_input": (I, [P, I, P, P, P, ctypes.c_float, P]),
    "satori_hip_group_set_output": (I, [P, I, P, P]),
    "satori_hip_group_destroy": (I, [P]),
    "satori_hip_step_create": (I, [P, P, I, PP]),
    "satori_hip_step_execute": (I, [P, P]),
    "satori_hip_step_destroy": (I, [P]),
    "satori_hip_device_alloc": (I, [P, SZ, PP]),
    "satori_hip_device_free": (I, [P, P]),
    "satori_hip_copy": (I, [P, P, P, SZ, I]),
    "satori_hip_synchronize": (I, [P]),
    "satori_hip_payload_length": (I, [I, I, I, I, ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_ternary2_validate": (I, [I, I, I, P, SZ]),
    "satori_hip_quantized_validate": (I, [I, I, I, P, SZ]),
    "satori_hip_ternary2_quantize": (I, [P, I, I, I, P, SZ]),
    "satori_hip_quantize_weights": (I, [I, P, I, I, P, SZ]),
    "satori_hip_bitplane_create": (I, [P, I, I, I, P, SZ, PP]),
    "satori_hip_bitplane_open": (I, [P, ctypes.c_char_p, PP]),
    "satori_hip_bitplane_load": (I, [ctypes.c_char_p, ctypes.POINTER(I), ctypes.POINTER(I), ctypes.POINTER(I), P, SZ,
                                     ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_bitplane_from_ternary2": (I, [I, I, I, P, SZ, P, SZ]),
    "satori_hip_bitplane_to_ternary2": (I, [I, I, I, P, SZ, P, SZ]),
    "satori_hip_bitplane_validate": (I, [I, I, I, P, SZ]),
    "satori_hip_capture_begin": (I, [P]),
    "satori_hip_capture_end": (I, [P, PP]),
    "satori_hip_rms_norm": (I, [P, P, P, ctypes.c_float, I, I, P, P]),
    "satori_hip_rms_norm_heads": (I, [P, P, P, ctypes.c_float, I, I, P]),
    "satori_hip_rope": (I, [P, P, I, I, I, P]),
    "satori_hip_rope_half": (I, [P, P, I, I, I, ctypes.c_double, I, P]),
    "satori_hip_swiglu": (I, [P, P, P, I, P, P]),
    "satori_hip_add": (I, [P, P, P, I, P, P]),
    "satori_hip_swiglu_q8k": (I, [P, P, P, I, P, P, P]),
    "satori_hip_add_rms_norm_q8k": (I, [P, P, P, P, ctypes.c_float, I, P, P, P]),
    "satori_hip_quantize_q8k_device": (I, [P, P, I, I, P, P]),
    "satori_hip_grouped_attention": (I, [P, P, P, P, I, I, I, I, P, P]),
    "satori_hip_grouped_attention_static": (I, [P, P, P, P, I, I, I, I, P, P]),
    "satori_hip_attention_decode": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I, ctypes.c_double, I, P, P, P]),
    "satori_hip_rope_table": (I, [P, I, I, ctypes.c_double, P, P]),
    "satori_hip_add_rms_norm": (I, [P, P, P, P, ctypes.c_float, I, P, P]),
    "satori_hip_attention_inputs": (I, [P, P, P, P, P, P, P, P, P, I, I, I, I, ctypes.c_double, I, P]),
    "satori_hip_matrix_decode_row": (I, [P, I, P, P]),
    "satori_hip_gguf_open": (I, [ctypes.c_char_p, PP]),
    "satori_hip_gguf_close": (I, [P]),
    "satori_hip_gguf_data_offset": (I, [P, ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_tensor_count": (I, [P, ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_tensor_find": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_tensor_info": (I, [P, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(I),
                                        ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_uint32),
                                        ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_tensor_window": (I, [P, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, PP]),
    "satori_hip_gguf_metadata_count": (I, [P, ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_metadata_find": (I, [P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_metadata_info": (I, [P, ctypes.c_int64, ctypes.POINTER(ctypes.c_char_p),
                                          ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(ctypes.c_int64),
                                          ctypes.POINTER(ctypes.c_int64), ctypes.POINTER(ctypes.c_int64),
                                          ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_metadata_window": (I, [P, ctypes.c_int64, PP, ctypes.POINTER(ctypes.c_int64)]),
    "satori_hip_gguf_matrix_create": (I, [P, P, ctypes.c_int64, PP]),
}

_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library; raises if it has not been built (``python -m satori_amd.build``)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(f"{LIB_PATH} is missing: build it with `python -m satori_amd.build`")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (restype, argtypes) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        _lib = handle
    return _lib
