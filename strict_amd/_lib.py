"""ctypes declarations of the libstrict_hip C ABI (include/strict_hip.h).

Loading fails loudly when ``libstrict_hip.so`` has not been built: there is no
CPU fallback anywhere in the package.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

import os

# STRICT_HIP_LIBRARY names another build of the library (e.g. a diagnostic one)
LIB_PATH = Path(os.environ.get("STRICT_HIP_LIBRARY") or
                Path(__file__).resolve().parent / "libstrict_hip.so")

SH_OK = 0
SH_ERR_INVALID_ARGUMENT = 1
SH_ERR_NO_DEVICE = 2
SH_ERR_HIP = 3
SH_ERR_OUT_OF_MEMORY = 4
SH_ERR_COMPILE = 5
SH_ERR_NOT_FOUND = 6
SH_ERR_UNSUPPORTED = 7
SH_ERR_INVALID_FILE = 8

STATUS_NAMES = {
    SH_OK: "SH_OK",
    SH_ERR_INVALID_ARGUMENT: "SH_ERR_INVALID_ARGUMENT",
    SH_ERR_NO_DEVICE: "SH_ERR_NO_DEVICE",
    SH_ERR_HIP: "SH_ERR_HIP",
    SH_ERR_OUT_OF_MEMORY: "SH_ERR_OUT_OF_MEMORY",
    SH_ERR_COMPILE: "SH_ERR_COMPILE",
    SH_ERR_NOT_FOUND: "SH_ERR_NOT_FOUND",
    SH_ERR_UNSUPPORTED: "SH_ERR_UNSUPPORTED",
    SH_ERR_INVALID_FILE: "SH_ERR_INVALID_FILE",
}


class DeviceInfo(ctypes.Structure):
    _fields_ = [
        ("device", ctypes.c_int),
        ("compute_units", ctypes.c_int),
        ("wavefront_size", ctypes.c_int),
        ("clock_khz", ctypes.c_int),
        ("memory_clock_khz", ctypes.c_int),
        ("memory_bus_width_bits", ctypes.c_int),
        ("total_memory_bytes", ctypes.c_size_t),
        ("lds_bytes_per_block", ctypes.c_size_t),
        ("name", ctypes.c_char * 256),
        ("arch", ctypes.c_char * 64),
    ]


class BcInstruction(ctypes.Structure):
    """sh_bc_instruction: one flattened Strict bytecode instruction."""
    _fields_ = [
        ("type", ctypes.c_int),
        ("register_count", ctypes.c_int),
        ("registers", ctypes.c_int * 3),
        ("identifier", ctypes.c_char_p),
        ("number", ctypes.c_double),
    ]


class StrictBinaryConstant(ctypes.Structure):
    """sh_strictbinary_constant: one value-carrying instruction of a method."""
    _fields_ = [
        ("instruction", ctypes.c_int),
        ("instruction_type", ctypes.c_int),
        ("kind", ctypes.c_int),
        ("register_id", ctypes.c_int),
        ("identifier", ctypes.c_char_p),
        ("count", ctypes.c_size_t),
    ]


class LlmConfig(ctypes.Structure):
    _fields_ = [
        ("arch", ctypes.c_int),
        ("layers", ctypes.c_int),
        ("hidden", ctypes.c_int),
        ("heads", ctypes.c_int),
        ("kv_heads", ctypes.c_int),
        ("head_dim", ctypes.c_int),
        ("intermediate", ctypes.c_int),
        ("vocab", ctypes.c_int),
        ("max_positions", ctypes.c_int),
        ("max_batch", ctypes.c_int),
        ("rope_theta", ctypes.c_float),
        ("norm_eps", ctypes.c_float),
    ]


_P = ctypes.c_void_p
_PP = ctypes.POINTER(ctypes.c_void_p)
_I = ctypes.c_int
_SZ = ctypes.c_size_t
_F = ctypes.c_float
_U = ctypes.c_uint

# name -> (restype, argtypes). Every entry point include/strict_hip.h declares.
SIGNATURES = {
    "sh_last_error": (ctypes.c_char_p, []),
    "sh_version": (_I, []),
    "sh_range_loop_target": (_I, [ctypes.c_longlong, _I]),
    "sh_device_count": (_I, [ctypes.POINTER(_I)]),
    "sh_create": (_I, [_I, _PP]),
    "sh_destroy": (_I, [_P]),
    "sh_device_info": (_I, [_P, ctypes.POINTER(DeviceInfo)]),
    "sh_sync": (_I, [_P]),
    "sh_stream": (_I, [_P, _PP]),
    "sh_alloc": (_I, [_P, _SZ, _PP]),
    "sh_free": (_I, [_P, _P]),
    "sh_upload": (_I, [_P, _P, _P, _SZ]),
    "sh_download": (_I, [_P, _P, _P, _SZ]),
    "sh_copy": (_I, [_P, _P, _P, _SZ]),
    "sh_memset": (_I, [_P, _P, _I, _SZ]),
    "sh_register_external": (_I, [_P, _P, _SZ]),
    "sh_unregister_external": (_I, [_P, _P]),
    "sh_timer_start": (_I, [_P]),
    "sh_timer_stop": (_I, [_P, ctypes.POINTER(_F)]),
    "sh_event_create": (_I, [_P, _PP]),
    "sh_event_record": (_I, [_P]),
    "sh_event_elapsed": (_I, [_P, _P, ctypes.POINTER(_F)]),
    "sh_event_destroy": (_I, [_P]),
    "sh_compile": (_I, [ctypes.c_char_p, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), _I,
                        _PP]),
    "sh_program_code": (_I, [_P, _PP, ctypes.POINTER(_SZ)]),
    "sh_program_log": (ctypes.c_char_p, [_P]),
    "sh_program_destroy": (_I, [_P]),
    "sh_instructions_to_hip": (_I, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), _I, _I,
                                    _P, _I, ctypes.c_char_p, _SZ, ctypes.POINTER(_SZ)]),
    "sh_strictbinary_load": (_I, [_P, _SZ, _PP]),
    "sh_strictbinary_free": (_I, [_P]),
    "sh_strictbinary_type_count": (_I, [_P, ctypes.POINTER(_I)]),
    "sh_strictbinary_type": (_I, [_P, _I, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I),
                                  ctypes.POINTER(_I)]),
    "sh_strictbinary_member": (_I, [_P, _I, _I, _I, ctypes.POINTER(ctypes.c_char_p),
                                    ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_I)]),
    "sh_strictbinary_method": (_I, [_P, _I, _I, ctypes.POINTER(ctypes.c_char_p),
                                    ctypes.POINTER(_I), ctypes.POINTER(ctypes.c_char_p),
                                    ctypes.POINTER(_I)]),
    "sh_strictbinary_entry_point": (_I, [_P, ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "sh_strictbinary_find": (_I, [_P, ctypes.c_char_p, ctypes.c_char_p, _I, ctypes.c_char_p,
                                  ctypes.POINTER(_I), ctypes.POINTER(_I)]),
    "sh_strictbinary_instructions": (_I, [_P, _I, _I, _P, _I, ctypes.POINTER(_I)]),
    "sh_strictbinary_constants": (_I, [_P, _I, _I, _P, _I, ctypes.POINTER(_I)]),
    "sh_strictbinary_constant_values": (_I, [_P, _I, _I, _I, _P, _SZ]),
    "sh_strictbinary_upload_f32": (_I, [_P, _P, _I, _I, _I, _P, _SZ]),
    "sh_strictbinary_serialize": (_I, [_P, _P, _SZ, ctypes.POINTER(_SZ)]),
    "sh_module_load": (_I, [_P, _P, _SZ, _PP]),
    "sh_module_function": (_I, [_P, ctypes.c_char_p, _PP]),
    "sh_module_unload": (_I, [_P]),
    "sh_launch": (_I, [_P, ctypes.POINTER(_U), ctypes.POINTER(_U), _U, _PP,
                       ctypes.POINTER(_F)]),
    "sh_binary_f32": (_I, [_P, _I, _P, _P, _P, _SZ]),
    "sh_fill_f32": (_I, [_P, _F, _P, _SZ]),
    "sh_saxpy_f32": (_I, [_P, _F, _P, _P, _P, _SZ]),
    "sh_sigmoid_f32": (_I, [_P, _P, _P, _SZ]),
    "sh_adjust_brightness_u8": (_I, [_P, _P, _P, _I, _I, _I, _I, _I]),
    "sh_box_blur5_u8": (_I, [_P, _P, _P, _I, _I, _I, _I]),
    "sh_bgr_to_rgba_u8": (_I, [_P, _P, _I, ctypes.c_size_t, _P, _I, _I]),
    "sh_rgb_to_bgr_u8": (_I, [_P, _P, _P, _I, _I, ctypes.c_size_t]),
    "sh_brightness_blur5_u8": (_I, [_P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "sh_gemm_bf16": (_I, [_P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "sh_gemm_fp8": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _I]),
    "sh_quantize_e4m3": (_I, [_P, _P, _I, _I, _P, _P]),
    "sh_pack_e4m3_tiles": (_I, [_P, _P, _I, _I, _P]),
    "sh_gemv_w8a16": (_I, [_P, _P, _P, _P, _P, _I, _I, _I]),
    "sh_rmsnorm_f32": (_I, [_P, _P, _P, _P, _I, _I, _F]),
    "sh_layernorm_f32": (_I, [_P, _P, _P, _P, _P, _I, _I, _F]),
    "sh_rope_f32": (_I, [_P, _P, _P, _I, _I, _I, _F]),
    "sh_swiglu_f32": (_I, [_P, _P, _P, _P, _SZ]),
    "sh_gelu_f32": (_I, [_P, _P, _P, _SZ]),
    "sh_argmax_f32": (_I, [_P, _P, _I, _I, _P]),
    "sh_attn_decode_f16": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F]),
    "sh_attn_decode_f16_noalloc": (_I, [_P, _P, _P, _P, _P, _P, _I, _I, _I, _I, _I, _F]),
    "sh_llm_create": (_I, [_P, ctypes.POINTER(LlmConfig), _PP]),
    "sh_llm_destroy": (_I, [_P]),
    "sh_llm_init_random": (_I, [_P, ctypes.c_uint64, _F]),
    "sh_llm_load_linear": (_I, [_P, ctypes.c_char_p, _I, _P]),
    "sh_llm_tensor": (_I, [_P, ctypes.c_char_p, _I, _PP, ctypes.POINTER(_SZ)]),
    "sh_llm_reset": (_I, [_P, _I]),
    "sh_llm_step": (_I, [_P, _P, _I]),
    "sh_llm_next_tokens": (_I, [_P, _P]),
    "sh_llm_generate": (_I, [_P, _P, _I, _I, _P]),
}

_lib = None


def load():
    """Load libstrict_hip.so and declare every C-ABI entry point."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(
                f"{LIB_PATH} is not built; run `make -C strict_amd/csrc` or "
                "__graft_entry__.build() (there is no CPU fallback)")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib
