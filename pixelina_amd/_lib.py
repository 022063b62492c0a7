"""ctypes binding of libpixhip.so (include/pixhip.h) for tests and the bench.

Loading fails loudly when the HIP library has not been built: there is no
CPU fallback anywhere on the product path.
"""
import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIBRARY = os.path.join(HERE, "libpixhip.so")

OK = 0
ERR_ARGUMENT = -1
ERR_UNSUPPORTED = -2
ERR_MEMORY = -3
ERR_DEVICE = -4
ERR_STATE = -5
ERR_OPEN = -6
ERR_FORMAT = -7

Q8_0 = 8
Q5_K = 13
Q6_K = 14

STAGE_QUANTIZE = 1
STAGE_MULTIPLY = 2

# Exported C symbols and their ctypes signatures (restype, argtypes).
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u64 = ctypes.c_uint64
_u32 = ctypes.c_uint32
_int = ctypes.c_int
SIGNATURES = {
    "pixhip_version": (_int, []),
    "pixhip_last_error": (ctypes.c_char_p, []),
    "pixhip_session_create": (_int, [_int, ctypes.POINTER(_vp)]),
    "pixhip_session_destroy": (None, [_vp]),
    "pixhip_session_set_stream": (_int, [_vp, _vp]),
    "pixhip_session_stream": (_vp, [_vp]),
    "pixhip_device_name": (_int, [_vp, ctypes.c_char_p, _sz]),
    "pixhip_memory_limits": (_int, [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "pixhip_prepare_stage": (_int, [_vp, _u64, _u64]),
    "pixhip_set_weight_budget": (_int, [_vp, _u64]),
    "pixhip_allocate": (_vp, [_vp, _sz]),
    "pixhip_free": (None, [_vp, _vp]),
    "pixhip_synchronize": (_int, [_vp]),
    "pixhip_copy_to_device": (_int, [_vp, _vp, _vp, _sz]),
    "pixhip_copy_to_host": (_int, [_vp, _vp, _vp, _sz]),
    "pixhip_copy_device": (_int, [_vp, _vp, _vp, _sz]),
    "pixhip_weight_get": (_int, [_vp, ctypes.c_char_p, _vp, _u64, _u32, _u64, _u64, ctypes.POINTER(_vp)]),
    "pixhip_weight_cache_info": (_int, [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "pixhip_weight_residency": (_int, [_vp, ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "pixhip_weight_shape": (_int, [_vp, ctypes.POINTER(_u32), ctypes.POINTER(_u64), ctypes.POINTER(_u64)]),
    "pixhip_matmul": (_int, [_vp, _vp, _vp, _sz, _vp]),
    "pixhip_matmul_ex": (_int, [_vp, _vp, _vp, _sz, _vp, _vp, _sz, _sz]),
    "pixhip_matmul_stage": (_int, [_vp, _vp, _vp, _sz, _vp, _vp, _sz, _sz, ctypes.c_uint]),
    "pixhip_matmul_ex_noalloc": (_int, [_vp, _vp, _vp, _sz, _vp, _vp, _sz, _sz]),
    "pixhip_quant_matmul": (_int, [_vp, _vp, _u32, _vp, _vp, _sz, _sz, _sz]),
    "pixhip_quantize_q8_0": (_int, [_vp, _vp, _vp, _sz, _sz]),
    "pixhip_quantize_q8_K": (_int, [_vp, _vp, _vp, _sz, _sz]),
    "pixhip_norm_quantize": (_int, [_vp, _u32, _vp, _sz, _sz, _vp, ctypes.c_float, _int, _vp, _vp, _vp]),
    "pixhip_silu_gate_quantize": (_int, [_vp, _u32, _vp, _vp, _sz, _sz, _vp, _vp]),
    "pixhip_pointwise": (_int, [_vp, ctypes.c_uint, _vp, _vp, _sz, _sz]),
    "pixhip_rope": (_int, [_vp, _vp, _sz, _sz, _sz, _vp, _vp, _int]),
    "pixhip_attention": (_int, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz, _int, _vp]),
    "pixhip_attention_ranges": (_int, [_vp, _vp, _sz, _vp, _vp, _sz, _sz, _sz, _sz, _vp, _sz, _sz, _vp]),
    "pixhip_model_open": (_int, [ctypes.c_char_p, _int, ctypes.POINTER(_vp)]),
    "pixhip_model_close": (None, [_vp]),
    "pixhip_model_data": (_vp, [_vp, ctypes.POINTER(_u64)]),
    "pixhip_model_tensor_count": (_u64, [_vp]),
    "pixhip_model_tensor_at": (_int, [_vp, _u64, _vp]),
    "pixhip_model_tensor": (_int, [_vp, ctypes.c_char_p, _vp]),
    "pixhip_model_metadata_count": (_u64, [_vp]),
    "pixhip_model_metadata_key": (ctypes.c_int64, [_vp, _u64, ctypes.c_char_p, _sz]),
    "pixhip_model_metadata_value": (ctypes.c_int64, [_vp, _u64, ctypes.c_char_p, _sz]),
    "pixhip_model_metadata": (ctypes.c_int64, [_vp, ctypes.c_char_p, ctypes.c_char_p, _sz]),
    "pixhip_model_weight": (_int, [_vp, _vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "pixhip_conv_weight_get": (_int, [_vp, ctypes.c_char_p, _vp, _u64, _u32, _u64, _u64, _u64, _u64, ctypes.POINTER(_vp)]),
    "pixhip_conv2d": (_int, [_vp, _vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    "pixhip_model_conv_weight": (_int, [_vp, _vp, ctypes.c_char_p, ctypes.POINTER(_vp)]),
    "pixhip_pointwise_ex": (_int, [_vp, ctypes.c_uint, _vp, _vp, _vp, _sz, _sz, ctypes.c_uint, ctypes.c_float, ctypes.c_float]),
    "pixhip_qwen_modulate": (_int, [_vp, _vp, _sz, _sz, _vp, _sz, _sz, _sz, _vp]),
    "pixhip_l2norm": (_int, [_vp, _vp, _sz, _sz, _vp, ctypes.c_float, _vp]),
    "pixhip_groupnorm": (_int, [_vp, _vp, _sz, _sz, _vp, _vp, _vp]),
    "pixhip_embedding": (_int, [_vp, _vp, ctypes.c_uint32, ctypes.c_uint64, ctypes.c_uint64, _vp, _sz, _vp]),
    "pixhip_rows": (_int, [_vp, _vp, _sz, _vp, _sz, _sz, _vp, _sz, _int]),
    "pixhip_copy_rows": (_int, [_vp, _vp, _sz, _sz, _vp, _sz, _sz, _sz, _sz, _sz, _sz]),
    "pixhip_copy_features": (_int, [_vp, _vp, _sz, _vp, _sz, _sz]),
    "pixhip_layout": (_int, [_vp, ctypes.c_uint, _vp, _sz, _sz, _vp, _sz, _sz, _sz, _sz]),
    "pixhip_shortcut": (_int, [_vp, _vp, _sz, _sz, _sz, _vp, _sz, _sz, _int, _int]),
    "pixhip_block_sums": (_int, [_vp, _vp, _vp, _sz, _vp, _vp]),
    "pixhip_timer_start": (_int, [_vp]),
    "pixhip_timer_stop": (_int, [_vp, ctypes.POINTER(ctypes.c_float)]),
    "pixhip_bench_matmul": (_int, [_vp, ctypes.POINTER(_vp), _sz, _vp, _sz, _vp, ctypes.c_uint, _sz,
                                   ctypes.POINTER(ctypes.c_float)]),
}

_lib = None


def load():
    """Load libpixhip.so once; raise if it is missing (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIBRARY):
        raise RuntimeError(f"{LIBRARY} is not built: run `python -m pixelina_amd.build` (HIP is required, there is no CPU path)")
    lib = ctypes.CDLL(LIBRARY)
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    _lib = lib
    return lib


class PixhipError(RuntimeError):
    def __init__(self, code, what):
        msg = load().pixhip_last_error().decode(errors="replace")
        super().__init__(f"{what} failed ({code}): {msg}")
        self.code = code


class ConvGeometry(ctypes.Structure):
    """pixhip_conv_geometry (PixConv2D, src/tensor.h:65-68)."""
    _fields_ = [("stride_x", ctypes.c_size_t), ("stride_y", ctypes.c_size_t), ("left", ctypes.c_size_t),
                ("right", ctypes.c_size_t), ("top", ctypes.c_size_t), ("bottom", ctypes.c_size_t)]


def check(code, what):
    if code != OK:
        raise PixhipError(code, what)
    return code


class AttentionRange(ctypes.Structure):
    """pixhip_attention_range (PixAttentionRange, src/tensor.h:58-63)."""
    _fields_ = [("query_begin", ctypes.c_size_t), ("query_end", ctypes.c_size_t), ("key_end", ctypes.c_size_t),
                ("causal", ctypes.c_int)]
