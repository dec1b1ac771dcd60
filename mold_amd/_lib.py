"""ctypes binding of libmoldq.so (the C ABI in include/moldq.h).

The HIP library is the product: there is no fallback.  Loading fails loudly
when the shared object is missing or was not built for this tree.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmoldq.so")

MQ_OK, MQ_E_INVALID, MQ_E_HIP, MQ_E_OOM, MQ_E_UNSUPPORTED, MQ_E_IO = 0, -1, -2, -3, -4, -5
MQ_X_Q8K, MQ_X_Q8K_BLOCK_BYTES = 100, 304   # mq_quantize_x_q8k's activation blocks

# Every symbol include/moldq.h declares, with (restype, argtypes).
_vp, _i64, _int, _sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
_pp = ctypes.POINTER(ctypes.c_void_p)
SIGNATURES = {
    "mq_last_error": (ctypes.c_char_p, []),
    "mq_version": (_int, []),
    "mq_block_size": (_int, [_int]),
    "mq_type_size": (_int, [_int]),
    "mq_ctx_create": (_int, [_int, _pp]),
    "mq_ctx_destroy": (None, [_vp]),
    "mq_ctx_reserve_arena": (_int, [_vp, _sz]),
    "mq_ctx_reserve_scratch": (_int, [_vp, _sz]),
    "mq_ctx_reserve_stream_scratch": (_int, [_vp, _vp, _sz]),
    "mq_ctx_set_stream_tail_split": (_int, [_vp, _vp, _int]),
    "mq_qmatmul_workspace_size": (_int, [_vp, _vp, _int, _i64, _int, ctypes.POINTER(_sz)]),
    "mq_qtensor_upload": (_int, [_vp, _int, _i64, _i64, _vp, _sz, _pp]),
    "mq_qtensor_from_device": (_int, [_vp, _int, _i64, _i64, _vp, _sz, _vp, _pp]),
    "mq_quantize": (_int, [_vp, _int, _i64, _i64, _vp, _i64, _vp, _pp]),
    "mq_lora_apply": (_int, [_vp, _i64, _i64, _i64, _vp, _i64, _vp, _i64, _int, ctypes.c_float, _vp]),
    "mq_quantize_fp8": (_int, [_vp, _int, _i64, _i64, _vp, _i64, ctypes.c_float, _vp, _pp]),
    "mq_qtensor_download": (_int, [_vp, _vp, _vp, _sz]),
    "mq_qtensor_concat_rows": (_int, [_vp, _vp, _i64, _pp]),
    "mq_qtensor_free": (None, [_vp]),
    "mq_qtensor_info": (_int, [_vp, ctypes.POINTER(_int), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                               ctypes.POINTER(_sz), ctypes.POINTER(_sz)]),
    "mq_dequantize": (_int, [_vp, _vp, _vp, _int, _vp]),
    "mq_qmatmul": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _int, _i64, _vp, _int, _vp]),
    "mq_qmatmul_act_from": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _int, _i64, _vp, _int, _i64, _vp]),
    "mq_quantize_x_q8k": (_int, [_vp, _vp, _int, _i64, _i64, _i64, _vp, _vp]),
    "mq_qmatmul_noalloc": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _int, _i64, _vp, _int, _vp]),
    "mq_qmatmul_gated_add": (_int, [_vp, _vp, _vp, _int, _i64, _i64, _vp, _i64, _vp, _vp, _vp]),
    "mq_adaln_modulate": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, ctypes.c_float, _vp, _i64, _vp]),
    "mq_gelu_tanh_bf16": (_int, [_vp, _int, _i64, _i64, _i64, _vp, _i64, _vp]),
    "mq_qk_norm_rope": (_int, [_vp, _int, _i64, _i64, _int, _int, _vp, _vp, ctypes.c_float, _vp, _vp, _vp, _vp,
                               _vp, _i64, _i64, _vp]),
    "mq_attn_pad_correct": (_int, [_vp, _i64, _int, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _vp, _vp, _i64, _i64,
                                   _vp, _vp]),
    "mq_gguf_open": (_int, [ctypes.c_char_p, _pp]),
    "mq_gguf_close": (None, [_vp]),
    "mq_gguf_tensor_count": (_i64, [_vp]),
    "mq_gguf_find": (_i64, [_vp, ctypes.c_char_p]),
    "mq_gguf_tensor_info": (_int, [_vp, _i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_int),
                                   ctypes.POINTER(_int), ctypes.POINTER(_i64), ctypes.POINTER(ctypes.c_uint64),
                                   ctypes.POINTER(_sz)]),
    "mq_gguf_load_tensor": (_int, [_vp, _vp, _i64, _pp]),
    "mq_gguf_load_tensors": (_int, [_vp, _vp, _vp, _i64, _vp]),
    "mq_gguf_read_tensor": (_int, [_vp, _i64, _vp, _sz]),
    "mq_gguf_version": (_int, [_vp]),
    "mq_gguf_kv_count": (_i64, [_vp]),
    "mq_gguf_find_kv": (_i64, [_vp, ctypes.c_char_p]),
    "mq_gguf_kv_info": (_int, [_vp, _i64, ctypes.POINTER(ctypes.c_char_p), ctypes.POINTER(_int), ctypes.POINTER(_int),
                               ctypes.POINTER(ctypes.c_uint64)]),
    "mq_gguf_kv_int": (_int, [_vp, _i64, ctypes.c_uint64, ctypes.POINTER(_i64)]),
    "mq_gguf_kv_float": (_int, [_vp, _i64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_double)]),
    "mq_gguf_kv_str": (_int, [_vp, _i64, ctypes.c_uint64, ctypes.POINTER(ctypes.c_void_p),
                              ctypes.POINTER(ctypes.c_uint64)]),
    "mq_gguf_writer_create": (_int, [ctypes.c_char_p, ctypes.c_uint32, _pp]),
    "mq_gguf_writer_free": (None, [_vp]),
    "mq_gguf_writer_kv_scalar": (_int, [_vp, ctypes.c_char_p, _int, _vp]),
    "mq_gguf_writer_kv_str": (_int, [_vp, ctypes.c_char_p, ctypes.c_char_p]),
    "mq_gguf_writer_kv_array": (_int, [_vp, ctypes.c_char_p, _int, _vp, ctypes.c_uint64]),
    "mq_gguf_writer_kv_str_array": (_int, [_vp, ctypes.c_char_p, ctypes.POINTER(ctypes.c_char_p), ctypes.c_uint64]),
    "mq_gguf_writer_add_tensor": (_int, [_vp, ctypes.c_char_p, _int, _int, ctypes.POINTER(_i64), _vp, _sz]),
    "mq_gguf_writer_add_qtensor": (_int, [_vp, _vp, ctypes.c_char_p, _vp, _int, ctypes.POINTER(_i64)]),
    "mq_gguf_writer_finish": (_int, [_vp]),
}

_lib = None


class MoldqError(RuntimeError):
    """A negative return code from libmoldq, with mq_last_error()'s message."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"moldq error {code}: {msg}")
        self.code = code


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libmoldq.so once.  Raises ImportError when it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise ImportError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    # torch first: it brings the process's HIP runtime (libamdhip64.so.7), which
    # libmoldq then shares by SONAME, so device pointers and streams agree.
    try:
        import torch  # noqa: F401
    except Exception:
        pass
    lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def check(rc: int) -> None:
    if rc != MQ_OK:
        msg = load().mq_last_error()
        raise MoldqError(rc, msg.decode() if msg else "")
