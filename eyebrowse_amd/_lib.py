"""ctypes binding of libeyebrowse_hip.so (the C ABI in include/eyebrowse_hip.h).

The library is built in-tree by ``eyebrowse_amd.build``. Loading fails loudly when it is
missing: there is no CPU or PyTorch fallback for any entry point.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libeyebrowse_hip.so")

c_size = ctypes.c_size_t
c_f32p = ctypes.POINTER(ctypes.c_float)
c_vp = ctypes.c_void_p
c_int = ctypes.c_int
c_float = ctypes.c_float
c_st = ctypes.c_int  # eb_status


class AttentionDesc(ctypes.Structure):
    """eb_attention_desc."""
    _fields_ = [
        ("n_heads", c_size),
        ("n_kv_heads", c_size),
        ("head_dim", c_size),
        ("scale", c_float),
        ("norm_eps", c_float),
        ("q_norm", c_vp),
        ("k_norm", c_vp),
        ("v_norm", c_vp),
        ("window", c_size),
        ("q_proj", c_vp),
        ("k_proj", c_vp),
        ("v_proj", c_vp),
        ("o_proj", c_vp),
        ("hidden", c_size),
    ]


# name -> (restype, argtypes); every symbol include/eyebrowse_hip.h declares.
SIGNATURES = {
    "eb_last_error": (ctypes.c_char_p, []),
    "eb_status_name": (ctypes.c_char_p, [c_st]),
    "eb_dtype_size": (c_size, [c_int]),
    "eb_version": (ctypes.c_char_p, []),
    "eb_device_new": (c_st, [c_int, ctypes.POINTER(c_vp)]),
    "eb_device_release": (None, [c_vp]),
    "eb_device_synchronize": (c_st, [c_vp]),
    "eb_device_stream": (c_vp, [c_vp]),
    "eb_device_cu_count": (c_int, [c_vp]),
    "eb_device_pooled": (c_size, [c_vp, c_size]),
    "eb_pool_max_bytes": (c_size, []),
    "eb_tensor_empty": (c_st, [c_vp, ctypes.POINTER(c_size), c_size, c_int, ctypes.POINTER(c_vp)]),
    "eb_tensor_from_f32": (c_st, [c_vp, ctypes.POINTER(c_size), c_size, c_f32p, c_size,
                                  ctypes.POINTER(c_vp)]),
    "eb_tensor_from_u32": (c_st, [c_vp, ctypes.POINTER(c_size), c_size,
                                  ctypes.POINTER(ctypes.c_uint32), c_size, ctypes.POINTER(c_vp)]),
    "eb_tensor_to_f32": (c_st, [c_vp, c_f32p, c_size]),
    "eb_tensor_read_bytes": (c_st, [c_vp, c_vp, c_size]),
    "eb_tensor_release": (None, [c_vp]),
    "eb_tensor_ndim": (c_size, [c_vp]),
    "eb_tensor_dim": (c_size, [c_vp, c_size]),
    "eb_tensor_numel": (c_size, [c_vp]),
    "eb_tensor_nbytes": (c_size, [c_vp]),
    "eb_tensor_dtype": (c_int, [c_vp]),
    "eb_tensor_data": (c_vp, [c_vp]),
    "eb_recorder_new": (c_st, [c_vp, ctypes.POINTER(c_vp)]),
    "eb_recorder_new_deferred": (c_st, [c_vp, ctypes.POINTER(c_vp)]),
    "eb_recorder_submit": (c_st, [c_vp]),
    "eb_recorder_release": (None, [c_vp]),
    "eb_attn_prefill": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size,
                               c_float]),
    "eb_attn_prefill_fast": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size,
                                    c_size, c_float]),
    "eb_attn_prefill_pv16": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size,
                                    c_size, c_float]),
    "eb_launch_attn_prefill_pv16": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                           c_size, c_size, c_size, c_size, c_size, c_float]),
    "eb_launch_attn_prefill_pv16_ws": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                              c_vp, c_size, c_size, c_size, c_size, c_size,
                                              c_float, c_vp, c_size]),
    "eb_launch_attn_prefill_fast": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                           c_size, c_size, c_size, c_size, c_size, c_float]),
    "eb_attn_prefill_fast_workspace_floats": (c_size, [c_size, c_size, c_size, c_size]),
    "eb_launch_attn_prefill_fast_ws": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                              c_vp, c_size, c_size, c_size, c_size, c_size,
                                              c_float, c_vp, c_size]),
    "eb_attn_decode": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size,
                              c_size, c_float]),
    "eb_attn_decode_step": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size,
                                   c_size, c_size, c_size, c_float]),
    "eb_attn_decode_window": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size,
                                     c_size, c_size, c_float, c_size]),
    "eb_attn_decode_step_window": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_size,
                                          c_size, c_size, c_size, c_size, c_float, c_size]),
    "eb_attn_prefill_chunk": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size,
                                     c_size, c_size, c_size, c_float, c_size]),
    "eb_kv_write": (c_st, [c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size, c_size]),
    "eb_rmsnorm": (c_st, [c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_float]),
    "eb_rope": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size, c_size]),
    "eb_launch_kv_write": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_size, c_size, c_size,
                                  c_size, c_size]),
    "eb_launch_attn_prefill": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                      c_size, c_size, c_size, c_size, c_size, c_float]),
    "eb_launch_attn_prefill_chunk": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                            c_vp, c_size, c_size, c_size, c_size, c_size,
                                            c_size, c_size, c_float, c_size]),
    "eb_attn_prefill_workspace_floats": (c_size, [c_size, c_size, c_size, c_size, c_size,
                                                  c_size]),
    "eb_launch_attn_prefill_ws": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                         c_size, c_size, c_size, c_size, c_size, c_float, c_vp,
                                         c_size]),
    "eb_launch_attn_prefill_chunk_ws": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                               c_vp, c_size, c_size, c_size, c_size, c_size,
                                               c_size, c_size, c_float, c_size, c_vp, c_size]),
    "eb_launch_attn_prefill_chunk_f16_ws": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp,
                                                   c_size, c_vp, c_size, c_size, c_size, c_size,
                                                   c_size, c_size, c_size, c_float, c_size, c_vp,
                                                   c_size]),
    "eb_attn_decode_workspace_floats": (c_size, [c_size, c_size, c_size, c_size, c_int]),
    "eb_launch_attn_decode": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                     c_size, c_size, c_size, c_size, c_size, c_size, c_float,
                                     c_vp, c_size, c_int]),
    "eb_launch_attn_decode_window": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                            c_vp, c_size, c_size, c_size, c_size, c_size,
                                            c_size, c_float, c_size, c_vp, c_size, c_int]),
    "eb_launch_attn_decode_step": (c_st, [c_vp, c_vp, c_size, c_vp, c_vp, c_size, c_vp, c_size,
                                          c_vp, c_size, c_vp, c_size, c_size, c_size, c_size,
                                          c_size, c_size, c_float, c_vp, c_size, c_int]),
    "eb_device_begin_capture": (c_st, [c_vp]),
    "eb_device_end_capture": (c_st, [c_vp, ctypes.POINTER(c_vp)]),
    "eb_graph_launch": (c_st, [c_vp]),
    "eb_graph_release": (None, [c_vp]),
    "eb_tensor_write": (c_st, [c_vp, c_vp, c_size]),
    "eb_argmax": (c_st, [c_vp, c_vp, c_vp, c_size]),
    "eb_argmax_workspace_floats": (c_size, [c_size]),
    "eb_launch_argmax": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size]),
    "eb_linear_f16w": (c_st, [c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size]),
    "eb_linear_f16w_multi": (c_st, [c_vp, c_vp, c_size, ctypes.POINTER(c_vp),
                                    ctypes.POINTER(c_vp), ctypes.POINTER(c_size), c_size,
                                    c_size]),
    "eb_linear_workspace_floats": (c_size, [c_size, c_size]),
    "eb_launch_linear_f16w": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_size,
                                     c_size, c_size, c_vp, c_size]),
    "eb_launch_kv_write_f16": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_size, c_size, c_size,
                                      c_size, c_size]),
    "eb_launch_attn_prefill_chunk_f16": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                                c_vp, c_size, c_size, c_size, c_size, c_size,
                                                c_size, c_size, c_float, c_size]),
    "eb_launch_attn_decode_f16": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                         c_size, c_size, c_size, c_size, c_size, c_size, c_float,
                                         c_size, c_vp, c_size, c_int]),
    "eb_launch_attn_decode_step_f16": (c_st, [c_vp, c_vp, c_size, c_vp, c_vp, c_size, c_vp,
                                              c_size, c_vp, c_size, c_vp, c_size, c_size, c_size,
                                              c_size, c_size, c_size, c_float, c_size, c_vp,
                                              c_size, c_int]),
    "eb_launch_kv_write_f8": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_size, c_size, c_size,
                                     c_size, c_size]),
    "eb_launch_attn_prefill_chunk_f8": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size,
                                               c_vp, c_size, c_size, c_size, c_size, c_size,
                                               c_size, c_size, c_float, c_size]),
    "eb_launch_attn_prefill_chunk_f8_ws": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp,
                                                  c_size, c_vp, c_size, c_size, c_size, c_size,
                                                  c_size, c_size, c_size, c_float, c_size, c_vp,
                                                  c_size]),
    "eb_launch_attn_decode_f8": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                        c_size, c_size, c_size, c_size, c_size, c_size, c_float,
                                        c_size, c_vp, c_size, c_int]),
    "eb_launch_attn_decode_step_f8": (c_st, [c_vp, c_vp, c_size, c_vp, c_vp, c_size, c_vp,
                                             c_size, c_vp, c_size, c_vp, c_size, c_size, c_size,
                                             c_size, c_size, c_size, c_float, c_size, c_vp,
                                             c_size, c_int]),
    "eb_launch_rmsnorm": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_size,
                                 c_size, c_float]),
    "eb_launch_rope": (c_st, [c_vp, c_vp, c_size, c_vp, c_vp, c_size, c_vp, c_size, c_size,
                              c_size, c_size, c_size]),
    "eb_launch_selftest_lane_ops": (c_st, [c_vp, c_vp, c_vp]),
    "eb_attn_decode_noalloc_max_floats": (c_size, []),
    "eb_launch_attn_decode_step_noalloc": (c_st, [c_vp, c_vp, c_size, c_vp, c_vp, c_size, c_vp,
                                                  c_size, c_vp, c_size, c_vp, c_size, c_size,
                                                  c_size, c_size, c_size, c_size, c_float,
                                                  c_int]),
    "eb_launch_attn_prologue": (c_st, [c_vp, c_vp, c_size, c_vp, c_size, c_vp, c_size, c_size,
                                       c_size, c_size, c_size, c_vp, c_vp, c_vp, c_float, c_vp,
                                       c_vp, c_size, c_size, c_vp, c_size, c_vp, c_size, c_vp,
                                       c_size, c_size, c_int]),
    "eb_rope_build_partial": (c_st, [c_vp, c_size, c_size, c_size, c_float,
                                     ctypes.POINTER(c_vp)]),
    "eb_rope_tables_release": (None, [c_vp]),
    "eb_rope_tables_cos": (c_vp, [c_vp]),
    "eb_rope_tables_sin": (c_vp, [c_vp]),
    "eb_rope_apply": (c_st, [c_vp, c_vp, c_vp, c_size, c_size, c_size, ctypes.POINTER(c_vp)]),
    "eb_kv_cache_new_per_layer": (c_st, [c_vp, ctypes.POINTER(c_size), c_size, c_size, c_size,
                                         ctypes.POINTER(c_vp)]),
    "eb_kv_cache_new_per_layer_dtype": (c_st, [c_vp, ctypes.POINTER(c_size), c_size, c_size,
                                               c_size, c_int, ctypes.POINTER(c_vp)]),
    "eb_kv_cache_release": (None, [c_vp]),
    "eb_kv_cache_k": (c_vp, [c_vp, c_size]),
    "eb_kv_cache_v": (c_vp, [c_vp, c_size]),
    "eb_kv_cache_max_seq": (c_size, [c_vp]),
    "eb_attention_new": (c_st, [ctypes.POINTER(AttentionDesc), ctypes.POINTER(c_vp)]),
    "eb_attention_release": (None, [c_vp]),
    "eb_attention_forward": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_size, c_size, c_size,
                                    ctypes.POINTER(c_vp)]),
    "eb_attention_forward_qkv": (c_st, [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_vp, c_size,
                                        c_size, c_size, ctypes.POINTER(c_vp)]),
}

_lib = None


def lib():
    """The loaded library (raises if it was never built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(
            f"{LIB_PATH} is missing: build it with `python -m eyebrowse_amd.build` "
            "(there is no fallback implementation)")
    l = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(l, name)
        fn.restype = res
        fn.argtypes = args
    _lib = l
    return l
