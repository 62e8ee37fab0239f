"""eyebrowse_amd: the eyebrowse attention hot path (prefill, decode, kv-write) on MI355X.

The compute lives in ``libeyebrowse_hip.so`` (hand-written gfx950 HIP kernels behind the C
ABI in ``include/eyebrowse_hip.h``); this package is a thin ctypes mirror of the
reference's Rust interface:

- ``gpu``: DType, EyebrowseError, Device, Tensor, Recorder (crates/eyebrowse-gpu);
- ``kernels``: attn_prefill, attn_decode, kv_write, rmsnorm, rope (crates/eyebrowse-kernels),
  linear_f16w (the projections around attention), plus chunked / windowed attention, the
  fused decode step and IEEE-half and OCP FP8 E4M3 caches;
- ``nn``: Linear, Rope, KvCache, Attention (crates/eyebrowse-nn).
"""
from ._lib import LIB_PATH, lib
from .gpu import (DType, Device, DeviceUnavailable, EyebrowseError, Graph, LoadError,
                  OutOfMemory, Recorder, ShapeMismatch, Tensor, UnsupportedConfig)
from .kernels import (argmax, argmax_workspace_floats, attn_decode, attn_decode_step,
                      attn_decode_step_window, attn_decode_window, attn_decode_workspace_floats,
                      attn_prefill, attn_prefill_chunk, attn_prefill_fast,
                      attn_prefill_workspace_floats, launch_attn_prefill_fast,
                      attn_prefill_fast_workspace_floats, launch_attn_prefill_fast_ws,
                      kv_write, launch_argmax,
                      launch_attn_decode, launch_attn_decode_f16, launch_attn_decode_step,
                      launch_attn_decode_step_f16, launch_attn_decode_window,
                      launch_attn_prefill, launch_attn_prefill_chunk,
                      launch_attn_prefill_chunk_f16, launch_attn_prefill_chunk_ws,
                      launch_attn_prefill_ws, launch_kv_write, launch_kv_write_f16,
                      launch_attn_prologue, launch_attn_decode_step_noalloc,
                      launch_kv_write_f8, launch_attn_prefill_chunk_f8, launch_attn_decode_f8,
                      launch_attn_decode_step_f8,
                      attn_decode_noalloc_max_floats, launch_linear_f16w, launch_rmsnorm, launch_rope, linear_f16w,
                      linear_f16w_multi, linear_workspace_floats, rmsnorm, rope,
                      LANE_OPS_ROWS, launch_selftest_lane_ops, attn_prefill_pv16,
                      launch_attn_prefill_pv16, launch_attn_prefill_pv16_ws)
from .nn import Attention, KvCache, Linear, Rope

__all__ = [
    "LIB_PATH", "lib", "DType", "Device", "DeviceUnavailable", "EyebrowseError", "Graph",
    "LoadError", "argmax", "argmax_workspace_floats", "launch_argmax",
    "OutOfMemory", "Recorder", "ShapeMismatch", "Tensor", "UnsupportedConfig", "attn_decode",
    "attn_decode_step", "attn_decode_step_window", "attn_decode_window",
    "attn_decode_workspace_floats", "attn_prefill", "attn_prefill_chunk", "kv_write",
    "attn_prefill_fast", "launch_attn_prefill_fast", "attn_prefill_fast_workspace_floats",
    "launch_attn_prefill_fast_ws",
    "launch_attn_decode", "launch_attn_decode_f16", "launch_attn_decode_step",
    "launch_attn_decode_step_f16", "launch_attn_decode_window", "launch_attn_prefill",
    "launch_attn_prefill_chunk", "launch_attn_prefill_chunk_f16", "launch_attn_prefill_chunk_ws",
    "launch_attn_prefill_ws", "attn_prefill_workspace_floats", "launch_kv_write",
    "launch_kv_write_f16", "launch_kv_write_f8", "launch_attn_prefill_chunk_f8",
    "launch_attn_decode_f8", "launch_attn_decode_step_f8", "launch_linear_f16w", "linear_f16w", "linear_f16w_multi",
    "linear_workspace_floats", "launch_rmsnorm",
    "launch_rope", "launch_attn_prologue", "launch_attn_decode_step_noalloc",
    "attn_decode_noalloc_max_floats", "rmsnorm", "rope", "Attention", "KvCache", "Linear", "Rope",
    "LANE_OPS_ROWS", "launch_selftest_lane_ops", "attn_prefill_pv16", "launch_attn_prefill_pv16",
    "launch_attn_prefill_pv16_ws",
]
