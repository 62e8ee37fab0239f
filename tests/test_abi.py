"""CPU checks of the C ABI: the library loads, exports every symbol the header declares,
and its host-side validation rejects bad shapes before touching a GPU.

Mirrors the failure paths of the reference that a CPU can force (the reference has no
error channel; these follow crates/eyebrowse-core/src/lib.rs:27-41 for the codes).
"""
import ctypes
import os
import re

import pytest

import eyebrowse_amd as eb
from eyebrowse_amd import _lib
from eyebrowse_amd.gpu import check

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "eyebrowse_hip.h")
HAS_GPU = os.path.exists("/dev/kfd")


def header_functions():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(eb_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_header_symbol():
    lib = ctypes.CDLL(_lib.LIB_PATH)
    names = header_functions()
    assert len(names) >= 40
    missing = [n for n in names if not hasattr(lib, n)]
    assert missing == []


def test_binding_covers_the_header_exactly():
    assert sorted(_lib.SIGNATURES) == header_functions()


def test_status_and_dtype_tables():
    l = eb.lib()
    names = [l.eb_status_name(i).decode() for i in range(7)]
    assert names == ["Ok", "DeviceUnavailable", "Load", "UnsupportedConfig", "ShapeMismatch",
                     "OutOfMemory", "Other"]
    # DType::size (crates/eyebrowse-core/src/lib.rs:14-24 and its test :31-38)
    assert [eb.DType(i).size() for i in range(4)] == [4, 2, 4, 4]
    assert eb.DType.F8E4M3.size() == 1  # the E4M3 cache element (no reference counterpart)
    assert l.eb_pool_max_bytes() == 64 * 1024 * 1024
    assert b"gfx950" in l.eb_version()


@pytest.mark.skipif(HAS_GPU, reason="a GPU is visible")
def test_no_gpu_is_device_unavailable():
    with pytest.raises(eb.DeviceUnavailable):
        eb.Device.new(0)


def _err(fn, *args):
    st = fn(*args)
    return st, eb.lib().eb_last_error().decode()


def test_kv_write_validation():
    l = eb.lib()
    # dst_start + count > max_seq: rejected (the reference writes out of bounds silently)
    st, msg = _err(l.eb_launch_kv_write, None, None, 8 * 2 * 4, None, 2 * 2 * 4, 2, 2, 4, 8, 7)
    assert st == 4 and "max_seq" in msg
    # cache smaller than max_seq * hkv * hd
    st, msg = _err(l.eb_launch_kv_write, None, None, 10, None, 8, 2, 1, 4, 8, 3)
    assert st == 4 and "cache" in msg
    # src smaller than count * hkv * hd
    st, msg = _err(l.eb_launch_kv_write, None, None, 64, None, 7, 2, 1, 4, 8, 3)
    assert st == 4 and "src" in msg
    # null pointers with a valid shape
    st, msg = _err(l.eb_launch_kv_write, None, None, 64, None, 8, 2, 1, 4, 8, 3)
    assert st == 4 and "null" in msg
    # count == 0 is a no-op that never touches the pointers
    assert l.eb_launch_kv_write(None, None, 64, None, 0, 2, 0, 4, 8, 3) == 0


def test_wrapping_shapes_are_refused():
    """Shape products that wrap 64 bits are refused, not checked as their small remainder."""
    l = eb.lib()
    huge = 1 << 62
    # cache: 4 rows x 2^62 heads x 4 dims = 2^66 elements, 0 after wrapping
    st, msg = _err(l.eb_launch_kv_write, None, None, 64, None, 64, huge, 1, 4, 4, 0)
    assert st == 3 and "overflows" in msg
    st, msg = _err(l.eb_launch_attn_prefill, None, None, 64, None, 64, None, 64, None, 64, huge,
                   huge, 4, 8, 0.3)
    assert st == 3 and "overflows" in msg


def test_prefill_validation():
    l = eb.lib()
    st, msg = _err(l.eb_launch_attn_prefill, None, None, 1 << 20, None, 1 << 20, None, 1 << 20,
                   None, 1 << 20, 6, 4, 5, 8, 0.3)
    assert st == 4 and "multiple" in msg          # h % hkv != 0
    st, msg = _err(l.eb_launch_attn_prefill, None, None, 1 << 20, None, 1 << 20, None, 1 << 20,
                   None, 1 << 20, 4, 2, 5, 136, 0.3)
    assert st == 3 and "head_dim" in msg          # unsupported head_dim (not 4, 8k <= 128, 16k)
    st, msg = _err(l.eb_launch_attn_prefill, None, None, 5 * 4 * 8 - 1, None, 1 << 20, None,
                   1 << 20, None, 1 << 20, 4, 2, 5, 8, 0.3)
    assert st == 4 and "q holds" in msg
    st, msg = _err(l.eb_launch_attn_prefill, None, None, 160, None, 80, None, 80, None, 160, 4, 2,
                   5, 8, 0.3)
    assert st == 4 and "null" in msg
    # s == 0 is a no-op
    assert l.eb_launch_attn_prefill(None, None, 0, None, 0, None, 0, None, 0, 4, 2, 0, 8, 0.3) == 0
    # element counts beyond the 32-bit index range are refused
    big = 1 << 32
    st, msg = _err(l.eb_launch_attn_prefill, None, None, big, None, big, None, big, None, big, 16,
                   8, 1 << 20, 256, 0.1)
    assert st == 3 and "2^31" in msg


def test_decode_validation_and_workspace():
    l = eb.lib()
    n = 16 * 8 * 128
    st, msg = _err(l.eb_launch_attn_decode, None, None, 16 * 128, None, n, None, n, None,
                   16 * 128, 16, 8, 16, 128, 16, 0.1, None, 0, 256)
    assert st == 4 and "pos" in msg               # pos >= max_seq
    st, msg = _err(l.eb_launch_attn_decode, None, None, 16 * 128, None, n - 1, None, n, None,
                   16 * 128, 16, 8, 5, 128, 16, 0.1, None, 0, 256)
    assert st == 4 and "kcache" in msg
    # a long cache needs a split workspace; too small a workspace is refused
    ms = 32768
    need = l.eb_attn_decode_workspace_floats(32, 8, ms - 1, 128, 256)
    assert need > 0
    big = ms * 8 * 128
    st, msg = _err(l.eb_launch_attn_decode, None, ctypes.c_void_p(16), 32 * 128,
                   ctypes.c_void_p(16), big, ctypes.c_void_p(16), big, ctypes.c_void_p(16),
                   32 * 128, 32, 8, ms - 1, 128, ms, 0.1, None, need - 1, 256)
    assert st == 4 and "workspace" in msg
    # short caches run as one split with no workspace
    assert l.eb_attn_decode_workspace_floats(4, 2, 5, 8, 256) == 0
    # workspace = nsplit * h * (hd + 2) partial floats (acc, max, sum per split and head)
    w1 = l.eb_attn_decode_workspace_floats(16, 8, 8191, 128, 256)
    w2 = l.eb_attn_decode_workspace_floats(16, 8, 32767, 128, 256)
    assert w1 % (16 * 130) == 0 and w2 % (16 * 130) == 0 and w2 >= w1
    assert l.eb_attn_decode_workspace_floats(6, 4, 5, 8, 256) == 0  # bad heads -> 0


def test_prefill_record_workspace_sizes():
    """One record per (KV head, 32-key tile), copied into LDS with 64-bit addresses (no bound
    on a KV head's records). One KV head, head_dim 128: a pre-split record is the split tile
    image, 64*128 + 64 floats rounded up to whole KiB (8448 floats), an f16-mode record the
    f16 image, 32*128 floats."""
    l = eb.lib()
    rec, frec = 8448, 32 * 128
    # 2^20 keys: 32768 records, 1.1 GB; 2^21 keys: 2.2 GB
    assert l.eb_attn_prefill_workspace_floats(1, 1, 128, 0, 1 << 20, 0) == 32768 * rec
    assert l.eb_attn_prefill_workspace_floats(1, 1, 128, 0, 1 << 21, 0) == 65536 * rec
    assert l.eb_attn_prefill_fast_workspace_floats(1, 1, 128, 1 << 21) == 65536 * frec
    assert l.eb_attn_prefill_fast_workspace_floats(1, 1, 128, 1 << 22) == 131072 * frec


def test_chunk_and_window_validation():
    l = eb.lib()
    # rows [60, 76) past max_seq 70
    st, msg = _err(l.eb_launch_attn_prefill_chunk, None, None, 16 * 4 * 8, None, 1 << 20, None,
                   1 << 20, None, 16 * 4 * 8, 4, 2, 60, 16, 8, 70, 0.3, 0)
    assert st == 4 and "max_seq" in msg
    # unsupported head_dim
    st, msg = _err(l.eb_launch_attn_prefill_chunk, None, None, 1, None, 1, None, 1, None, 1, 4,
                   2, 0, 1, 6, 8, 0.3, 0)
    assert st == 3 and "head_dim" in msg
    # zero rows is a no-op
    assert l.eb_launch_attn_prefill_chunk(None, None, 0, None, 64, None, 64, None, 0, 4, 2, 3,
                                          0, 8, 4, 0.3, 0) == 0
    # windowed decode checks like decode
    st, msg = _err(l.eb_launch_attn_decode_window, None, None, 16 * 128, None, 16 * 8 * 128,
                   None, 16 * 8 * 128, None, 16 * 128, 16, 8, 16, 128, 16, 0.1, 4, None, 0, 256)
    assert st == 4 and "pos" in msg


def test_rmsnorm_rope_validation():
    l = eb.lib()
    st, msg = _err(l.eb_launch_rmsnorm, None, None, 30, None, 9, None, 30, 3, 10, 1e-6)
    assert st == 4 and "weight" in msg
    st, msg = _err(l.eb_launch_rope, None, None, 64, None, None, 16, None, 64, 4, 2, 7, 0)
    assert st == 4 and "even" in msg
    # tables must cover rows base_pos .. base_pos + seq
    st, msg = _err(l.eb_launch_rope, None, None, 64, None, None, 4 * 4 + 3, None, 64, 4, 2, 8, 1)
    assert st == 4 and "tables" in msg


def test_errors_map_to_exception_types():
    with pytest.raises(eb.ShapeMismatch):
        check(eb.lib().eb_launch_kv_write(None, None, 8, None, 8, 1, 2, 4, 1, 0))
    with pytest.raises(eb.UnsupportedConfig):
        check(eb.lib().eb_launch_attn_prefill(None, None, 1, None, 1, None, 1, None, 1, 1, 1, 1,
                                              6, 1.0))
