"""CPU oracle for the attention hot path — TEST INFRASTRUCTURE ONLY.

ctypes bindings over ``oracle/liboracle.so`` (built from ``oracle/oracle.c`` by
``oracle/Makefile``). The C code restates the reference's Rust CPU attention
(``crates/eyebrowse-kernels/src/testutil.rs:130-218``) and its helpers; this module
only marshals numpy arrays. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it: the product library never does.

Every function is pinned by an independent check in ``tests/test_oracle.py``
(float64 textbook attention, closed forms, invariants, the reference's own
known-answer cases).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_f32p = ctypes.POINTER(ctypes.c_float)
_sz = ctypes.c_size_t


def build() -> None:
    """Compile the oracle with its Makefile (gcc, -O2 -ffp-contract=off)."""
    subprocess.run(["make", "-s", "-C", _HERE], check=True)


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_LIB_PATH):
        build()
    lib = ctypes.CDLL(_LIB_PATH)
    lib.ebo_rel_l2.restype = ctypes.c_float
    lib.ebo_rel_l2.argtypes = [_f32p, _f32p, _sz]
    lib.ebo_prng.restype = None
    lib.ebo_prng.argtypes = [_f32p, _sz, ctypes.c_uint64]
    lib.ebo_randn.restype = None
    lib.ebo_randn.argtypes = [_f32p, _sz, ctypes.c_uint64]
    lib.ebo_rmsnorm.restype = None
    lib.ebo_rmsnorm.argtypes = [_f32p, _f32p, _f32p, _sz, _sz, ctypes.c_float]
    lib.ebo_rope_tables.restype = None
    lib.ebo_rope_tables.argtypes = [_f32p, _f32p, _sz, _sz, _sz, ctypes.c_float]
    lib.ebo_rope.restype = None
    lib.ebo_rope.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz]
    lib.ebo_kv_write.restype = None
    lib.ebo_kv_write.argtypes = [_f32p, _f32p, _sz, _sz, _sz, _sz]
    lib.ebo_attn_prefill_rows.restype = ctypes.c_int
    lib.ebo_attn_prefill_rows.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz,
                                          ctypes.c_float, _sz, _sz, ctypes.c_int]
    lib.ebo_attn_chunk.restype = ctypes.c_int
    lib.ebo_attn_chunk.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz,
                                   ctypes.c_float, _sz, ctypes.c_int]
    lib.ebo_attn_decode.restype = ctypes.c_int
    lib.ebo_attn_decode.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz,
                                    ctypes.c_float, ctypes.c_int]
    lib.ebo_linear_f16w.restype = None
    lib.ebo_linear_f16w.argtypes = [_f32p, ctypes.POINTER(ctypes.c_uint16), _f32p, _sz, _sz, _sz,
                                    ctypes.c_int]
    lib.ebo_f16_to_f32.restype = ctypes.c_float
    lib.ebo_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.ebo_f8e4m3_bits_n.restype = None
    lib.ebo_f8e4m3_bits_n.argtypes = [_f32p, ctypes.POINTER(ctypes.c_uint8), _sz]
    lib.ebo_f8e4m3_to_f32_n.restype = None
    lib.ebo_f8e4m3_to_f32_n.argtypes = [ctypes.POINTER(ctypes.c_uint8), _f32p, _sz]
    lib.ebo_argmax.restype = ctypes.c_uint32
    lib.ebo_argmax.argtypes = [_f32p, _sz]
    lib.ebo_default_scale.restype = ctypes.c_float
    lib.ebo_default_scale.argtypes = [_sz]
    lib.ebo_max_threads.restype = ctypes.c_int
    lib.ebo_max_threads.argtypes = []
    _lib = lib
    return lib


def _p(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags["C_CONTIGUOUS"], "oracle wants contiguous f32"
    return a.ctypes.data_as(_f32p)


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def rel_l2(a, b) -> float:
    """||a-b|| / (||b|| + 1e-12) in f64 (testutil.rs:16-26)."""
    a, b = _f32(a).ravel(), _f32(b).ravel()
    assert a.size == b.size, "rel_l2 length mismatch"
    return float(_load().ebo_rel_l2(_p(a), _p(b), a.size))


def prng(n: int, seed: int) -> np.ndarray:
    """Reference xorshift stream in [-1, 1) (nn/src/testutil.rs:30-41)."""
    out = np.empty(n, np.float32)
    _load().ebo_prng(_p(out), n, seed)
    return out


def randn(shape, seed: int) -> np.ndarray:
    """Seeded N(0,1) f32: xorshift64 uniforms + Box-Muller in f64."""
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    _load().ebo_randn(_p(out), n, seed)
    return out.reshape(shape)


def default_scale(hd: int) -> float:
    """1.0 / (hd as f32).sqrt() (testutil.rs:140)."""
    return float(_load().ebo_default_scale(hd))


def max_threads() -> int:
    return int(_load().ebo_max_threads())


def rmsnorm(x, w, rows: int, dim: int, eps: float) -> np.ndarray:
    """testutil.rs:83-97."""
    x, w = _f32(x).ravel(), _f32(w).ravel()
    assert x.size == rows * dim and w.size == dim
    out = np.empty_like(x)
    _load().ebo_rmsnorm(_p(x), _p(w), _p(out), rows, dim, eps)
    return out


def rope_tables(max_seq: int, hd: int, theta: float, rope_angles: int | None = None):
    """Rope::build / build_partial tables (nn/src/rope.rs:24-50); returns (cos, sin)."""
    half = hd // 2
    ra = half if rope_angles is None else rope_angles
    c = np.empty(max_seq * half, np.float32)
    s = np.empty(max_seq * half, np.float32)
    _load().ebo_rope_tables(_p(c), _p(s), max_seq, hd, ra, theta)
    return c.reshape(max_seq, half), s.reshape(max_seq, half)


def rope(x, cos, sin, seq: int, n_heads: int, hd: int, base_pos: int = 0) -> np.ndarray:
    """testutil.rs:101-125 with the kernel's base_pos row offset (rope.rs:25-26)."""
    x, cos, sin = _f32(x).ravel(), _f32(cos).ravel(), _f32(sin).ravel()
    assert x.size == seq * n_heads * hd
    assert cos.size >= (seq + base_pos) * (hd // 2) and sin.size == cos.size
    out = np.empty_like(x)
    _load().ebo_rope(_p(x), _p(cos), _p(sin), _p(out), seq, n_heads, hd, base_pos)
    return out


def kv_write(cache, src, hkv: int, count: int, hd: int, dst_start: int) -> np.ndarray:
    """ops.rs:70-87 semantics; returns a new cache array."""
    cache = _f32(cache).ravel().copy()
    src = _f32(src).ravel()
    assert src.size >= count * hkv * hd
    assert cache.size >= (dst_start + count) * hkv * hd
    _load().ebo_kv_write(_p(cache), _p(src), hkv, count, hd, dst_start)
    return cache


def attn_prefill(q, k, v, h: int, hkv: int, s: int, hd: int, scale: float | None = None,
                 rows: tuple[int, int] | None = None, threads: int = 1) -> np.ndarray:
    """Causal GQA prefill (testutil.rs:130-172). ``rows=(row0, n)`` computes only those
    query rows (other rows of the result are NaN). Returns o [s, h, hd]."""
    q, k, v = _f32(q).ravel(), _f32(k).ravel(), _f32(v).ravel()
    assert q.size == s * h * hd and k.size == s * hkv * hd and v.size == k.size
    if scale is None:
        scale = default_scale(hd)
    row0, n = (0, s) if rows is None else rows
    o = np.full(s * h * hd, np.nan, np.float32)
    rc = _load().ebo_attn_prefill_rows(_p(q), _p(k), _p(v), _p(o), h, hkv, s, hd, scale,
                                       row0, n, threads)
    if rc != 0:
        raise ValueError("oracle attn_prefill: bad shape")
    return o.reshape(s, h, hd)


def attn_decode(q, kc, vc, h: int, hkv: int, pos: int, hd: int, max_seq: int,
                scale: float | None = None, threads: int = 1) -> np.ndarray:
    """Single decode step over keys 0..=pos (testutil.rs:177-218). Returns o [h, hd]."""
    q, kc, vc = _f32(q).ravel(), _f32(kc).ravel(), _f32(vc).ravel()
    assert q.size == h * hd and kc.size >= (pos + 1) * hkv * hd and vc.size == kc.size
    if scale is None:
        scale = default_scale(hd)
    o = np.empty(h * hd, np.float32)
    rc = _load().ebo_attn_decode(_p(q), _p(kc), _p(vc), _p(o), h, hkv, pos, hd, max_seq,
                                 scale, threads)
    if rc != 0:
        raise ValueError("oracle attn_decode: bad shape")
    return o.reshape(h, hd)


def attn_chunk(q, k, v, h: int, hkv: int, pos0: int, rows: int, hd: int,
               scale: float | None = None, window: int = 0, threads: int = 1) -> np.ndarray:
    """Chunked causal attention with an optional sliding window: row r of q [rows, h, hd]
    at position pos0 + r attends keys max(0, p - window + 1)..=p (window 0: all of 0..=p)
    of k/v [>= pos0 + rows, hkv, hd]. Same per-row arithmetic as attn_prefill /
    attn_decode (testutil.rs:142-169); the reference has no chunked or windowed attention.
    Returns o [rows, h, hd]."""
    q, k, v = _f32(q).ravel(), _f32(k).ravel(), _f32(v).ravel()
    assert q.size == rows * h * hd and k.size >= (pos0 + rows) * hkv * hd and v.size == k.size
    if scale is None:
        scale = default_scale(hd)
    o = np.empty(rows * h * hd, np.float32)
    rc = _load().ebo_attn_chunk(_p(q), _p(k), _p(v), _p(o), h, hkv, pos0, rows, hd, scale,
                                window, threads)
    if rc != 0:
        raise ValueError("oracle attn_chunk: bad shape")
    return o.reshape(rows, h, hd)


def f16_bits(x) -> np.ndarray:
    """IEEE 754 binary16 bit patterns of f32 values, rounded to nearest even (overflow to
    +-inf, gradual underflow to subnormals, NaN stays NaN): numpy's float32 -> float16
    conversion. The f16 KV cache stores these; the reference's caches are f32 only."""
    with np.errstate(over="ignore"):
        return np.ascontiguousarray(_f32(x)).astype(np.float16).view(np.uint16)


def f16_values(bits) -> np.ndarray:
    """f32 values of binary16 bit patterns (exact: every half is an f32)."""
    return np.ascontiguousarray(bits, np.uint16).view(np.float16).astype(np.float32)


def kv_write_f16(cache_bits, src, hkv: int, count: int, hd: int, dst_start: int) -> np.ndarray:
    """kv_write (ops.rs:70-87 row placement) into a binary16 cache: rows dst_start..
    dst_start+count of cache_bits [uint16] take f16_bits of src. Returns a new array."""
    cache = np.ascontiguousarray(cache_bits, np.uint16).ravel().copy()
    src = _f32(src).ravel()
    n = count * hkv * hd
    assert src.size >= n and cache.size >= (dst_start + count) * hkv * hd
    cache[dst_start * hkv * hd:dst_start * hkv * hd + n] = f16_bits(src[:n])
    return cache


def f8_bits(x) -> np.ndarray:
    """OCP FP8 E4M3 (e4m3fn) bit patterns of f32 values, the FP8 cache's kv_write contract:
    nearest value, ties to even; finite values at or beyond 448 saturate to +-448; inf and
    NaN become NaN (0x7F | sign). The reference's caches are f32 only."""
    x = np.ascontiguousarray(_f32(x)).ravel()
    out = np.empty(x.size, np.uint8)
    _load().ebo_f8e4m3_bits_n(_p(x), out.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), x.size)
    return out


def f8_values(bits) -> np.ndarray:
    """f32 values of E4M3 bit patterns (exact)."""
    b = np.ascontiguousarray(bits, np.uint8).ravel()
    out = np.empty(b.size, np.float32)
    _load().ebo_f8e4m3_to_f32_n(b.ctypes.data_as(ctypes.POINTER(ctypes.c_uint8)), _p(out), b.size)
    return out


def kv_write_f8(cache_bits, src, hkv: int, count: int, hd: int, dst_start: int) -> np.ndarray:
    """kv_write (ops.rs:70-87 row placement) into an E4M3 cache: rows dst_start..
    dst_start+count of cache_bits [uint8] take f8_bits of src. Returns a new array."""
    cache = np.ascontiguousarray(cache_bits, np.uint8).ravel().copy()
    src = _f32(src).ravel()
    n = count * hkv * hd
    assert src.size >= n and cache.size >= (dst_start + count) * hkv * hd
    cache[dst_start * hkv * hd:dst_start * hkv * hd + n] = f8_bits(src[:n])
    return cache


def linear_f16w(x, w_bits, m: int, in_f: int, out_f: int, threads: int = 1) -> np.ndarray:
    """linear_f16w (testutil.rs:68-80 on f16-rounded weights): y [m, out_f] = x [m, in_f]
    times w^T, w the f16 bit patterns of [out_f, in_f] (flat)."""
    x = _f32(x).ravel()
    w = np.ascontiguousarray(w_bits, np.uint16).ravel()
    assert x.size == m * in_f and w.size >= out_f * in_f
    y = np.empty(m * out_f, np.float32)
    _load().ebo_linear_f16w(_p(x), w.ctypes.data_as(ctypes.POINTER(ctypes.c_uint16)), _p(y), m,
                            in_f, out_f, threads)
    return y.reshape(m, out_f)


def pack_f16(x) -> np.ndarray:
    """The reference's packed-u32 weight format (crates/eyebrowse-gpu/src/tensor.rs:7-23):
    u32[w] = bits(f16(x[2w])) | bits(f16(x[2w+1])) << 16, odd tail zero-padded."""
    b = f16_bits(np.ravel(x))
    if b.size % 2:
        b = np.concatenate([b, np.zeros(1, np.uint16)])
    return b[0::2].astype(np.uint32) | (b[1::2].astype(np.uint32) << 16)


def argmax(x) -> int:
    """argmax (sampling.rs:6-38), the reference's 256-lane scan and tree: the maximum;
    ties to the lane (index mod 256) first in bit-reversed order, then the smallest index;
    NaN and values <= -3e38 never win (0 if nothing does)."""
    x = _f32(x).ravel()
    return int(_load().ebo_argmax(_p(x), x.size))
