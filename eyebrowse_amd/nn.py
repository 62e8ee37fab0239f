"""eyebrowse-nn pieces on the attention path over the C ABI: Rope, KvCache, RmsNorm
weights and the Attention forward between the projections.

Mirrors crates/eyebrowse-nn/src/{rope,kv_cache,attention}.rs. The q/k/v/o projections are
outside this path: ``Attention.forward_qkv`` starts from the projected q, k, v.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Optional

from ._lib import AttentionDesc, c_size, c_vp, lib
from .gpu import DType, Device, Recorder, Tensor, check
from .kernels import linear_f16w


class _Borrowed(Tensor):
    """A tensor owned by another object (rope tables, cache layers): never released here."""

    def __init__(self, handle: int, dev: Device, owner):
        super().__init__(handle, dev)
        self._owner = owner

    def release(self) -> None:
        self._h = c_vp()


class Rope:
    """Rope (crates/eyebrowse-nn/src/rope.rs:10-75): cos/sin tables [max_seq, hd/2]."""

    def __init__(self, handle: int, dev: Device, head_dim: int, max_seq: int):
        self._h = c_vp(handle)
        self.dev = dev
        self.head_dim = head_dim
        self.max_seq = max_seq

    @classmethod
    def build(cls, dev: Device, max_seq: int, head_dim: int, theta: float) -> "Rope":
        return cls.build_partial(dev, max_seq, head_dim, head_dim // 2, theta)

    @classmethod
    def build_partial(cls, dev: Device, max_seq: int, head_dim: int, rope_angles: int,
                      theta: float) -> "Rope":
        out = c_vp()
        check(lib().eb_rope_build_partial(dev.handle, max_seq, head_dim, rope_angles, theta,
                                          ctypes.byref(out)))
        return cls(out.value, dev, head_dim, max_seq)

    @property
    def handle(self):
        return self._h

    @property
    def cos(self) -> Tensor:
        return _Borrowed(lib().eb_rope_tables_cos(self._h), self.dev, self)

    @property
    def sin(self) -> Tensor:
        return _Borrowed(lib().eb_rope_tables_sin(self._h), self.dev, self)

    def apply(self, rec: Recorder, x: Tensor, seq: int, n_heads: int, base_pos: int) -> Tensor:
        out = c_vp()
        check(lib().eb_rope_apply(self._h, rec.handle, x.handle, seq, n_heads, base_pos,
                                  ctypes.byref(out)))
        return Tensor(out.value, self.dev)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().eb_rope_tables_release(h)
            self._h = c_vp()


class Linear:
    """Linear (crates/eyebrowse-nn/src/linear.rs:5-23): bias-free, packed-f16 weight
    [out_f, in_f] (HF layout)."""

    def __init__(self, w: Tensor, in_f: int, out_f: int):
        self.w, self.in_f, self.out_f = w, in_f, out_f

    def forward(self, rec: Recorder, x: Tensor, rows: int) -> Tensor:
        out = Tensor.empty(rec.dev, (rows, self.out_f))
        linear_f16w(rec, x, self.w, out, rows, self.in_f, self.out_f)
        return out


class KvCache:
    """KvCache (crates/eyebrowse-nn/src/kv_cache.rs:9-50): per-layer K/V tensors
    [max_seq, n_kv_heads, head_dims[l]]."""

    def __init__(self, handle: int, dev: Device, n_layers: int, max_seq: int, n_kv_heads: int,
                 dtype: DType = DType.F32):
        self._h = c_vp(handle)
        self.dev = dev
        self.max_seq = max_seq
        self.n_kv_heads = n_kv_heads
        self.dtype = dtype
        self.k = [_Borrowed(lib().eb_kv_cache_k(self._h, l), dev, self) for l in range(n_layers)]
        self.v = [_Borrowed(lib().eb_kv_cache_v(self._h, l), dev, self) for l in range(n_layers)]

    @classmethod
    def new(cls, dev: Device, n_layers: int, max_seq: int, n_kv_heads: int,
            head_dim: int, dtype: DType = DType.F32) -> "KvCache":
        return cls.new_per_layer(dev, [head_dim] * n_layers, max_seq, n_kv_heads, dtype)

    @classmethod
    def new_per_layer(cls, dev: Device, head_dims, max_seq: int, n_kv_heads: int,
                      dtype: DType = DType.F32) -> "KvCache":
        """dtype F32 is the reference's cache; F16 (IEEE half) halves and F8E4M3 (OCP FP8
        E4M3) quarters the cache bytes that decode streams (neither has a counterpart in
        the reference)."""
        arr = (c_size * max(1, len(head_dims)))(*head_dims)
        out = c_vp()
        check(lib().eb_kv_cache_new_per_layer_dtype(dev.handle, arr, len(head_dims), max_seq,
                                                    n_kv_heads, int(dtype), ctypes.byref(out)))
        return cls(out.value, dev, len(head_dims), max_seq, n_kv_heads, DType(dtype))

    @property
    def handle(self):
        return self._h

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().eb_kv_cache_release(h)
            self._h = c_vp()


@dataclass
class Attention:
    """Attention (crates/eyebrowse-nn/src/attention.rs:10-23): head counts, scale, optional
    per-head q/k/v RMSNorm weights ([head_dim] f32 tensors) and, optionally, the four
    packed-f16 projections (all or none) with the model width `hidden`."""
    n_heads: int
    n_kv_heads: int
    head_dim: int
    scale: float
    q_norm: Optional[Tensor] = None
    k_norm: Optional[Tensor] = None
    v_norm: Optional[Tensor] = None
    norm_eps: float = 1e-6
    window: int = 0  # sliding window of a local layer (0: global attention)
    q_proj: Optional[Tensor] = None  # [n_heads*head_dim, hidden]
    k_proj: Optional[Tensor] = None  # [n_kv_heads*head_dim, hidden]
    v_proj: Optional[Tensor] = None
    o_proj: Optional[Tensor] = None  # [hidden, n_heads*head_dim]
    hidden: int = 0

    def __post_init__(self):
        h = lambda t: t.handle if t is not None else None  # noqa: E731
        d = AttentionDesc(self.n_heads, self.n_kv_heads, self.head_dim, self.scale, self.norm_eps,
                          h(self.q_norm), h(self.k_norm), h(self.v_norm), self.window,
                          h(self.q_proj), h(self.k_proj), h(self.v_proj), h(self.o_proj),
                          self.hidden)
        out = c_vp()
        check(lib().eb_attention_new(ctypes.byref(d), ctypes.byref(out)))
        self._h = out

    def forward_qkv(self, rec: Recorder, q: Tensor, k: Tensor, v: Tensor, rope: Rope,
                    kv: KvCache, layer: int, rows: int, base_pos: int) -> Tensor:
        """Attention::forward (attention.rs:30-185) from the projected q [rows, H*hd],
        k/v [rows, Hkv*hd]: norms, RoPE, kv_write, then prefill (base_pos == 0 and
        rows > 1), chunked prefill over the cache (base_pos > 0 and rows > 1) or the fused
        decode step (rows == 1). Returns [rows, H*hd], the o_proj input."""
        out = c_vp()
        check(lib().eb_attention_forward_qkv(self._h, rec.handle, q.handle, k.handle, v.handle,
                                             rope.handle, kv.handle, layer, rows, base_pos,
                                             ctypes.byref(out)))
        return Tensor(out.value, rec.dev)

    def forward(self, rec: Recorder, x: Tensor, rope: Rope, kv: KvCache, layer: int, rows: int,
                base_pos: int) -> Tensor:
        """Attention::forward (attention.rs:30-45) whole: x [rows, hidden] -> [rows, hidden]
        (q/k/v projections in one launch, forward_qkv, o_proj)."""
        out = c_vp()
        check(lib().eb_attention_forward(self._h, rec.handle, x.handle, rope.handle, kv.handle,
                                         layer, rows, base_pos, ctypes.byref(out)))
        return Tensor(out.value, rec.dev)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().eb_attention_release(h)
            self._h = c_vp()
