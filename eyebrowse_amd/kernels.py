"""eyebrowse-kernels entry points over the C ABI (same names and argument order as
crates/eyebrowse-kernels/src/{attention,ops,rmsnorm,rope}.rs), plus the raw launches on
caller-owned device memory.
"""
from __future__ import annotations

from ._lib import c_size, c_vp, lib
from .gpu import Recorder, Tensor, check


def attn_prefill(rec: Recorder, q: Tensor, k: Tensor, v: Tensor, o: Tensor, h: int, hkv: int,
                 s: int, hd: int, scale: float) -> None:
    """attention.rs:94-120: causal GQA prefill, q [s,h,hd], k/v [s,hkv,hd] -> o [s,h,hd]."""
    check(lib().eb_attn_prefill(rec.handle, q.handle, k.handle, v.handle, o.handle, h, hkv, s,
                                hd, scale))


def attn_prefill_fast(rec: Recorder, q: Tensor, k: Tensor, v: Tensor, o: Tensor, h: int,
                      hkv: int, s: int, hd: int, scale: float) -> None:
    """attn_prefill in the opt-in f16 mode: one f16 matrix-core product per product (q, K,
    V, P rounded to f16 once), f32 softmax and accumulation; |scale| <= 1/sqrt(hd)."""
    check(lib().eb_attn_prefill_fast(rec.handle, q.handle, k.handle, v.handle, o.handle, h, hkv,
                                     s, hd, scale))


def attn_prefill_pv16(rec: Recorder, q: Tensor, k: Tensor, v: Tensor, o: Tensor, h: int,
                      hkv: int, s: int, hd: int, scale: float) -> None:
    """attn_prefill in the opt-in scores-accurate mode: scores as attn_prefill computes them,
    O += P V as one f16 product (max-abs within 2^-11 of the largest |V|)."""
    check(lib().eb_attn_prefill_pv16(rec.handle, q.handle, k.handle, v.handle, o.handle, h, hkv,
                                     s, hd, scale))


def attn_decode(rec: Recorder, q: Tensor, kcache: Tensor, vcache: Tensor, o: Tensor, h: int,
                hkv: int, pos: int, hd: int, max_seq: int, scale: float) -> None:
    """attention.rs:124-162: q [h,hd] attends keys 0..=pos of [max_seq,hkv,hd] caches."""
    check(lib().eb_attn_decode(rec.handle, q.handle, kcache.handle, vcache.handle, o.handle, h,
                               hkv, pos, hd, max_seq, scale))


def attn_decode_step(rec: Recorder, q: Tensor, knew: Tensor, vnew: Tensor, kcache: Tensor,
                     vcache: Tensor, o: Tensor, h: int, hkv: int, pos: int, hd: int,
                     max_seq: int, scale: float) -> None:
    """kv_write(K), kv_write(V), attn_decode of Attention::decode
    (crates/eyebrowse-nn/src/attention.rs:149-183) in one launch."""
    check(lib().eb_attn_decode_step(rec.handle, q.handle, knew.handle, vnew.handle,
                                    kcache.handle, vcache.handle, o.handle, h, hkv, pos, hd,
                                    max_seq, scale))


def attn_decode_window(rec: Recorder, q: Tensor, kcache: Tensor, vcache: Tensor, o: Tensor,
                       h: int, hkv: int, pos: int, hd: int, max_seq: int, scale: float,
                       window: int) -> None:
    """attn_decode over keys pos - window + 1..=pos only (window 0: all keys)."""
    check(lib().eb_attn_decode_window(rec.handle, q.handle, kcache.handle, vcache.handle,
                                      o.handle, h, hkv, pos, hd, max_seq, scale, window))


def attn_decode_step_window(rec: Recorder, q: Tensor, knew: Tensor, vnew: Tensor,
                            kcache: Tensor, vcache: Tensor, o: Tensor, h: int, hkv: int,
                            pos: int, hd: int, max_seq: int, scale: float, window: int) -> None:
    """attn_decode_step over keys pos - window + 1..=pos only (window 0: all keys)."""
    check(lib().eb_attn_decode_step_window(rec.handle, q.handle, knew.handle, vnew.handle,
                                           kcache.handle, vcache.handle, o.handle, h, hkv, pos,
                                           hd, max_seq, scale, window))


def attn_prefill_chunk(rec: Recorder, q: Tensor, kcache: Tensor, vcache: Tensor, o: Tensor,
                       h: int, hkv: int, pos0: int, rows: int, hd: int, max_seq: int,
                       scale: float, window: int = 0) -> None:
    """Chunked causal prefill: q [rows,h,hd] at positions pos0.. attends the cache keys
    0..=pos0+r (or the last `window`) of [max_seq,hkv,hd] caches that already hold them."""
    check(lib().eb_attn_prefill_chunk(rec.handle, q.handle, kcache.handle, vcache.handle,
                                      o.handle, h, hkv, pos0, rows, hd, max_seq, scale, window))


def kv_write(rec: Recorder, cache: Tensor, src: Tensor, hkv: int, count: int, hd: int,
             max_seq: int, dst_start: int) -> None:
    """ops.rs:150-179: copy src [count,hkv,hd] into cache rows dst_start.."""
    check(lib().eb_kv_write(rec.handle, cache.handle, src.handle, hkv, count, hd, max_seq,
                            dst_start))


def rmsnorm(rec: Recorder, x: Tensor, weight: Tensor, out: Tensor, rows: int, dim: int,
            eps: float) -> None:
    """rmsnorm.rs:42-64."""
    check(lib().eb_rmsnorm(rec.handle, x.handle, weight.handle, out.handle, rows, dim, eps))


def rope(rec: Recorder, x: Tensor, cos: Tensor, sin: Tensor, out: Tensor, seq: int,
         n_heads: int, head_dim: int, base_pos: int) -> None:
    """rope.rs:38-69."""
    check(lib().eb_rope(rec.handle, x.handle, cos.handle, sin.handle, out.handle, seq, n_heads,
                        head_dim, base_pos))


def linear_f16w(rec: Recorder, a: Tensor, w: Tensor, c: Tensor, m: int, in_f: int,
                out_f: int) -> None:
    """linear_f16w (crates/eyebrowse-kernels/src/matmul.rs:120-140): c = a . w^T, w the
    packed-f16 [out_f, in_f] weight (a U32 tensor of packed words, or an F16 tensor)."""
    check(lib().eb_linear_f16w(rec.handle, a.handle, w.handle, c.handle, m, in_f, out_f))


def linear_f16w_multi(rec: Recorder, a: Tensor, ws, cs, out_fs, m: int, in_f: int) -> None:
    """Up to three projections of the same a in one launch (no counterpart in the
    reference): cs[i] = a . ws[i]^T."""
    n = len(ws)
    assert len(cs) == n and len(out_fs) == n
    warr = (c_vp * max(n, 1))(*[t.handle for t in ws])
    carr = (c_vp * max(n, 1))(*[t.handle for t in cs])
    oarr = (c_size * max(n, 1))(*out_fs)
    check(lib().eb_linear_f16w_multi(rec.handle, a.handle, n, warr, carr, oarr, m, in_f))


def linear_workspace_floats(m: int, in_f: int) -> int:
    return int(lib().eb_linear_workspace_floats(m, in_f))


def argmax(rec: Recorder, logits: Tensor, out_idx: Tensor, vocab: int) -> None:
    """argmax (crates/eyebrowse-kernels/src/sampling.rs:42-53): out_idx[0] = index of the
    largest logit, with the reference's tie order."""
    check(lib().eb_argmax(rec.handle, logits.handle, out_idx.handle, vocab))


def argmax_workspace_floats(vocab: int) -> int:
    return int(lib().eb_argmax_workspace_floats(vocab))


# ---- raw launches on caller memory (stream and pointers as ints) ------------------------

def launch_argmax(stream: int, logits: int, logits_numel: int, out_idx: int, vocab: int,
                  workspace: int, workspace_floats: int) -> None:
    check(lib().eb_launch_argmax(stream, logits, logits_numel, out_idx, vocab, workspace,
                                 workspace_floats))


def launch_linear_f16w(stream: int, a: int, a_numel: int, w: int, w_halves: int, c: int,
                       c_numel: int, m: int, in_f: int, out_f: int, workspace: int,
                       workspace_floats: int) -> None:
    check(lib().eb_launch_linear_f16w(stream, a, a_numel, w, w_halves, c, c_numel, m, in_f,
                                      out_f, workspace, workspace_floats))



def launch_kv_write(stream: int, cache: int, cache_numel: int, src: int, src_numel: int,
                    hkv: int, count: int, hd: int, max_seq: int, dst_start: int) -> None:
    check(lib().eb_launch_kv_write(stream, cache, cache_numel, src, src_numel, hkv, count, hd,
                                   max_seq, dst_start))


def launch_attn_prefill(stream: int, q: int, q_numel: int, k: int, k_numel: int, v: int,
                        v_numel: int, o: int, o_numel: int, h: int, hkv: int, s: int, hd: int,
                        scale: float) -> None:
    check(lib().eb_launch_attn_prefill(stream, q, q_numel, k, k_numel, v, v_numel, o, o_numel,
                                       h, hkv, s, hd, scale))


def launch_attn_prefill_fast(stream: int, q: int, q_numel: int, k: int, k_numel: int, v: int,
                             v_numel: int, o: int, o_numel: int, h: int, hkv: int, s: int,
                             hd: int, scale: float) -> None:
    check(lib().eb_launch_attn_prefill_fast(stream, q, q_numel, k, k_numel, v, v_numel, o,
                                            o_numel, h, hkv, s, hd, scale))


def launch_attn_prefill_pv16(stream: int, q: int, q_numel: int, k: int, k_numel: int, v: int,
                             v_numel: int, o: int, o_numel: int, h: int, hkv: int, s: int,
                             hd: int, scale: float) -> None:
    check(lib().eb_launch_attn_prefill_pv16(stream, q, q_numel, k, k_numel, v, v_numel, o,
                                            o_numel, h, hkv, s, hd, scale))


def launch_attn_prefill_pv16_ws(stream: int, q: int, q_numel: int, k: int, k_numel: int, v: int,
                                v_numel: int, o: int, o_numel: int, h: int, hkv: int, s: int,
                                hd: int, scale: float, workspace: int,
                                workspace_floats: int) -> None:
    check(lib().eb_launch_attn_prefill_pv16_ws(stream, q, q_numel, k, k_numel, v, v_numel, o,
                                               o_numel, h, hkv, s, hd, scale, workspace,
                                               workspace_floats))


def attn_prefill_fast_workspace_floats(h: int, hkv: int, hd: int, s: int) -> int:
    return int(lib().eb_attn_prefill_fast_workspace_floats(h, hkv, hd, s))


def launch_attn_prefill_fast_ws(stream: int, q: int, q_numel: int, k: int, k_numel: int, v: int,
                                v_numel: int, o: int, o_numel: int, h: int, hkv: int, s: int,
                                hd: int, scale: float, workspace: int,
                                workspace_floats: int) -> None:
    check(lib().eb_launch_attn_prefill_fast_ws(stream, q, q_numel, k, k_numel, v, v_numel, o,
                                               o_numel, h, hkv, s, hd, scale, workspace,
                                               workspace_floats))


def attn_prefill_workspace_floats(h: int, hkv: int, hd: int, pos0: int, rows: int,
                                  window: int = 0) -> int:
    """Floats of workspace the _ws prefill launches need for this shape (0: none)."""
    return int(lib().eb_attn_prefill_workspace_floats(h, hkv, hd, pos0, rows, window))


def launch_attn_prefill_ws(stream: int, q: int, q_numel: int, k: int, k_numel: int, v: int,
                           v_numel: int, o: int, o_numel: int, h: int, hkv: int, s: int, hd: int,
                           scale: float, ws: int, ws_floats: int) -> None:
    check(lib().eb_launch_attn_prefill_ws(stream, q, q_numel, k, k_numel, v, v_numel, o,
                                          o_numel, h, hkv, s, hd, scale, ws, ws_floats))


def launch_attn_prefill_chunk_ws(stream: int, q: int, q_numel: int, kc: int, kc_numel: int,
                                 vc: int, vc_numel: int, o: int, o_numel: int, h: int, hkv: int,
                                 pos0: int, rows: int, hd: int, max_seq: int, scale: float,
                                 window: int, ws: int, ws_floats: int, f16: bool = False,
                                 f8: bool = False) -> None:
    fn = (lib().eb_launch_attn_prefill_chunk_f8_ws if f8 else
          lib().eb_launch_attn_prefill_chunk_f16_ws if f16 else
          lib().eb_launch_attn_prefill_chunk_ws)
    check(fn(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o, o_numel, h, hkv, pos0, rows, hd,
             max_seq, scale, window, ws, ws_floats))


def launch_attn_prefill_chunk(stream: int, q: int, q_numel: int, kc: int, kc_numel: int,
                              vc: int, vc_numel: int, o: int, o_numel: int, h: int, hkv: int,
                              pos0: int, rows: int, hd: int, max_seq: int, scale: float,
                              window: int = 0) -> None:
    check(lib().eb_launch_attn_prefill_chunk(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                             o_numel, h, hkv, pos0, rows, hd, max_seq, scale,
                                             window))


def attn_decode_workspace_floats(h: int, hkv: int, pos: int, hd: int, cu_count: int) -> int:
    return int(lib().eb_attn_decode_workspace_floats(h, hkv, pos, hd, cu_count))


def launch_attn_decode(stream: int, q: int, q_numel: int, kc: int, kc_numel: int, vc: int,
                       vc_numel: int, o: int, o_numel: int, h: int, hkv: int, pos: int, hd: int,
                       max_seq: int, scale: float, workspace: int, workspace_floats: int,
                       cu_count: int) -> None:
    check(lib().eb_launch_attn_decode(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                      o_numel, h, hkv, pos, hd, max_seq, scale, workspace,
                                      workspace_floats, cu_count))


def launch_attn_decode_window(stream: int, q: int, q_numel: int, kc: int, kc_numel: int,
                              vc: int, vc_numel: int, o: int, o_numel: int, h: int, hkv: int,
                              pos: int, hd: int, max_seq: int, scale: float, window: int,
                              workspace: int, workspace_floats: int, cu_count: int) -> None:
    check(lib().eb_launch_attn_decode_window(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                             o_numel, h, hkv, pos, hd, max_seq, scale, window,
                                             workspace, workspace_floats, cu_count))


def launch_attn_decode_step(stream: int, q: int, q_numel: int, knew: int, vnew: int,
                            new_numel: int, kc: int, kc_numel: int, vc: int, vc_numel: int,
                            o: int, o_numel: int, h: int, hkv: int, pos: int, hd: int,
                            max_seq: int, scale: float, workspace: int, workspace_floats: int,
                            cu_count: int) -> None:
    check(lib().eb_launch_attn_decode_step(stream, q, q_numel, knew, vnew, new_numel, kc,
                                           kc_numel, vc, vc_numel, o, o_numel, h, hkv, pos, hd,
                                           max_seq, scale, workspace, workspace_floats,
                                           cu_count))


# ---- raw launches over IEEE-half caches (no counterpart in the reference) --------------

def launch_kv_write_f16(stream: int, cache: int, cache_numel: int, src: int, src_numel: int,
                        hkv: int, count: int, hd: int, max_seq: int, dst_start: int) -> None:
    """kv_write into a uint16 (IEEE half) cache; f32 rows round to nearest even."""
    check(lib().eb_launch_kv_write_f16(stream, cache, cache_numel, src, src_numel, hkv, count,
                                       hd, max_seq, dst_start))


def launch_attn_prefill_chunk_f16(stream: int, q: int, q_numel: int, kc: int, kc_numel: int,
                                  vc: int, vc_numel: int, o: int, o_numel: int, h: int,
                                  hkv: int, pos0: int, rows: int, hd: int, max_seq: int,
                                  scale: float, window: int = 0) -> None:
    check(lib().eb_launch_attn_prefill_chunk_f16(stream, q, q_numel, kc, kc_numel, vc, vc_numel,
                                                 o, o_numel, h, hkv, pos0, rows, hd, max_seq,
                                                 scale, window))


def launch_attn_decode_f16(stream: int, q: int, q_numel: int, kc: int, kc_numel: int, vc: int,
                           vc_numel: int, o: int, o_numel: int, h: int, hkv: int, pos: int,
                           hd: int, max_seq: int, scale: float, window: int, workspace: int,
                           workspace_floats: int, cu_count: int) -> None:
    check(lib().eb_launch_attn_decode_f16(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                          o_numel, h, hkv, pos, hd, max_seq, scale, window,
                                          workspace, workspace_floats, cu_count))


def launch_attn_decode_step_f16(stream: int, q: int, q_numel: int, knew: int, vnew: int,
                                new_numel: int, kc: int, kc_numel: int, vc: int, vc_numel: int,
                                o: int, o_numel: int, h: int, hkv: int, pos: int, hd: int,
                                max_seq: int, scale: float, window: int, workspace: int,
                                workspace_floats: int, cu_count: int) -> None:
    check(lib().eb_launch_attn_decode_step_f16(stream, q, q_numel, knew, vnew, new_numel, kc,
                                               kc_numel, vc, vc_numel, o, o_numel, h, hkv, pos,
                                               hd, max_seq, scale, window, workspace,
                                               workspace_floats, cu_count))


# ---- raw launches over OCP FP8 E4M3 caches (no counterpart in the reference) -----------

def launch_kv_write_f8(stream: int, cache: int, cache_numel: int, src: int, src_numel: int,
                       hkv: int, count: int, hd: int, max_seq: int, dst_start: int) -> None:
    """kv_write into a uint8 (E4M3) cache: nearest value, ties to even, finite values
    saturating at +-448, inf and NaN to NaN."""
    check(lib().eb_launch_kv_write_f8(stream, cache, cache_numel, src, src_numel, hkv, count,
                                      hd, max_seq, dst_start))


def launch_attn_prefill_chunk_f8(stream: int, q: int, q_numel: int, kc: int, kc_numel: int,
                                 vc: int, vc_numel: int, o: int, o_numel: int, h: int,
                                 hkv: int, pos0: int, rows: int, hd: int, max_seq: int,
                                 scale: float, window: int = 0) -> None:
    check(lib().eb_launch_attn_prefill_chunk_f8(stream, q, q_numel, kc, kc_numel, vc, vc_numel,
                                                o, o_numel, h, hkv, pos0, rows, hd, max_seq,
                                                scale, window))


def launch_attn_decode_f8(stream: int, q: int, q_numel: int, kc: int, kc_numel: int, vc: int,
                          vc_numel: int, o: int, o_numel: int, h: int, hkv: int, pos: int,
                          hd: int, max_seq: int, scale: float, window: int, workspace: int,
                          workspace_floats: int, cu_count: int) -> None:
    check(lib().eb_launch_attn_decode_f8(stream, q, q_numel, kc, kc_numel, vc, vc_numel, o,
                                         o_numel, h, hkv, pos, hd, max_seq, scale, window,
                                         workspace, workspace_floats, cu_count))


def launch_attn_decode_step_f8(stream: int, q: int, q_numel: int, knew: int, vnew: int,
                               new_numel: int, kc: int, kc_numel: int, vc: int, vc_numel: int,
                               o: int, o_numel: int, h: int, hkv: int, pos: int, hd: int,
                               max_seq: int, scale: float, window: int, workspace: int,
                               workspace_floats: int, cu_count: int) -> None:
    check(lib().eb_launch_attn_decode_step_f8(stream, q, q_numel, knew, vnew, new_numel, kc,
                                              kc_numel, vc, vc_numel, o, o_numel, h, hkv, pos,
                                              hd, max_seq, scale, window, workspace,
                                              workspace_floats, cu_count))


def launch_rmsnorm(stream: int, x: int, x_numel: int, w: int, w_numel: int, out: int,
                   out_numel: int, rows: int, dim: int, eps: float) -> None:
    check(lib().eb_launch_rmsnorm(stream, x, x_numel, w, w_numel, out, out_numel, rows, dim,
                                  eps))


def launch_rope(stream: int, x: int, x_numel: int, cos: int, sin: int, table_numel: int,
                out: int, out_numel: int, seq: int, n_heads: int, head_dim: int,
                base_pos: int) -> None:
    check(lib().eb_launch_rope(stream, x, x_numel, cos, sin, table_numel, out, out_numel, seq,
                               n_heads, head_dim, base_pos))


def launch_attn_prologue(stream: int, q: int, q_numel: int, k: int, k_numel: int, v: int,
                         v_numel: int, rows: int, h: int, hkv: int, hd: int, q_norm: int,
                         k_norm: int, v_norm: int, eps: float, rope_cos: int, rope_sin: int,
                         table_numel: int, base_pos: int, q_out: int, q_out_numel: int,
                         kcache: int, kc_numel: int, vcache: int, vc_numel: int, max_seq: int,
                         cache_dtype: int) -> None:
    """eb_launch_attn_prologue: Attention::prefill between the projections and the attention
    (crates/eyebrowse-nn/src/attention.rs:62-97) in one launch. Null (0) gains: no norm;
    null tables: no RoPE."""
    check(lib().eb_launch_attn_prologue(stream, q, q_numel, k, k_numel, v, v_numel, rows, h, hkv,
                                        hd, q_norm, k_norm, v_norm, eps, rope_cos, rope_sin,
                                        table_numel, base_pos, q_out, q_out_numel, kcache,
                                        kc_numel, vcache, vc_numel, max_seq, int(cache_dtype)))


LANE_OPS_ROWS = 14  # EB_LANE_OPS_ROWS


def launch_selftest_lane_ops(stream: int, inp: int, out: int) -> None:
    """eb_launch_selftest_lane_ops: one wave's lane-exchange results for a = in[0:64],
    b = in[64:128], LANE_OPS_ROWS rows of 64 floats (device pointers)."""
    check(lib().eb_launch_selftest_lane_ops(stream, inp, out))


def attn_decode_noalloc_max_floats() -> int:
    """Floats of split partials the no-allocation decode step's static scratch holds."""
    return int(lib().eb_attn_decode_noalloc_max_floats())


def launch_attn_decode_step_noalloc(stream: int, q: int, q_numel: int, knew: int, vnew: int,
                                    new_numel: int, kc: int, kc_numel: int, vc: int,
                                    vc_numel: int, o: int, o_numel: int, h: int, hkv: int,
                                    pos: int, hd: int, max_seq: int, scale: float,
                                    cu_count: int) -> None:
    """eb_launch_attn_decode_step_noalloc: the fused decode step with its split partials in
    the library's static device scratch (no allocation, no workspace argument)."""
    check(lib().eb_launch_attn_decode_step_noalloc(stream, q, q_numel, knew, vnew, new_numel, kc,
                                                   kc_numel, vc, vc_numel, o, o_numel, h, hkv,
                                                   pos, hd, max_seq, scale, cu_count))
