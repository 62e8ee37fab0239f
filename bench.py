#!/usr/bin/env python3
"""Benchmark of the eyebrowse attention hot path on one MI355X.

Headline (`value`): BASELINE config 2 at its largest point: a Qwen3-0.6B-shaped batch-1
decode step at L = 8191 (new token's K/V written at position 8191 by kv_write, then
attention over 8192 keys of a max_seq 8192 f32 cache, 16 query / 8 KV heads, hd 128).
value = KV bytes read per step (2 * keys * Hkv * hd * 4) * steps / time, in GB/s.

One step = one HIP-graph launch of [kv_write K, kv_write V, attn_decode] (the kernels the
library records for Attention::decode, crates/eyebrowse-nn/src/attention.rs:149-183).
Steps rotate over enough distinct caches that the working set exceeds the 256 MB Infinity
Cache, so the K/V bytes come from HBM. Inputs are resident in HBM before timing starts.

Also reported: prefill TFLOP/s (2*H*hd*T*(T+1) algorithmic FLOPs) for the BASELINE
prefill configs, decode GB/s at every BASELINE decode config, the roofline of the dominant
kernel, and the CPU oracle timed on this host (cpu_baseline).

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

METRIC = "prefill attn TFLOP/s + decode KV-read GB/s, as % of MI355X roofline"
HBM_PEAK_GBS = 8000.0          # MI355X HBM3E, GB/s
FP32_MFMA_PEAK_TFLOPS = 157.3  # MI355X dense FP32 matrix
F16_MFMA_PEAK_TFLOPS = 2500.0  # MI355X dense f16 matrix
MALL_BYTES = 256 << 20


# ------------------------------------------------------------------ HIP runtime via ctypes

class Hip:
    """The few HIP runtime calls the harness needs: events and stream capture."""

    def __init__(self):
        self.l = ctypes.CDLL("libamdhip64.so")
        vp, pvp = ctypes.c_void_p, ctypes.POINTER(ctypes.c_void_p)
        sig = {
            "hipEventCreate": [pvp], "hipEventRecord": [vp, vp], "hipEventSynchronize": [vp],
            "hipEventElapsedTime": [ctypes.POINTER(ctypes.c_float), vp, vp],
            "hipEventDestroy": [vp], "hipStreamBeginCapture": [vp, ctypes.c_int],
            "hipStreamEndCapture": [vp, pvp],
            "hipGraphInstantiate": [pvp, vp, vp, ctypes.c_char_p, ctypes.c_size_t],
            "hipGraphLaunch": [vp, vp], "hipGraphExecDestroy": [vp], "hipGraphDestroy": [vp],
            "hipStreamSynchronize": [vp], "hipDeviceSynchronize": [],
        }
        for name, args in sig.items():
            f = getattr(self.l, name)
            f.restype = ctypes.c_int
            f.argtypes = args

    def ok(self, rc, what):
        if rc != 0:
            raise RuntimeError(f"{what} failed with hipError {rc}")

    def event(self):
        e = ctypes.c_void_p()
        self.ok(self.l.hipEventCreate(ctypes.byref(e)), "hipEventCreate")
        return e

    def elapsed_ms(self, a, b):
        self.ok(self.l.hipEventSynchronize(b), "hipEventSynchronize")
        ms = ctypes.c_float()
        self.ok(self.l.hipEventElapsedTime(ctypes.byref(ms), a, b), "hipEventElapsedTime")
        return float(ms.value)

    def capture(self, stream, fn):
        """Record fn()'s launches on `stream` into an executable graph."""
        s = ctypes.c_void_p(stream)
        self.ok(self.l.hipStreamBeginCapture(s, 0), "hipStreamBeginCapture")
        try:
            fn()
        finally:
            g = ctypes.c_void_p()
            rc = self.l.hipStreamEndCapture(s, ctypes.byref(g))
        self.ok(rc, "hipStreamEndCapture")
        ge = ctypes.c_void_p()
        self.ok(self.l.hipGraphInstantiate(ctypes.byref(ge), g, None, None, 0),
                "hipGraphInstantiate")
        self.ok(self.l.hipGraphDestroy(g), "hipGraphDestroy")
        return ge

    def launch(self, ge, stream):
        self.ok(self.l.hipGraphLaunch(ge, ctypes.c_void_p(stream)), "hipGraphLaunch")

    def time_loop(self, stream, n, body):
        """Average ms of body(i) over n iterations, bracketed by HIP events on `stream`."""
        a, b = self.event(), self.event()
        s = ctypes.c_void_p(stream)
        self.ok(self.l.hipStreamSynchronize(s), "hipStreamSynchronize")
        self.ok(self.l.hipEventRecord(a, s), "hipEventRecord")
        for i in range(n):
            body(i)
        self.ok(self.l.hipEventRecord(b, s), "hipEventRecord")
        ms = self.elapsed_ms(a, b)
        self.l.hipEventDestroy(a)
        self.l.hipEventDestroy(b)
        return ms / n


# ------------------------------------------------------------------ workloads

def randn(rng, shape):
    return rng.standard_normal(shape, dtype=np.float32)


class DecodeWorkload:
    """Batch-1 decode step at position `pos` over `n_caches` distinct [max_seq, Hkv, hd]
    K/V caches (rows 0..pos-1 filled), with the new token's K/V written at `pos`.

    A step is eb_launch_attn_decode_step: kv_write of K and V at `pos` plus attention over
    pos+1 keys, one kernel. `per_graph` consecutive steps (cycling through the caches) are
    captured in one HIP graph so the host launch cost is paid once per graph."""

    def __init__(self, eb, hip, dev, H, Hkv, hd, max_seq, pos, scale, seed=0, per_graph=64,
                 f16=False):
        self.eb, self.hip, self.dev = eb, hip, dev
        self.H, self.Hkv, self.hd, self.max_seq, self.pos, self.scale = H, Hkv, hd, max_seq, pos, scale
        self.f16 = f16
        esize = 2 if f16 else 4
        self.keys = pos + 1
        self.kv_bytes = 2 * self.keys * Hkv * hd * esize
        cache_bytes = 2 * max_seq * Hkv * hd * esize
        self.n_caches = max(3, int(np.ceil(1.5 * MALL_BYTES / cache_bytes)) + 1)
        rng = np.random.default_rng(seed)
        kfill = eb.Tensor.from_f32(dev, (max_seq, Hkv, hd), randn(rng, (max_seq, Hkv, hd)))
        vfill = eb.Tensor.from_f32(dev, (max_seq, Hkv, hd), randn(rng, (max_seq, Hkv, hd)))
        self.caches = []
        for _ in range(self.n_caches):
            pair = []
            for fill in (kfill, vfill):
                if f16:
                    t = eb.Tensor.empty(dev, fill.shape, eb.DType.F16)
                    eb.launch_kv_write_f16(dev.stream, t.data_ptr, t.numel(), fill.data_ptr,
                                           fill.numel(), Hkv, max_seq, hd, max_seq, 0)
                else:
                    t = eb.Tensor.empty(dev, fill.shape)
                    eb.launch_kv_write(dev.stream, t.data_ptr, t.numel(), fill.data_ptr,
                                       fill.numel(), Hkv, max_seq, hd, max_seq, 0)
                pair.append(t)
            self.caches.append(tuple(pair))
        dev.synchronize()
        del kfill, vfill
        self.q = eb.Tensor.from_f32(dev, (H, hd), randn(rng, (H, hd)))
        self.knew = eb.Tensor.from_f32(dev, (1, Hkv, hd), randn(rng, (1, Hkv, hd)))
        self.vnew = eb.Tensor.from_f32(dev, (1, Hkv, hd), randn(rng, (1, Hkv, hd)))
        self.o = eb.Tensor.empty(dev, (H, hd))
        self.cus = dev.cu_count
        self.wsn = eb.attn_decode_workspace_floats(H, Hkv, pos, hd, self.cus)
        self.ws = eb.Tensor.empty(dev, (max(self.wsn, 1),))
        self.per_graph = max(per_graph // self.n_caches, 1) * self.n_caches
        self.graph = hip.capture(dev.stream, lambda: [self._step(self.caches[i % self.n_caches])
                                                      for i in range(self.per_graph)])

    def _step(self, cache):
        kc, vc = cache
        if self.f16:
            self.eb.launch_attn_decode_step_f16(
                self.dev.stream, self.q.data_ptr, self.q.numel(), self.knew.data_ptr,
                self.vnew.data_ptr, self.knew.numel(), kc.data_ptr, kc.numel(), vc.data_ptr,
                vc.numel(), self.o.data_ptr, self.o.numel(), self.H, self.Hkv, self.pos,
                self.hd, self.max_seq, self.scale, 0, self.ws.data_ptr, self.wsn, self.cus)
            return
        self.eb.launch_attn_decode_step(
            self.dev.stream, self.q.data_ptr, self.q.numel(), self.knew.data_ptr,
            self.vnew.data_ptr, self.knew.numel(), kc.data_ptr, kc.numel(), vc.data_ptr,
            vc.numel(), self.o.data_ptr, self.o.numel(), self.H, self.Hkv, self.pos, self.hd,
            self.max_seq, self.scale, self.ws.data_ptr, self.wsn, self.cus)

    def run_steps(self, n):
        """Average ms per step over at least n steps (whole graphs)."""
        reps = max(1, -(-n // self.per_graph))
        st = self.dev.stream
        ms = self.hip.time_loop(st, reps, lambda i: self.hip.launch(self.graph, st))
        return ms / self.per_graph, reps * self.per_graph

    def close(self):
        self.hip.l.hipGraphExecDestroy(self.graph)


class PrefillWorkload:
    """Causal prefill over T tokens: K/V written by kv_write into a [T, Hkv, hd] cache,
    attention over the fresh K/V."""

    def __init__(self, eb, dev, H, Hkv, hd, T, scale, seed=0, presplit=True):
        self.eb, self.dev = eb, dev
        self.H, self.Hkv, self.hd, self.T, self.scale = H, Hkv, hd, T, scale
        self.flops = 2.0 * H * hd * T * (T + 1)
        rng = np.random.default_rng(seed)
        self.q = eb.Tensor.from_f32(dev, (T, H, hd), randn(rng, (T, H, hd)))
        self.k = eb.Tensor.from_f32(dev, (T, Hkv, hd), randn(rng, (T, Hkv, hd)))
        self.v = eb.Tensor.from_f32(dev, (T, Hkv, hd), randn(rng, (T, Hkv, hd)))
        self.o = eb.Tensor.empty(dev, (T, H, hd))
        # The pre-split workspace (head_dim 32..128, T >= 256): K/V split once per key, then
        # the attention kernel; both launches are inside every timed step.
        self.ws_floats = eb.attn_prefill_workspace_floats(H, Hkv, hd, 0, T) if presplit else 0
        self.ws = eb.Tensor.empty(dev, (self.ws_floats,)) if self.ws_floats else None

    def launch(self):
        e = self.eb
        args = (self.dev.stream, self.q.data_ptr, self.q.numel(), self.k.data_ptr,
                self.k.numel(), self.v.data_ptr, self.v.numel(), self.o.data_ptr,
                self.o.numel(), self.H, self.Hkv, self.T, self.hd, self.scale)
        if self.ws is not None:
            e.launch_attn_prefill_ws(*args, self.ws.data_ptr, self.ws_floats)
        else:
            e.launch_attn_prefill(*args)


# ------------------------------------------------------------------ CPU baseline

def cpu_baseline(budget_s: float = 12.0) -> dict:
    """The oracle (a C restatement of the reference's CPU attention,
    crates/eyebrowse-kernels/src/testutil.rs:177-218) timed on this host's cores, single
    thread, on the headline decode step (8192 keys, Qwen shape) repeated for ~budget_s."""
    import oracle

    H, Hkv, hd, max_seq, pos = 16, 8, 128, 8192, 8191
    rng = np.random.default_rng(1)
    q = randn(rng, (H, hd))
    kc = randn(rng, (max_seq, Hkv, hd))
    vc = randn(rng, (max_seq, Hkv, hd))
    sc = float(oracle.default_scale(hd))
    oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, max_seq, sc)  # warm
    n, t0 = 0, time.perf_counter()
    while True:
        oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, max_seq, sc)
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget_s:
            break
    kv_bytes = 2 * (pos + 1) * Hkv * hd * 4
    gbs = kv_bytes * n / dt / 1e9

    # prefill sample: the last 16 query rows of Qwen T=4096 (the heaviest rows)
    T = 4096
    pq, pk, pv = randn(rng, (T, H, hd)), randn(rng, (T, Hkv, hd)), randn(rng, (T, Hkv, hd))
    rows = 16
    t1 = time.perf_counter()
    oracle.attn_prefill(pq, pk, pv, H, Hkv, T, hd, sc, rows=(T - rows, rows), threads=1)
    pdt = time.perf_counter() - t1
    pflops = sum(2.0 * 2 * H * hd * (i + 1) for i in range(T - rows, T))

    # secondary: the same decode with the oracle's heads spread over the host's cores
    # (16 at most: the GPU box's CPU share)
    mt = max(1, min(16, os.cpu_count() or 1))
    m, t2 = 0, time.perf_counter()
    while True:
        oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, max_seq, sc, threads=mt)
        m += 1
        mdt = time.perf_counter() - t2
        if mdt >= budget_s / 4:
            break
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"oracle attn_decode, Qwen3 shape 16/8 heads hd128, 8192 keys, {n} calls "
                  f"in {dt:.1f} s, 1 thread",
        "prefill_gflops": round(pflops / pdt / 1e9, 3),
        "prefill_sample": f"oracle attn_prefill, Qwen3 T=4096, last {rows} rows, 1 thread, "
                          f"{pdt:.1f} s",
        "host_cpus": os.cpu_count(),
        "all_cores_value": round(kv_bytes * m / mdt / 1e9, 3),
        "all_cores": mt,
        "all_cores_sample": f"the same decode, heads over {mt} OpenMP threads, {m} calls in "
                            f"{mdt:.1f} s",
    }


def decode_extras(eb, hip, dev, sc128) -> dict:
    """Decode step GB/s at every BASELINE decode config (kv_write + attention, graph-launched,
    caches rotated past the Infinity Cache)."""
    out = {}
    cfgs = [("qwen_L512", 16, 8, 128, 8192, 512, sc128),
            ("qwen_L2048", 16, 8, 128, 8192, 2048, sc128),
            ("qwen_L4096", 16, 8, 128, 8192, 4096, sc128),
            ("mistral_keys8193", 32, 8, 128, 32768, 8192, sc128),
            ("mistral_keys32768", 32, 8, 128, 32768, 32767, sc128),
            ("gemma_keys16384", 16, 8, 256, 16384, 16383, 1.0)]
    # IEEE-half caches (no counterpart in the reference): half the bytes per key.
    cfgs += [("f16_qwen_L8191", 16, 8, 128, 8192, 8191, sc128, True),
             ("f16_mistral_keys32768", 32, 8, 128, 32768, 32767, sc128, True),
             ("f16_gemma_keys16384", 16, 8, 256, 16384, 16383, 1.0, True)]
    for name, H, Hkv, hd, ms, pos, sc, *f16 in cfgs:
        w = DecodeWorkload(eb, hip, dev, H, Hkv, hd, ms, pos, sc, f16=bool(f16))
        w.run_steps(20)
        t_step, _ = w.run_steps(500)
        out[f"decode_{name}"] = {
            "keys": pos + 1, "kv_bytes": w.kv_bytes, "ms_step": round(t_step, 5),
            "GBs": round(w.kv_bytes / t_step / 1e6, 1),
            "frac_hbm": round(w.kv_bytes / t_step / 1e6 / HBM_PEAK_GBS, 4)}
        w.close()
        del w
        dev.synchronize()
    return out


def prefill_extras(eb, hip, dev, sc128) -> dict:
    """Causal prefill TFLOP/s (2*H*hd*T*(T+1) algorithmic FLOPs) for the BASELINE prefill
    configs, HIP events around back-to-back launches. Each step is the pre-split pass plus
    the attention kernel (eb_launch_attn_prefill_ws); the plain raw launch, which splits K/V
    while staging them, is reported beside it."""
    out = {}
    cfgs = [("qwen_T512", 16, 8, 128, 512, sc128),
            ("qwen_T2048", 16, 8, 128, 2048, sc128),
            ("qwen_T4096", 16, 8, 128, 4096, sc128),
            ("mistral_T4096", 32, 8, 128, 4096, sc128),
            ("gemma_T4096", 16, 8, 256, 4096, 1.0)]
    for name, H, Hkv, hd, T, sc in cfgs:
        p = PrefillWorkload(eb, dev, H, Hkv, hd, T, sc)
        for _ in range(3):
            p.launch()
        reps = 20 if T >= 2048 else 100
        t = hip.time_loop(dev.stream, reps, lambda i: p.launch())
        tf_s = p.flops / (t * 1e-3) / 1e12
        # both products on the f16 matrix cores as three split products each (f32 accuracy)
        f16_work = 3 * tf_s
        staged = {}
        if p.ws is not None:
            ps = PrefillWorkload(eb, dev, H, Hkv, hd, T, sc, presplit=False)
            ps.launch()
            t2 = hip.time_loop(dev.stream, reps, lambda i: ps.launch())
            staged = {"TFLOPs_split_while_staging": round(p.flops / (t2 * 1e-3) / 1e12, 2)}
            del ps
        out[f"prefill_{name}"] = {
            "gflop": round(p.flops / 1e9, 3), "ms": round(t, 4), "TFLOPs": round(tf_s, 2),
            "path": "pre-split pass + attention" if p.ws is not None else "attention",
            **staged,
            "mfma": "f16 split x3 (v_mfma_f32_32x32x16_f16) for Q K^T and V^T P^T",
            "frac_fp32_mfma_peak": round(tf_s / FP32_MFMA_PEAK_TFLOPS, 4),
            "f16_mfma_work_TFLOPs": round(f16_work, 1),
            "frac_f16_mfma_peak_of_mfma_work": round(f16_work / F16_MFMA_PEAK_TFLOPS, 4)}
        del p
        dev.synchronize()
    out.update(chunk_extras(eb, hip, dev))
    return out


def chunk_extras(eb, hip, dev) -> dict:
    """Chunked prefill (a prompt continuation attending a filled cache): `rows` new query
    rows at positions pos0.. over [max_seq, hkv, hd] f32 caches, through
    eb_launch_attn_prefill_chunk_ws (pre-split pass where rows >= 256, key chunks merged by
    a second launch). FLOPs 4*H*hd*sum_r(pos0 + r + 1)."""
    rng = np.random.default_rng(5)
    out = {}
    for name, H, Hkv, hd, pos0, rows in (("qwen_128_over_8k", 16, 8, 128, 8064, 128),
                                         ("mistral_256_over_32k", 32, 8, 128, 32512, 256)):
        ms = pos0 + rows
        q = eb.Tensor.from_f32(dev, (rows, H, hd), randn(rng, (rows, H, hd)))
        kc = eb.Tensor.from_f32(dev, (ms, Hkv, hd), randn(rng, (ms, Hkv, hd)))
        vc = eb.Tensor.from_f32(dev, (ms, Hkv, hd), randn(rng, (ms, Hkv, hd)))
        o = eb.Tensor.empty(dev, (rows, H, hd))
        need = eb.attn_prefill_workspace_floats(H, Hkv, hd, pos0, rows)
        ws = eb.Tensor.empty(dev, (max(need, 1),))
        sc = float(1.0 / np.sqrt(hd))

        def launch(_i):
            eb.launch_attn_prefill_chunk_ws(dev.stream, q.data_ptr, q.numel(), kc.data_ptr,
                                            kc.numel(), vc.data_ptr, vc.numel(), o.data_ptr,
                                            o.numel(), H, Hkv, pos0, rows, hd, ms, sc, 0,
                                            ws.data_ptr, need)
        for _ in range(2):
            launch(0)
        t = hip.time_loop(dev.stream, 10, launch)
        flops = 4.0 * H * hd * (rows * (pos0 + 1) + rows * (rows - 1) / 2)
        out[f"prefill_chunk_{name}"] = {"gflop": round(flops / 1e9, 3), "ms": round(t, 4),
                                        "TFLOPs": round(flops / (t * 1e-3) / 1e12, 2)}
        del q, kc, vc, o, ws
        dev.synchronize()
    return out


def projection_extras(eb, hip, dev) -> dict:
    """linear_f16w (the projections around attention): the weight-streaming kernel on the
    Qwen3 LM head (151936 x 1024 halves, 311 MB, beyond the Infinity Cache: GB/s of
    weight), and the split-f16 matrix-core GEMM on prompt-sized projections (TFLOP/s of
    2*m*in*out algorithmic FLOPs)."""
    rng = np.random.default_rng(3)
    out = {}

    def bench_one(name, m, k, outs, reps):
        x = eb.Tensor.from_f32(dev, (m, k), randn(rng, (m, k)))
        ws = [eb.Tensor.from_f16_packed(dev, (o, k), randn(rng, (o, k)) * 0.05) for o in outs]
        cs = [eb.Tensor.empty(dev, (m, o)) for o in outs]
        need = eb.linear_workspace_floats(m, k)
        wsp = eb.Tensor.empty(dev, (max(need, 1),))

        def launch(_i):
            if len(outs) == 1:
                eb.launch_linear_f16w(dev.stream, x.data_ptr, x.numel(), ws[0].data_ptr,
                                      2 * ws[0].numel(), cs[0].data_ptr, cs[0].numel(), m, k,
                                      outs[0], wsp.data_ptr, need)
            else:
                rec = eb.Recorder(dev)
                eb.linear_f16w_multi(rec, x, ws, cs, outs, m, k)
                rec.submit()
        for _ in range(3):
            launch(0)
        t = hip.time_loop(dev.stream, reps, launch)
        flops = 2.0 * m * k * sum(outs)
        wbytes = 2.0 * k * sum(outs)
        r = {"m": m, "in": k, "out": list(outs), "ms": round(t, 5)}
        if m <= 8:
            r["GBs_weight"] = round(wbytes / t / 1e6, 1)
            r["frac_hbm"] = round(wbytes / t / 1e6 / HBM_PEAK_GBS, 4)
        else:
            r["TFLOPs"] = round(flops / t / 1e9, 1)
            # two f16 MFMAs (x_hi*w, x_lo*w) per algorithmic multiply-add
            r["frac_f16_mfma_peak_of_mfma_work"] = round(2 * flops / t / 1e9 / F16_MFMA_PEAK_TFLOPS, 4)
        out[f"linear_{name}"] = r
        dev.synchronize()

    bench_one("qwen_lm_head_m1", 1, 1024, (151936,), 50)
    bench_one("qwen_qkv_T4096", 4096, 1024, (2048, 1024, 1024), 10)
    bench_one("qwen_o_T4096", 4096, 2048, (1024,), 10)
    bench_one("mistral_qkv_T4096", 4096, 4096, (4096, 1024, 1024), 5)
    return out


def layer_step_extras(eb, hip, dev) -> dict:
    """One Qwen3-width attention layer decode step at pos 100 (fused q/k/v projection,
    decode step with QK-norm and RoPE folded in, o_proj, a 4096-row LM head, argmax):
    microseconds per step, recorded eagerly and replayed as a captured HIP graph."""
    H, Hkv, hd, hidden, vocab, max_seq, pos = 16, 8, 128, 1024, 4096, 256, 100
    rng = np.random.default_rng(4)
    w = {n: eb.Tensor.from_f16_packed(dev, sh, randn(rng, sh) * 0.03)
         for n, sh in (("q", (H * hd, hidden)), ("k", (Hkv * hd, hidden)),
                       ("v", (Hkv * hd, hidden)), ("o", (hidden, H * hd)), ("lm", (vocab, hidden)))}
    gq = eb.Tensor.from_f32(dev, (hd,), 1 + 0.1 * randn(rng, (hd,)))
    gk = eb.Tensor.from_f32(dev, (hd,), 1 + 0.1 * randn(rng, (hd,)))
    attn = eb.Attention(H, Hkv, hd, float(hd ** -0.5), q_norm=gq, k_norm=gk, q_proj=w["q"],
                        k_proj=w["k"], v_proj=w["v"], o_proj=w["o"], hidden=hidden)
    rope = eb.Rope.build(dev, max_seq, hd, 1e6)
    kv = eb.KvCache.new(dev, 1, max_seq, Hkv, hd)
    rec = eb.Recorder(dev)
    attn.forward(rec, eb.Tensor.from_f32(dev, (pos, hidden), randn(rng, (pos, hidden))), rope,
                 kv, 0, pos, 0)
    rec.submit()
    x = eb.Tensor.from_f32(dev, (1, hidden), randn(rng, (1, hidden)))

    def step():
        r = eb.Recorder(dev)
        y = attn.forward(r, x, rope, kv, 0, 1, pos)
        logits = eb.Tensor.empty(dev, (1, vocab))
        eb.linear_f16w(r, y, w["lm"], logits, 1, hidden, vocab)
        idx = eb.Tensor.empty(dev, (1,), eb.DType.U32)
        eb.argmax(r, logits, idx, vocab)
        r.submit()
        return y, logits, idx

    for _ in range(5):
        step()
    eager = hip.time_loop(dev.stream, 200, lambda i: step())
    dev.begin_capture()
    try:
        keep = step()
    finally:
        g = dev.end_capture()
    for _ in range(5):
        g.launch()
    graph = hip.time_loop(dev.stream, 200, lambda i: g.launch())
    dev.synchronize()
    g.release()
    del keep
    return {"layer_decode_step_qwen_pos100": {
        "kernels": 7, "eager_us": round(eager * 1e3, 2), "graph_us": round(graph * 1e3, 2)}}


def traffic_run(eb, hip, dev, sc128):
    """Dispatches for the HBM-traffic counter passes, each kernel launched directly (no
    graph) so that every dispatch is counted on its own:
      1. kv_write copying 256 MiB (a plain copy of known size: FETCH_SIZE and WRITE_SIZE
         of it calibrate the counters), 3 times;
      2. the headline decode step (Qwen L=8191) over 7 rotated caches, 14 times;
      3. Qwen T=4096 prefill, 3 times."""
    rows, hkv, hd = 65536, 8, 128
    src = eb.Tensor.empty(dev, (rows, hkv, hd))
    dst = eb.Tensor.empty(dev, (rows, hkv, hd))
    for _ in range(3):
        eb.launch_kv_write(dev.stream, dst.data_ptr, dst.numel(), src.data_ptr, src.numel(), hkv,
                           rows, hd, rows, 0)
    dev.synchronize()
    del src, dst
    w = DecodeWorkload(eb, hip, dev, 16, 8, 128, 8192, 8191, sc128, per_graph=1)
    for i in range(14):
        w._step(w.caches[i % w.n_caches])
    dev.synchronize()
    w.close()
    del w
    p = PrefillWorkload(eb, dev, 16, 8, 128, 4096, sc128)
    for _ in range(3):
        p.launch()
    dev.synchronize()
    print(json.dumps({"traffic_run": "done", "copy_bytes": rows * hkv * hd * 4}), flush=True)


def pmc_summary(fetch_csv: str, write_csv: str, out_json: str) -> None:
    """Per-kernel HBM traffic from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE, KiB
    per dispatch) over `bench.py --only traffic`. Each counter is scaled by what it reads
    for the 256 MiB kv_write copy in that run (bytes copied / counter bytes), so that
    traffic is in the same bytes as the algorithmic figures."""
    import csv
    import re

    copy = "kv_write_vec4_kernel"

    def load(path):
        # The first three kv_write dispatches are the calibration copies; later ones (the
        # decode workload filling its caches) are left out of every average.
        per, calib = {}, []
        rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
        for r in rows:
            name = re.sub(r"\(anonymous namespace\)::", "", r["Kernel_Name"]).split("(")[0]
            name = name.replace("void ", "").strip()
            if name == copy:
                if len(calib) < 3:
                    calib.append(float(r["Counter_Value"]))
                continue
            per.setdefault(name, []).append(float(r["Counter_Value"]))
        avg = {k: sum(v) / len(v) for k, v in per.items()}
        avg[copy] = sum(calib) / len(calib)
        return avg

    fetch, write = load(fetch_csv), load(write_csv)
    copy_bytes = 65536 * 8 * 128 * 4
    fs = copy_bytes / (fetch[copy] * 1024)
    ws = copy_bytes / (write[copy] * 1024)
    kernels = {k: {"fetch_bytes": round(fetch[k] * 1024 * fs), "write_bytes": round(write.get(k, 0) * 1024 * ws),
                   "FETCH_SIZE_KiB": round(fetch[k], 1), "WRITE_SIZE_KiB": round(write.get(k, 0), 1)}
               for k in fetch}
    out = {"commands": [
        "cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc FETCH_SIZE --kernel-trace -f csv "
        "-d $R/gpurun_out/pmc_fetch -o run -- python3 $R/bench.py --only traffic",
        "cd /tmp && export TMPDIR=/tmp && rocprofv3 --pmc WRITE_SIZE --kernel-trace -f csv "
        "-d $R/gpurun_out/pmc_write -o run -- python3 $R/bench.py --only traffic",
        "python bench.py --pmc-summary gpurun_out/pmc_fetch/run_counter_collection.csv "
        "gpurun_out/pmc_write/run_counter_collection.csv profiles/traffic.json"],
        "calibration": "the run's first three kv_write_vec4_kernel dispatches, each copying "
                       "256 MiB (65536 rows x 8 heads x 128 f32): scale = 268435456 / "
                       "(counter KiB * 1024)",
        "fetch_scale": round(fs, 4), "write_scale": round(ws, 4), "kernels": kernels}
    dk = next((k for k in kernels if re.match(r"decode_kernel<128, 2\b", k)), None)
    mk = next((k for k in kernels if k.startswith("decode_merge_kernel<128>")), None)
    if dk:
        t = kernels[dk]["fetch_bytes"] + kernels[dk]["write_bytes"]
        if mk:
            t += kernels[mk]["fetch_bytes"] + kernels[mk]["write_bytes"]
        out["decode_qwen_L8191"] = t
    json.dump(out, open(out_json, "w"), indent=1)
    print(json.dumps(out, indent=1))


# ------------------------------------------------------------------ main

def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=2000)
    ap.add_argument("--warmup", type=int, default=100)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--pmc-summary", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "OUT_JSON"),
                    help="no GPU: turn the counter_collection.csv files of the FETCH_SIZE and "
                         "WRITE_SIZE passes over `--only traffic` into per-kernel HBM bytes")
    ap.add_argument("--only", choices=["headline", "all", "prefill", "projections", "layer",
                                       "traffic"], default="all",
                    help="headline: the decode line only; prefill / projections / layer: "
                         "only those extras (prints their timings, not the contract line); "
                         "traffic: a short run for rocprofv3 --pmc passes")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the eyebrowse attention path is a single-device "
              "workload and this build has no multi-GPU path (run with --gpus 1).",
              file=sys.stderr)
        sys.exit(2)

    import eyebrowse_amd as eb
    hip = Hip()
    dev = eb.Device.new(0)
    sc128 = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    if args.only == "traffic":
        traffic_run(eb, hip, dev, sc128)
        return
    if args.only == "prefill":
        print(json.dumps(prefill_extras(eb, hip, dev, sc128)), flush=True)
        return
    if args.only == "projections":
        print(json.dumps(projection_extras(eb, hip, dev)), flush=True)
        return
    if args.only == "layer":
        print(json.dumps(layer_step_extras(eb, hip, dev)), flush=True)
        return

    # Headline: Qwen decode L=8191. A step is one kernel (kv_write + split-KV attention +
    # merge), so the step time is also the dominant kernel's average launch duration.
    head = DecodeWorkload(eb, hip, dev, 16, 8, 128, 8192, 8191, sc128)
    head.run_steps(args.warmup)
    dev.synchronize()
    ms_step, steps_run = head.run_steps(args.steps)
    dev.synchronize()
    value = head.kv_bytes / (ms_step * 1e-3) / 1e9
    achieved = value
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("decode_qwen_L8191")

    extra = {}
    if args.only == "all":
        extra.update(decode_extras(eb, hip, dev, sc128))
        extra.update(prefill_extras(eb, hip, dev, sc128))
        extra.update(projection_extras(eb, hip, dev))
        extra.update(layer_step_extras(eb, hip, dev))

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps_run,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "qwen3-0.6b-shaped batch-1 decode step at L=8191: kv_write of the new "
                        "token at pos 8191 + attention over 8192 keys (BASELINE configs[1])",
            "n_heads": 16, "n_kv_heads": 8, "head_dim": 128, "max_seq": 8192, "pos": 8191,
            "kv_caches_rotated": head.n_caches,
            "launch": f"eb_launch_attn_decode_step, {head.per_graph} steps per hipGraph",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_kernel<128,2,false> (new-token write + split-KV pass) + decode_merge_kernel<128>",
            "achieved": round(achieved, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
            "algorithmic_bytes_per_launch": head.kv_bytes, "avg_launch_ms": round(ms_step, 6),
        },
        "extra": extra,
    }
    head.close()
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
