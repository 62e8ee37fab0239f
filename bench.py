#!/usr/bin/env python3
"""Benchmark of the eyebrowse attention hot path on one MI355X.

Headline (`value`): the largest single-GPU BASELINE configuration, configs[3]: a
Mistral-7B-shaped batch-1 decode step at KV length 32768 (the new token's K/V written at
position 32767, then attention over 32768 keys of a max_seq 32768 f32 cache, 32 query /
8 KV heads, head_dim 128). value = KV bytes read per step (2 * keys * Hkv * hd * 4) *
steps / time, in GB/s.

One step = eb_launch_attn_decode_step (the kv_write(K), kv_write(V), attn_decode sequence
of Attention::decode, crates/eyebrowse-nn/src/attention.rs:149-183, fused: the split-KV
pass that also writes the new row, then the log-sum-exp merge). Exactly --steps steps are
timed, as HIP graphs of consecutive steps. Steps rotate over enough distinct caches that
the working set exceeds the 256 MB Infinity Cache, so the K/V bytes come from HBM. Inputs
are resident in HBM before timing starts.

The same line carries `roofline` (the decode step against HBM), `roofline_prefill` (the
Mistral T=4096 causal prefill of the same config against the f16 and FP32 matrix peaks),
`roofline_prefill_f16` (the same prefill in the opt-in f16 mode), `roofline_prefill_pv16`
(Gemma-4 T=4096 in the opt-in scores-accurate mode),
`cpu_baseline` (the oracle on this host's cores, the same decode config) and, under
`extra`, every other BASELINE decode / prefill config, the IEEE-half cache decodes,
chunked prefill, the projections and a layer decode step.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]
       python bench.py --only trace --workload NAME   (one workload, for rocprofv3)
       python bench.py --trace-summary OUT.md TITLE CMD LABEL=CSV ...   (no GPU)
       python bench.py --pmc-summary FETCH.csv WRITE.csv OUT.json       (no GPU)
       python bench.py --sq-summary OUT.md CMD [WORKLOAD=]CSV ...        (no GPU)
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

    def time_region(self, stream, body):
        """ms of body()'s work, bracketed by HIP events on `stream`."""
        a, b = self.event(), self.event()
        s = ctypes.c_void_p(stream)
        self.ok(self.l.hipStreamSynchronize(s), "hipStreamSynchronize")
        self.ok(self.l.hipEventRecord(a, s), "hipEventRecord")
        body()
        self.ok(self.l.hipEventRecord(b, s), "hipEventRecord")
        ms = self.elapsed_ms(a, b)
        self.l.hipEventDestroy(a)
        self.l.hipEventDestroy(b)
        return ms

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
                 f16=False, f8=False):
        self.eb, self.hip, self.dev = eb, hip, dev
        self.H, self.Hkv, self.hd, self.max_seq, self.pos, self.scale = H, Hkv, hd, max_seq, pos, scale
        self.f16, self.f8 = f16, f8
        esize = 1 if f8 else 2 if f16 else 4
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
                if f8:
                    t = eb.Tensor.empty(dev, fill.shape, eb.DType.F8E4M3)
                    eb.launch_kv_write_f8(dev.stream, t.data_ptr, t.numel(), fill.data_ptr,
                                          fill.numel(), Hkv, max_seq, hd, max_seq, 0)
                elif f16:
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
        self.rem_graphs = {}
        self.graph = hip.capture(dev.stream, lambda: [self._step(self.caches[i % self.n_caches])
                                                      for i in range(self.per_graph)])

    def _step(self, cache):
        kc, vc = cache
        if self.f16 or self.f8:
            fn = self.eb.launch_attn_decode_step_f8 if self.f8 else self.eb.launch_attn_decode_step_f16
            fn(
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

    def run_exact(self, n):
        """Average ms per step over exactly n steps: n // per_graph whole graphs, then one
        graph of the n % per_graph remaining steps (captured once per length), all inside
        one pair of HIP events."""
        full, rem = divmod(n, self.per_graph)
        st = self.dev.stream
        if rem and rem not in self.rem_graphs:
            self.rem_graphs[rem] = self.hip.capture(
                st, lambda: [self._step(self.caches[i % self.n_caches]) for i in range(rem)])
            # a graph's first launch uploads it: keep that out of the timed region
            self.hip.launch(self.rem_graphs[rem], st)
            self.hip.ok(self.hip.l.hipStreamSynchronize(ctypes.c_void_p(st)),
                        "hipStreamSynchronize")

        def body():
            for _ in range(full):
                self.hip.launch(self.graph, st)
            if rem:
                self.hip.launch(self.rem_graphs[rem], st)
        return self.hip.time_region(st, body) / max(n, 1)

    def close(self):
        self.hip.l.hipGraphExecDestroy(self.graph)
        for g in self.rem_graphs.values():
            self.hip.l.hipGraphExecDestroy(g)
        self.rem_graphs.clear()


class PrefillWorkload:
    """Causal prefill over T tokens: K/V written by kv_write into a [T, Hkv, hd] cache,
    attention over the fresh K/V."""

    def __init__(self, eb, dev, H, Hkv, hd, T, scale, seed=0, presplit=True, fast=False,
                 pv16=False):
        self.eb, self.dev = eb, dev
        self.fast = fast
        self.pv16 = pv16  # the scores-accurate mode (same workspace as the accurate one)
        self.H, self.Hkv, self.hd, self.T, self.scale = H, Hkv, hd, T, scale
        self.flops = 2.0 * H * hd * T * (T + 1)
        rng = np.random.default_rng(seed)
        self.q = eb.Tensor.from_f32(dev, (T, H, hd), randn(rng, (T, H, hd)))
        self.k = eb.Tensor.from_f32(dev, (T, Hkv, hd), randn(rng, (T, Hkv, hd)))
        self.v = eb.Tensor.from_f32(dev, (T, Hkv, hd), randn(rng, (T, Hkv, hd)))
        self.o = eb.Tensor.empty(dev, (T, H, hd))
        # The pre-split workspace (head_dim 32..128, T >= 256): K/V split once per key, then
        # the attention kernel; both launches are inside every timed step.
        if fast:  # the f16 mode's pre-convert records
            self.ws_floats = eb.attn_prefill_fast_workspace_floats(H, Hkv, hd, T) if presplit else 0
        else:
            self.ws_floats = eb.attn_prefill_workspace_floats(H, Hkv, hd, 0, T) if presplit else 0
        self.ws = eb.Tensor.empty(dev, (self.ws_floats,)) if self.ws_floats else None

    def launch(self):
        e = self.eb
        args = (self.dev.stream, self.q.data_ptr, self.q.numel(), self.k.data_ptr,
                self.k.numel(), self.v.data_ptr, self.v.numel(), self.o.data_ptr,
                self.o.numel(), self.H, self.Hkv, self.T, self.hd, self.scale)
        if self.fast and self.ws is not None:
            e.launch_attn_prefill_fast_ws(*args, self.ws.data_ptr, self.ws_floats)
        elif self.fast:
            e.launch_attn_prefill_fast(*args)
        elif self.pv16 and self.ws is not None:
            e.launch_attn_prefill_pv16_ws(*args, self.ws.data_ptr, self.ws_floats)
        elif self.pv16:
            e.launch_attn_prefill_pv16(*args)
        elif self.ws is not None:
            e.launch_attn_prefill_ws(*args, self.ws.data_ptr, self.ws_floats)
        else:
            e.launch_attn_prefill(*args)


# ------------------------------------------------------------------ CPU baseline

def cpu_model() -> str:
    """The host CPU's model name (/proc/cpuinfo)."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    import platform
    return platform.processor() or "unknown"


def cpu_baseline(budget_s: float = 12.0) -> dict:
    """The oracle (a C restatement of the reference's CPU attention,
    crates/eyebrowse-kernels/src/testutil.rs:130-218) timed on this host on the headline
    workload: the Mistral decode at 32768 keys, one thread pinned to one core
    (os.sched_setaffinity) for about budget_s; the prefill restatement on the last 32 query
    rows of Mistral T=4096 (the heaviest rows) on the same core; and, as a secondary figure,
    the same decode with the heads spread over up to 16 OpenMP threads (the GPU box's CPU
    share)."""
    import oracle

    H, Hkv, hd, max_seq, pos = 32, 8, 128, 32768, 32767
    rng = np.random.default_rng(1)
    q = randn(rng, (H, hd))
    kc = randn(rng, (max_seq, Hkv, hd))
    vc = randn(rng, (max_seq, Hkv, hd))
    sc = float(oracle.default_scale(hd))
    T = 4096
    pq, pk, pv = randn(rng, (T, H, hd)), randn(rng, (T, Hkv, hd)), randn(rng, (T, Hkv, hd))
    rows = 32
    allowed = os.sched_getaffinity(0)
    core = min(allowed)
    os.sched_setaffinity(0, {core})
    try:
        oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, max_seq, sc)  # warm
        n, t0 = 0, time.perf_counter()
        while True:
            oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, max_seq, sc)
            n += 1
            dt = time.perf_counter() - t0
            if dt >= budget_s:
                break
        t1 = time.perf_counter()
        oracle.attn_prefill(pq, pk, pv, H, Hkv, T, hd, sc, rows=(T - rows, rows), threads=1)
        pdt = time.perf_counter() - t1
    finally:
        os.sched_setaffinity(0, allowed)
    kv_bytes = 2 * (pos + 1) * Hkv * hd * 4
    gbs = kv_bytes * n / dt / 1e9
    pflops = sum(2.0 * 2 * H * hd * (i + 1) for i in range(T - rows, T))

    mt = max(1, min(16, len(allowed)))
    m, t2 = 0, time.perf_counter()
    while True:
        oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, max_seq, sc, threads=mt)
        m += 1
        mdt = time.perf_counter() - t2
        if mdt >= budget_s / 4:
            break
    return {
        "value": round(gbs, 3), "unit": "GB/s", "cores": 1, "kind": "port",
        "sample": f"oracle attn_decode on the headline workload (Mistral 32/8 heads, hd 128, "
                  f"32768 keys of a 32768-row f32 cache): {n} calls in {dt:.1f} s, 1 thread "
                  f"pinned to core {core}",
        "cpu_model": cpu_model(), "host_cpus": os.cpu_count(), "allowed_cpus": len(allowed),
        "prefill_gflops": round(pflops / pdt / 1e9, 3),
        "prefill_sample": f"oracle attn_prefill, Mistral T=4096, last {rows} query rows, "
                          f"1 thread pinned to core {core}, {pdt:.2f} s",
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
            ("qwen_L8191", 16, 8, 128, 8192, 8191, sc128),
            ("mistral_keys8193", 32, 8, 128, 32768, 8192, sc128),
            ("gemma_keys16384", 16, 8, 256, 16384, 16383, 1.0)]
    # IEEE-half caches (no counterpart in the reference): half the bytes per key.
    cfgs += [("f16_qwen_L8191", 16, 8, 128, 8192, 8191, sc128, "f16"),
             ("f16_mistral_keys32768", 32, 8, 128, 32768, 32767, sc128, "f16"),
             ("f16_gemma_keys16384", 16, 8, 256, 16384, 16383, 1.0, "f16")]
    # OCP FP8 E4M3 caches (no counterpart in the reference): a quarter of the f32 bytes.
    cfgs += [("f8_qwen_L8191", 16, 8, 128, 8192, 8191, sc128, "f8"),
             ("f8_mistral_keys32768", 32, 8, 128, 32768, 32767, sc128, "f8"),
             ("f8_gemma_keys16384", 16, 8, 256, 16384, 16383, 1.0, "f8")]
    for name, H, Hkv, hd, ms, pos, sc, *el in cfgs:
        w = DecodeWorkload(eb, hip, dev, H, Hkv, hd, ms, pos, sc, f16=el == ["f16"],
                           f8=el == ["f8"])
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
    out.update(fast_prefill_extras(eb, hip, dev, sc128))
    out.update(pv16_prefill_extras(eb, hip, dev, sc128))
    out.update(chunk_extras(eb, hip, dev))
    return out


def pv16_prefill_extras(eb, hip, dev, sc128) -> dict:
    """The opt-in scores-accurate prefill (eb_launch_attn_prefill_pv16_ws: three-product
    scores, one f16 P V product) on the BASELINE prefill configs, Gemma-4's scale 1.0
    included; TFLOP/s of the same algorithmic FLOPs, against the f16 peak."""
    out = {}
    for name, H, Hkv, hd, T, sc in (("qwen_T512", 16, 8, 128, 512, sc128),
                                    ("qwen_T2048", 16, 8, 128, 2048, sc128),
                                    ("qwen_T4096", 16, 8, 128, 4096, sc128),
                                    ("mistral_T4096", 32, 8, 128, 4096, sc128),
                                    ("gemma_T4096", 16, 8, 256, 4096, 1.0)):
        p = PrefillWorkload(eb, dev, H, Hkv, hd, T, sc, pv16=True)
        for _ in range(3):
            p.launch()
        reps = 20 if T >= 2048 else 100
        t = hip.time_loop(dev.stream, reps, lambda i: p.launch())
        tf_s = p.flops / (t * 1e-3) / 1e12
        out[f"prefill_pv16_{name}"] = {
            "gflop": round(p.flops / 1e9, 3), "ms": round(t, 4), "TFLOPs": round(tf_s, 2),
            "mfma": "v_mfma_f32_32x32x16_f16: Q K^T three products on exact hi/lo splits, "
                    "V^T P^T one product (f16 V, f16 P)",
            "tolerance": PV16_TOLERANCE,
            "frac_f16_mfma_peak": round(tf_s / F16_MFMA_PEAK_TFLOPS, 4)}
        del p
        dev.synchronize()
    return out


def fast_prefill_extras(eb, hip, dev, sc128) -> dict:
    """The opt-in single-product f16 prefill (eb_launch_attn_prefill_fast: q, K, V, P rounded
    to f16 once, one f16 MFMA per product) on the BASELINE prefill configs it accepts (scale
    1/sqrt(hd)); TFLOP/s of the same algorithmic FLOPs, against the f16 peak."""
    out = {}
    for name, H, Hkv, hd, T in (("qwen_T512", 16, 8, 128, 512), ("qwen_T2048", 16, 8, 128, 2048),
                                ("qwen_T4096", 16, 8, 128, 4096),
                                ("mistral_T4096", 32, 8, 128, 4096)):
        p = PrefillWorkload(eb, dev, H, Hkv, hd, T, sc128, fast=True)
        for _ in range(3):
            p.launch()
        reps = 20 if T >= 2048 else 100
        t = hip.time_loop(dev.stream, reps, lambda i: p.launch())
        tf_s = p.flops / (t * 1e-3) / 1e12
        out[f"prefill_f16fast_{name}"] = {
            "gflop": round(p.flops / 1e9, 3), "ms": round(t, 4), "TFLOPs": round(tf_s, 2),
            "mfma": "v_mfma_f32_32x32x16_f16, one product per product (f16 q, K, V, P)",
            "tolerance": "rel-L2 <= 1e-3, max-abs <= 2e-3 vs the f32 oracle (measured ~4e-4)",
            "frac_f16_mfma_peak": round(tf_s / F16_MFMA_PEAK_TFLOPS, 4)}
        del p
        dev.synchronize()
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
    microseconds per step (HIP events), recorded eagerly and replayed as captured HIP graphs
    of one and of eight steps, with the host time per call; and chains of 1 and 20 tiny
    kernels, eager and as graphs, which separate a graph launch's per-replay cost from its
    per-node cost."""
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

    def timed(fn, n, per=1):
        """(GPU µs per step from HIP events, host µs per call) over n calls of fn, each
        covering `per` steps."""
        for _ in range(5):
            fn()
        dev.synchronize()
        t0 = time.perf_counter()
        for _ in range(n):
            fn()
        host = (time.perf_counter() - t0) / n * 1e6
        dev.synchronize()
        return round(hip.time_loop(dev.stream, n, lambda i: fn()) * 1e3 / per, 2), round(host, 2)

    eager, eager_host = timed(step, 200)
    graphs = {}
    for nsteps in (1, 8):
        dev.begin_capture()
        try:
            keep = [step() for _ in range(nsteps)]
        finally:
            g = dev.end_capture()
        graphs[nsteps] = timed(g.launch, 400 // nsteps, nsteps)
        dev.synchronize()
        g.release()
        del keep
    # chains of a tiny kernel (argmax over 64 floats, one workgroup): the per-kernel cost of
    # eager launches and of graph nodes, and the per-replay cost of a graph launch
    xs = eb.Tensor.from_f32(dev, (64,), np.arange(64, dtype=np.float32))
    wst = eb.Tensor.empty(dev, (eb.argmax_workspace_floats(64),))
    idx = eb.Tensor.empty(dev, (1,), eb.DType.U32)

    def tiny(k):
        for _ in range(k):
            eb.launch_argmax(dev.stream, xs.data_ptr, 64, idx.data_ptr, 64, wst.data_ptr,
                             wst.numel())
    chains = {}
    for k in (1, 20):
        e_us, e_host = timed(lambda: tiny(k), 200, k)
        dev.begin_capture()
        try:
            tiny(k)
        finally:
            g = dev.end_capture()
        g_us, g_host = timed(g.launch, 200, k)
        dev.synchronize()
        g.release()
        chains[f"x{k}"] = {"eager_us_per_kernel": e_us, "graph_us_per_kernel": g_us,
                           "graph_launch_host_us": g_host}
    return {"layer_decode_step_qwen_pos100": {
        "kernels": 5, "eager_us": eager, "eager_host_us_per_step": eager_host,
        "graph_us": graphs[1][0], "graph_launch_host_us": graphs[1][1],
        "graph_8_steps_us_per_step": graphs[8][0],
        "graph_8_steps_launch_host_us": graphs[8][1],
        "tiny_kernel_chains": chains}}


def traffic_run(eb, hip, dev, sc128):
    """Dispatches for the HBM-traffic counter passes, each kernel launched directly (no
    graph) so that every dispatch is counted on its own:
      1. kv_write copying 256 MiB (a plain copy of known size: FETCH_SIZE and WRITE_SIZE
         of it calibrate the counters), 3 times;
      2. the headline decode step (Mistral, 32768 keys) over its rotated caches, 6 times;
      3. Mistral T=4096 prefill (pre-split pass + attention), 3 times;
      4. the Gemma-4 decode step at 16384 keys, 6 times, and its T=4096 prefill, 3 times.
    The four workloads use distinct kernel instantiations, so per-kernel averages do not mix
    them (Qwen shares the head_dim 128 merge and pre-split kernels with Mistral and is left
    out)."""
    rows, hkv, hd = 65536, 8, 128
    src = eb.Tensor.empty(dev, (rows, hkv, hd))
    dst = eb.Tensor.empty(dev, (rows, hkv, hd))
    for _ in range(3):
        eb.launch_kv_write(dev.stream, dst.data_ptr, dst.numel(), src.data_ptr, src.numel(), hkv,
                           rows, hd, rows, 0)
    dev.synchronize()
    del src, dst
    for H, Hkv, hdd, ms, pos, sc in ((32, 8, 128, 32768, 32767, sc128),
                                     (16, 8, 256, 16384, 16383, 1.0)):
        w = DecodeWorkload(eb, hip, dev, H, Hkv, hdd, ms, pos, sc, per_graph=1)
        for i in range(6):
            w._step(w.caches[i % w.n_caches])
        dev.synchronize()
        w.close()
        del w
        p = PrefillWorkload(eb, dev, H, Hkv, hdd, 4096, sc)
        for _ in range(3):
            p.launch()
        dev.synchronize()
        del p
        print(json.dumps({"traffic_run": f"H{H} hd{hdd} done"}), flush=True)
    print(json.dumps({"traffic_run": "done", "copy_bytes": rows * hkv * hd * 4}), flush=True)


def _kernel_name(raw: str) -> str:
    import re
    name = re.sub(r"\(anonymous namespace\)::", "", raw).split("(")[0]
    return name.replace("void ", "").strip()


def pmc_summary(fetch_csv: str, write_csv: str, out_json: str) -> None:
    """Per-kernel HBM traffic from two rocprofv3 --pmc passes (FETCH_SIZE, WRITE_SIZE, KiB
    per dispatch) over `bench.py --only traffic`. Each counter is scaled by what it reads
    for the 256 MiB kv_write copies in that run (bytes copied / counter bytes), so that
    traffic is in the same bytes as the algorithmic figures. On this part FETCH_SIZE reads
    half of a known copy's read bytes (its factor measures about 2.0 in every run) and
    WRITE_SIZE all of them (1.0): the factor is measured in each run, not assumed."""
    import csv
    import re

    copy = "kv_write_vec4_kernel"

    def load(path):
        # The first three kv_write dispatches are the calibration copies; later ones (the
        # decode workloads filling their caches) are left out of every average.
        per, calib = {}, []
        rows = sorted(csv.DictReader(open(path)), key=lambda r: int(r["Dispatch_Id"]))
        for r in rows:
            name = _kernel_name(r["Kernel_Name"])
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
        "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc FETCH_SIZE "
        "--kernel-trace -f csv -d $R/gpurun_out/pmc_fetch -o run -- python3 $R/bench.py "
        "--only traffic",
        "cd /tmp && export TMPDIR=/tmp && timeout -s KILL 120 rocprofv3 --pmc WRITE_SIZE "
        "--kernel-trace -f csv -d $R/gpurun_out/pmc_write -o run -- python3 $R/bench.py "
        "--only traffic",
        "python bench.py --pmc-summary gpurun_out/pmc_fetch/run_counter_collection.csv "
        "gpurun_out/pmc_write/run_counter_collection.csv profiles/traffic.json"],
        "calibration": "the run's first three kv_write_vec4_kernel dispatches, each copying "
                       "256 MiB (65536 rows x 8 heads x 128 f32): scale = 268435456 / "
                       "(counter KiB * 1024); FETCH_SIZE reads half of the copy's bytes, "
                       "WRITE_SIZE all of them",
        "fetch_scale": round(fs, 4), "write_scale": round(ws, 4), "kernels": kernels}

    def total(*patterns):
        t = 0
        for pat in patterns:
            k = next((k for k in kernels if re.fullmatch(pat, k)), None)
            if k is None:
                return None
            t += kernels[k]["fetch_bytes"] + kernels[k]["write_bytes"]
        return t
    # (template arguments: decode_kernel<head_dim, heads per workgroup, cache element bytes>,
    # presplit_kernel<head_dim, element bytes, non-temporal loads, V16>,
    # prefill_kernel<head_dim, heads, row blocks, key splits, range, element bytes, pre-split
    # records, f16 mode, scores-accurate mode>)
    out["decode_mistral_keys32768"] = total(r"decode_kernel<128, 4, 4>",
                                            r"decode_merge_kernel<128>")
    out["prefill_mistral_T4096"] = total(
        r"presplit_kernel<128, 4, false, false>",
        r"prefill_kernel<128, 4, 1, 1, false, 4, true, false, false>")
    out["decode_gemma_keys16384"] = total(r"decode_kernel<256, 2, 4>",
                                          r"decode_merge_kernel<256>")
    out["prefill_gemma_T4096"] = total(
        r"presplit_kernel<256, 4, false, false>",
        r"prefill_kernel<256, 2, 2, 1, false, 4, true, false, false>")
    json.dump(out, open(out_json, "w"), indent=1)
    print(json.dumps(out, indent=1))


def trace_summary(out_md: str, title: str, cmd: str, labelled: list) -> None:
    """A markdown table of rocprofv3 kernel traces (one run_kernel_trace.csv per workload,
    given as LABEL=CSV): per workload and kernel (and grid), the dispatch count and the
    average / min / max duration, with the kernel's resources."""
    import csv
    lines = [f"# {title}", "", "Command (from the repository root on the GPU box, `R=$PWD`):",
             "", "```", cmd, "```", "",
             "| workload | kernel | workgroups | threads/WG | VGPR | AGPR | LDS B | scratch | "
             "dispatches | avg µs | min µs | max µs |",
             "|---|---|---|---|---|---|---|---|---|---|---|---|"]
    for item in labelled:
        label, path = item.split("=", 1)
        groups = {}
        for r in csv.DictReader(open(path)):
            wg = 1
            for ax in "XYZ":
                wg *= int(r[f"Grid_Size_{ax}"]) // max(1, int(r[f"Workgroup_Size_{ax}"]))
            th = int(r["Workgroup_Size_X"]) * int(r["Workgroup_Size_Y"]) * int(r["Workgroup_Size_Z"])
            key = (_kernel_name(r["Kernel_Name"]), wg, th, int(r.get("VGPR_Count", 0) or 0),
                   int(r.get("Accum_VGPR_Count", 0) or 0), int(r.get("LDS_Block_Size", 0) or 0),
                   int(r.get("Scratch_Size", 0) or 0))
            dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1000.0
            groups.setdefault(key, []).append(dur)
        for (n, wg, th, v, a, lds, scr), ds in groups.items():
            ds.sort()
            lines.append(f"| {label} | `{n}` | {wg} | {th} | {v} | {a} | {lds} | {scr} | "
                         f"{len(ds)} | {sum(ds) / len(ds):.2f} | {ds[0]:.2f} | {ds[-1]:.2f} |")
    open(out_md, "w").write("\n".join(lines) + "\n")
    print("\n".join(lines))


def sq_summary(out_md: str, cmd: str, *csv_paths: str) -> None:
    """Per-dispatch averages of the SQ / GRBM counters of one or more rocprofv3 --pmc runs
    (each run averaged over its own dispatches, then merged per kernel and grid; the
    counters are whole-chip totals per dispatch), with: VALU instructions per MFMA
    instruction; MFMA busy cycles per MFMA instruction; the share of wave cycles spent
    waiting on any instruction, and on LDS instructions; LDS bank-conflict cycles per
    LDS-active cycle; and the matrix pipe's busy share, SQ_VALU_MFMA_BUSY_CYCLES /
    (1024 SIMDs x GRBM_GUI_ACTIVE / 8), GRBM_GUI_ACTIVE being the sum of the 8 XCDs' busy
    cycles (so the share is of the cycles the kernel ran, at the clock it ran at).
    A CSV given as WORKLOAD=PATH labels its rows with that workload (the passes of one
    workload merge into its rows), so that configs whose kernels share a grid stay apart.
    Where the pass's kernel trace lies beside its counter CSV (X_kernel_trace.csv next to
    X_counter_collection.csv), the kernel's average duration in that same pass and the clock
    it implies, GRBM_GUI_ACTIVE / 8 / duration, are reported too: the pipe-busy share is of
    the cycles at that clock."""
    import csv
    merged, ndisp, timing = {}, {}, {}
    for arg in csv_paths:
        label, path = arg.split("=", 1) if "=" in arg else ("", arg)
        tot, disp = {}, {}
        for r in csv.DictReader(open(path)):
            key = (label, _kernel_name(r["Kernel_Name"]), r.get("Grid_Size", ""))
            c = tot.setdefault(key, {})
            c[r["Counter_Name"]] = c.get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
            disp.setdefault(key, set()).add(r["Dispatch_Id"])
        durs = {}
        kt = path.replace("_counter_collection.csv", "_kernel_trace.csv")
        if kt != path and os.path.exists(kt):
            for r in csv.DictReader(open(kt)):
                g = int(r["Grid_Size_X"]) * int(r["Grid_Size_Y"]) * int(r["Grid_Size_Z"])
                key = (label, _kernel_name(r["Kernel_Name"]), str(g))
                durs.setdefault(key, []).append(
                    (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3)
        for key, c in tot.items():
            n = len(disp[key])
            m = merged.setdefault(key, {})
            for k, v in c.items():
                m.setdefault(k, v / n)  # (a counter in two runs: the first run's average)
            ndisp[key] = max(ndisp.get(key, 0), n)
            d = durs.get(key)
            if d and "GRBM_GUI_ACTIVE" in c and key not in timing:
                us = sum(d) / len(d)
                timing[key] = (us, c["GRBM_GUI_ACTIVE"] / n / 8 / us / 1e3)
    names = sorted({n for c in merged.values() for n in c})
    lines = ["# SQ counters per dispatch", "", "Command (from the repository root on the GPU "
             "box, `R=$PWD`):", "", "```", cmd, "```", "",
             "| workload | kernel | grid | dispatches | " + " | ".join(names) +
             " | VALU/MFMA | MFMA busy cyc/MFMA | wait share | LDS wait share |"
             " LDS conflict/active | MFMA pipe busy | pass µs | clock GHz |",
             "|---" * (4 + len(names) + 8) + "|"]
    for key, avg in merged.items():
        mf = avg.get("SQ_INSTS_MFMA", 0)
        ratio = lambda a, b: f"{a / b:.2f}" if b else "-"  # noqa: E731
        lines.append(f"| {key[0] or '-'} | `{key[1]}` | {key[2]} | {ndisp[key]} | " +
                     " | ".join(f"{avg[k]:.0f}" if k in avg else "-" for k in names) + " | " +
                     ratio(avg.get("SQ_INSTS_VALU", 0), mf) + " | " +
                     ratio(avg.get("SQ_VALU_MFMA_BUSY_CYCLES", 0), mf) + " | " +
                     ratio(avg.get("SQ_WAIT_INST_ANY", 0), avg.get("SQ_WAVE_CYCLES", 0)) + " | " +
                     ratio(avg.get("SQ_WAIT_INST_LDS", 0), avg.get("SQ_WAVE_CYCLES", 0)) + " | " +
                     ratio(avg.get("SQ_LDS_BANK_CONFLICT", 0), avg.get("SQ_LDS_IDX_ACTIVE", 0)) +
                     " | " + ratio(avg.get("SQ_VALU_MFMA_BUSY_CYCLES", 0),
                                   1024 * avg.get("GRBM_GUI_ACTIVE", 0) / 8) + " | " +
                     (f"{timing[key][0]:.1f} | {timing[key][1]:.2f}" if key in timing
                      else "- | -") + " |")
    open(out_md, "w").write("\n".join(lines) + "\n")
    print("\n".join(lines))


def trace_workload(eb, hip, dev, sc128, name: str) -> None:
    """One workload alone, for a rocprofv3 kernel trace: decode steps through HIP graphs
    (200 steps), prefill launches (3 warm-up + 20; prefill_f16fast_* in the f16 mode,
    prefill_pv16_* in the scores-accurate mode), the layer decode step (eager and graph),
    or a Gemma-4 prompt through Attention.forward_qkv (the fused pre-attention pass, the
    pre-split pass and the attention)."""
    decode = {"decode_mistral_keys32768": (32, 8, 128, 32768, 32767, sc128, False),
              "decode_gemma_keys16384": (16, 8, 256, 16384, 16383, 1.0, False),
              "decode_qwen_L8191": (16, 8, 128, 8192, 8191, sc128, False),
              "decode_f16_mistral_keys32768": (32, 8, 128, 32768, 32767, sc128, True),
              "decode_f8_mistral_keys32768": (32, 8, 128, 32768, 32767, sc128, "f8")}
    prefill = {"prefill_qwen_T512": (16, 8, 128, 512, sc128),
               "prefill_qwen_T2048": (16, 8, 128, 2048, sc128),
               "prefill_qwen_T4096": (16, 8, 128, 4096, sc128),
               "prefill_mistral_T4096": (32, 8, 128, 4096, sc128),
               "prefill_gemma_T4096": (16, 8, 256, 4096, 1.0)}
    if name in decode:
        H, Hkv, hd, ms, pos, sc, el = decode[name]
        w = DecodeWorkload(eb, hip, dev, H, Hkv, hd, ms, pos, sc, f16=el is True,
                           f8=el == "f8")
        w.run_exact(200)
        dev.synchronize()
        w.close()
    elif name.replace("f16fast_", "").replace("pv16_", "") in prefill:
        H, Hkv, hd, T, sc = prefill[name.replace("f16fast_", "").replace("pv16_", "")]
        p = PrefillWorkload(eb, dev, H, Hkv, hd, T, sc, fast="f16fast_" in name,
                            pv16="pv16_" in name)
        for _ in range(23):
            p.launch()
        dev.synchronize()
    elif name == "layer_step":
        print(json.dumps(layer_step_extras(eb, hip, dev)), flush=True)
    elif name == "prompt_gemma_T4096":
        H, Hkv, hd, T = 16, 8, 256, 4096
        rng = np.random.default_rng(6)
        gq = eb.Tensor.from_f32(dev, (hd,), 1 + 0.1 * randn(rng, (hd,)))
        gk = eb.Tensor.from_f32(dev, (hd,), 1 + 0.1 * randn(rng, (hd,)))
        ones = eb.Tensor.from_f32(dev, (hd,), np.ones(hd, np.float32))
        attn = eb.Attention(H, Hkv, hd, 1.0, q_norm=gq, k_norm=gk, v_norm=ones, norm_eps=1e-6)
        rope = eb.Rope.build_partial(dev, T, hd, 32, 1e6)
        kv = eb.KvCache.new(dev, 1, T, Hkv, hd)
        q = eb.Tensor.from_f32(dev, (T, H * hd), randn(rng, (T, H * hd)))
        k = eb.Tensor.from_f32(dev, (T, Hkv * hd), randn(rng, (T, Hkv * hd)))
        v = eb.Tensor.from_f32(dev, (T, Hkv * hd), randn(rng, (T, Hkv * hd)))
        for _ in range(10):
            rec = eb.Recorder(dev)
            attn.forward_qkv(rec, q, k, v, rope, kv, 0, T, 0)
            rec.submit()
        dev.synchronize()
    else:
        raise SystemExit(f"unknown workload {name}")
    print(json.dumps({"trace_workload": name, "done": True}), flush=True)


PV16_TOLERANCE = ("max-abs <= 2^-11 x max|V| (half an f16 ulp of V) vs the f32 oracle; "
                  "on the BASELINE configs rel-L2 <= 1e-3 and max-abs <= 2e-3 (measured "
                  "rel-L2 2.1e-4 - 2.7e-4, max-abs 1.95e-3 at Gemma-4)")


def pv16_roofline(eb, hip, dev, reps: int = 20) -> dict:
    """The opt-in scores-accurate prefill on Gemma-4 T=4096 (head_dim
    256, scale 1.0, which the f16 mode refuses): the pre-split pass plus the attention
    kernel, HIP events around `reps` back-to-back launches."""
    p = PrefillWorkload(eb, dev, 16, 8, 256, 4096, 1.0, pv16=True)
    for _ in range(3):
        p.launch()
    ms = hip.time_loop(dev.stream, reps, lambda i: p.launch())
    tf = p.flops / (ms * 1e-3) / 1e12
    del p
    dev.synchronize()
    return {
        "bound": "mfma",
        "config": "gemma-4-dense-shaped global-layer causal prefill, T=4096, 16 q / 8 KV heads, "
                  "head_dim 256, scale 1.0, f32 q/k/v (BASELINE configs[4]), opt-in "
                  "scores-accurate mode",
        "kernel": "presplit_kernel<256, 4, false, true> + prefill_kernel<256, 2, 2, 1, false, "
                  "4, true, false, true>",
        "mfma": "v_mfma_f32_32x32x16_f16: Q K^T three products on exact hi/lo splits, V^T P^T "
                "one product (f16 V, f16 P), f32 softmax and accumulation",
        "tolerance": PV16_TOLERANCE,
        "achieved": round(tf, 2), "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
        "frac": round(tf / F16_MFMA_PEAK_TFLOPS, 4),
        "algorithmic_flops_per_launch": p_flops(16, 256, 4096),
        "avg_launch_ms": round(ms, 5),
    }


def prefill_roofline(eb, hip, dev, sc128, reps: int = 20, fast: bool = False) -> dict:
    """The prefill half of the metric on the same config as the headline (BASELINE
    configs[3], Mistral-7B T=4096): the pre-split pass plus the attention kernel (f32-accurate
    default), or the opt-in single-product f16 mode (fast), HIP events around `reps`
    back-to-back launches."""
    if fast:
        p = PrefillWorkload(eb, dev, 32, 8, 128, 4096, sc128, fast=True)
        for _ in range(3):
            p.launch()
        ms = hip.time_loop(dev.stream, reps, lambda i: p.launch())
        tf = p.flops / (ms * 1e-3) / 1e12
        del p
        dev.synchronize()
        return {
            "bound": "mfma",
            "config": "mistral-7b-shaped causal prefill, T=4096, 32 q / 8 KV heads, head_dim "
                      "128, f32 q/k/v (BASELINE configs[3]), opt-in f16 mode",
            "kernel": "preconvert_kernel<128> + "
                      "prefill_kernel<128, 4, 1, 1, false, 4, true, true, false>",
            "mfma": "v_mfma_f32_32x32x16_f16, one product per product: q, K, V, P rounded to "
                    "f16 once, f32 softmax and accumulation",
            "tolerance": "rel-L2 <= 1e-3 and max-abs <= 2e-3 vs the f32 oracle (measured "
                         "about 4e-4 rel-L2)",
            "achieved": round(tf, 2), "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
            "frac": round(tf / F16_MFMA_PEAK_TFLOPS, 4),
            "algorithmic_flops_per_launch": p_flops(32, 128, 4096),
            "avg_launch_ms": round(ms, 5),
        }
    p = PrefillWorkload(eb, dev, 32, 8, 128, 4096, sc128)
    for _ in range(3):
        p.launch()
    ms = hip.time_loop(dev.stream, reps, lambda i: p.launch())
    tf = p.flops / (ms * 1e-3) / 1e12
    traffic = None
    tfp = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tfp):
        traffic = json.load(open(tfp)).get("prefill_mistral_T4096")
    del p
    dev.synchronize()
    return {
        "bound": "mfma",
        "config": "mistral-7b-shaped causal prefill, T=4096, 32 q / 8 KV heads, head_dim 128, "
                  "f32 q/k/v (BASELINE configs[3])",
        "kernel": "presplit_kernel<128, 4, false, false> + "
                  "prefill_kernel<128, 4, 1, 1, false, 4, true, false, false>",
        "mfma": "v_mfma_f32_32x32x16_f16 on exact f16 hi/lo splits of the f32 operands, "
                "three products per product (f32-accurate), f32 accumulation",
        "achieved": round(tf, 2), "peak": F16_MFMA_PEAK_TFLOPS, "unit": "TFLOP/s",
        "frac": round(tf / F16_MFMA_PEAK_TFLOPS, 4),
        "peak_fp32_mfma": FP32_MFMA_PEAK_TFLOPS,
        "frac_fp32_mfma": round(tf / FP32_MFMA_PEAK_TFLOPS, 4),
        "issued_f16_mfma_TFLOPs": round(3 * tf, 1),
        "frac_issued_f16_mfma": round(3 * tf / F16_MFMA_PEAK_TFLOPS, 4),
        "traffic": traffic, "algorithmic_flops_per_launch": p_flops(32, 128, 4096),
        "avg_launch_ms": round(ms, 5),
    }


def p_flops(H, hd, T):
    return 2.0 * H * hd * T * (T + 1)


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
    ap.add_argument("--trace-summary", nargs="+", metavar="ARG",
                    help="no GPU: OUT_MD TITLE CMD LABEL=KERNEL_TRACE_CSV ...")
    ap.add_argument("--sq-summary", nargs="+", metavar="ARG",
                    help="no GPU: per-kernel SQ counter table of a --pmc run")
    ap.add_argument("--only", choices=["headline", "all", "prefill", "projections", "layer",
                                       "traffic", "trace"], default="all",
                    help="headline: the contract line without extras; prefill / projections / "
                         "layer: only those extras; traffic: a short run for rocprofv3 --pmc "
                         "passes; trace: one --workload for a rocprofv3 kernel trace")
    ap.add_argument("--workload", default="", help="the workload of --only trace")
    args = ap.parse_args()
    if args.pmc_summary:
        pmc_summary(*args.pmc_summary)
        return
    if args.trace_summary:
        if len(args.trace_summary) < 4:
            raise SystemExit("--trace-summary OUT_MD TITLE CMD LABEL=CSV ...")
        out_md, title, cmd, *labelled = args.trace_summary
        trace_summary(out_md, title, cmd, labelled)
        return
    if args.sq_summary:
        if len(args.sq_summary) < 3:
            raise SystemExit("--sq-summary OUT_MD CMD [WORKLOAD=]CSV ...")
        sq_summary(*args.sq_summary)
        return
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: the eyebrowse attention path is a single-device "
              "workload and this build has no multi-GPU path (run with --gpus 1).",
              file=sys.stderr)
        sys.exit(2)
    if args.steps < 1 or args.warmup < 0:
        raise SystemExit("--steps must be >= 1 and --warmup >= 0")

    import eyebrowse_amd as eb
    hip = Hip()
    dev = eb.Device.new(0)
    sc128 = float(np.float32(1.0) / np.sqrt(np.float32(128)))
    if args.only == "traffic":
        traffic_run(eb, hip, dev, sc128)
        return
    if args.only == "trace":
        trace_workload(eb, hip, dev, sc128, args.workload)
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

    # Headline: Mistral decode at 32768 keys (the largest single-GPU
    # decode). A step is the fused decode launch (new-row write + split-KV pass) and the
    # merge, so the step time bounds the dominant kernel's launch duration from above.
    H, Hkv, hd, max_seq, pos = 32, 8, 128, 32768, 32767
    head = DecodeWorkload(eb, hip, dev, H, Hkv, hd, max_seq, pos, sc128)
    # Clocks settle under load: the step runs untimed for about 0.3 s before the W warm-up
    # steps (a short timed region right after an idle start reads several percent low).
    t_end = time.perf_counter() + 0.3
    while time.perf_counter() < t_end:
        for _ in range(8):
            hip.launch(head.graph, dev.stream)
        dev.synchronize()
    if args.warmup:
        head.run_exact(args.warmup)
    dev.synchronize()
    ms_step = head.run_exact(args.steps)
    dev.synchronize()
    value = head.kv_bytes / (ms_step * 1e-3) / 1e9
    traffic = None
    tf = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tf):
        traffic = json.load(open(tf)).get("decode_mistral_keys32768")
    n_caches, per_graph, kv_bytes = head.n_caches, head.per_graph, head.kv_bytes
    head.close()
    del head
    dev.synchronize()
    print(f"[bench] headline decode {ms_step * 1e3:.2f} us/step, {value:.1f} GB/s",
          file=sys.stderr, flush=True)
    pf = prefill_roofline(eb, hip, dev, sc128)
    print(f"[bench] prefill {pf['achieved']} TFLOP/s", file=sys.stderr, flush=True)
    pff = prefill_roofline(eb, hip, dev, sc128, fast=True)
    print(f"[bench] prefill f16 mode {pff['achieved']} TFLOP/s", file=sys.stderr, flush=True)
    pfv = pv16_roofline(eb, hip, dev)
    print(f"[bench] prefill scores-accurate mode (Gemma-4) {pfv['achieved']} TFLOP/s",
          file=sys.stderr, flush=True)

    extra = {}
    if args.only == "all":
        extra.update(decode_extras(eb, hip, dev, sc128))
        extra.update(prefill_extras(eb, hip, dev, sc128))
        extra.update(projection_extras(eb, hip, dev))
        extra.update(layer_step_extras(eb, hip, dev))
        print("[bench] extras done", file=sys.stderr, flush=True)

    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": "mistral-7b-shaped batch-1 decode step at KV length 32768: kv_write "
                        "of the new token at pos 32767 + attention over 32768 keys of a "
                        "max_seq 32768 f32 cache (BASELINE configs[3])",
            "n_heads": H, "n_kv_heads": Hkv, "head_dim": hd, "max_seq": max_seq, "pos": pos,
            "kv_caches_rotated": n_caches,
            "launch": f"eb_launch_attn_decode_step, HIP graphs of {per_graph} steps plus one "
                      f"of the remainder (exactly --steps steps timed)",
        },
        "roofline": {
            "bound": "hbm",
            "kernel": "decode_kernel<128, 4, 4> (new-row write + split-KV pass) + "
                      "decode_merge_kernel<128>",
            "achieved": round(value, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(value / HBM_PEAK_GBS, 4), "traffic": traffic,
            "algorithmic_bytes_per_launch": kv_bytes, "avg_launch_ms": round(ms_step, 6),
        },
        "roofline_prefill": pf,
        "roofline_prefill_f16": pff,
        "roofline_prefill_pv16": pfv,
        "extra": extra,
    }
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline()
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
