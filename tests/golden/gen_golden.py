"""Writes the committed golden vectors under tests/golden/ (run from the repo root:
``python tests/golden/gen_golden.py``).

The reference ships no fixtures for its attention path, so these are produced by the CPU
oracle (oracle/oracle.c, a restatement of crates/eyebrowse-kernels/src/testutil.rs) and
each is cross-checked here against an independent float64 evaluation of the textbook
formula before it is written. Inputs that come from the seeded generator are stored as
seeds plus a SHA-256 of their bytes (the test regenerates and checks them); small
reference-shaped inputs (ramps) are stored in full.
"""
import hashlib
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
from tests._textbook import (attention_f64, ramp, rel_l2_f64, rmsnorm_f64,  # noqa: E402
                             rope_f64)

TOL = 2e-6


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, np.float32).tobytes()).hexdigest()


def qwen_t64():
    """Qwen3-0.6B-shaped causal prefill, T=64, H=16, Hkv=8, hd=128."""
    T, H, Hkv, hd = 64, 16, 8, 128
    q = oracle.randn((T, H, hd), 1)
    k = oracle.randn((T, Hkv, hd), 2)
    v = oracle.randn((T, Hkv, hd), 3)
    sc = oracle.default_scale(hd)
    o = oracle.attn_prefill(q, k, v, H, Hkv, T, hd, sc)
    assert rel_l2_f64(o, attention_f64(q, k, v, sc)) < TOL
    np.savez(os.path.join(HERE, "qwen_t64_prefill.npz"), T=T, H=H, Hkv=Hkv, hd=hd, scale=sc,
             seeds=np.array([1, 2, 3]), sha_q=sha(q), sha_k=sha(k), sha_v=sha(v), o=o)


def qwen_decode_small():
    """Qwen-shaped decode over a short cache: max_seq 256, pos 200 (201 keys)."""
    H, Hkv, hd, max_seq, pos = 16, 8, 128, 256, 200
    q = oracle.randn((H, hd), 1)
    kc = oracle.randn((max_seq, Hkv, hd), 2)
    vc = oracle.randn((max_seq, Hkv, hd), 3)
    sc = oracle.default_scale(hd)
    o = oracle.attn_decode(q, kc, vc, H, Hkv, pos, hd, max_seq, sc)
    want = attention_f64(q[None], kc[: pos + 1], vc[: pos + 1], sc, causal=False)[0]
    assert rel_l2_f64(o, want) < TOL
    np.savez(os.path.join(HERE, "qwen_decode_small.npz"), H=H, Hkv=Hkv, hd=hd, max_seq=max_seq,
             pos=pos, scale=sc, seeds=np.array([1, 2, 3]), sha_q=sha(q), sha_kc=sha(kc),
             sha_vc=sha(vc), o=o)


def reference_ramp_cases():
    """The reference kernel tests' own inputs (crates/eyebrowse-kernels/src/attention.rs:
    175-233 and ops.rs:271-292), stored in full with the oracle's outputs."""
    h, hkv, s, hd = 2, 1, 5, 8
    pq = ramp(h * s * hd, -0.5, 0.011)
    pk = ramp(hkv * s * hd, -0.3, 0.007)
    pv = ramp(hkv * s * hd, 0.2, 0.013)
    po = oracle.attn_prefill(pq, pk, pv, h, hkv, s, hd)
    assert rel_l2_f64(po, attention_f64(pq.reshape(s, h, hd), pk.reshape(s, hkv, hd),
                                        pv.reshape(s, hkv, hd), 1 / np.sqrt(8))) < TOL
    dh, dhkv, dhd, dms, dpos = 4, 2, 8, 16, 5
    dq = ramp(dh * dhd, -0.4, 0.02)
    dk = ramp(dhkv * dms * dhd, -0.2, 0.005)
    dv = ramp(dhkv * dms * dhd, 0.1, 0.009)
    do = oracle.attn_decode(dq, dk, dv, dh, dhkv, dpos, dhd, dms)
    kk = dk.reshape(dms, dhkv, dhd)[: dpos + 1]
    vv = dv.reshape(dms, dhkv, dhd)[: dpos + 1]
    assert rel_l2_f64(do, attention_f64(dq.reshape(1, dh, dhd), kk, vv, 1 / np.sqrt(8),
                                        causal=False)[0]) < TOL
    cache = np.zeros(8 * 2 * 4, np.float32)
    src = np.arange(8, dtype=np.float32) + 1
    kvw = oracle.kv_write(cache, src, 2, 1, 4, 3)
    np.savez(os.path.join(HERE, "reference_ramp_cases.npz"), prefill_q=pq, prefill_k=pk,
             prefill_v=pv, prefill_o=po, decode_q=dq, decode_k=dk, decode_v=dv, decode_o=do,
             kvw_src=src, kvw_cache=kvw)


def gemma_t32():
    """Gemma-4 global-layer shape, short: T=32, H=16, Hkv=8, hd=256, scale 1.0,
    q/k RMSNorm with gains 1 + 0.1 z, weightless v RMSNorm, partial RoPE (32 of 128
    pairs, theta 1e6), then causal prefill."""
    T, H, Hkv, hd, eps = 32, 16, 8, 256, 1e-6
    q = oracle.randn((T, H, hd), 1)
    k = oracle.randn((T, Hkv, hd), 2)
    v = oracle.randn((T, Hkv, hd), 3)
    gq = (1 + 0.1 * oracle.randn((hd,), 4)).astype(np.float32)
    gk = (1 + 0.1 * oracle.randn((hd,), 5)).astype(np.float32)
    qn = oracle.rmsnorm(q, gq, T * H, hd, eps)
    kn = oracle.rmsnorm(k, gk, T * Hkv, hd, eps)
    vn = oracle.rmsnorm(v, np.ones(hd, np.float32), T * Hkv, hd, eps)
    c, s = oracle.rope_tables(T, hd, 1e6, rope_angles=32)
    qr = oracle.rope(qn, c, s, T, H, hd)
    kr = oracle.rope(kn, c, s, T, Hkv, hd)
    o = oracle.attn_prefill(qr, kr, vn, H, Hkv, T, hd, 1.0)
    # f64 chain
    qr64 = rope_f64(rmsnorm_f64(q, gq, hd, eps), T, H, hd, 1e6, rope_angles=32)
    kr64 = rope_f64(rmsnorm_f64(k, gk, hd, eps), T, Hkv, hd, 1e6, rope_angles=32)
    vn64 = rmsnorm_f64(v, np.ones(hd), hd, eps).reshape(T, Hkv, hd)
    want = attention_f64(qr64, kr64, vn64, 1.0)
    # scale 1.0 with unit-RMS heads gives score std ~16: f32 rounding of the inputs is
    # amplified, so the f32-vs-f64 residual is larger than for the 1/sqrt(hd) configs.
    assert rel_l2_f64(o, want) < 1e-4
    np.savez(os.path.join(HERE, "gemma_t32_prefill.npz"), T=T, H=H, Hkv=Hkv, hd=hd, eps=eps,
             theta=1e6, rope_angles=32, seeds=np.array([1, 2, 3, 4, 5]), sha_q=sha(q),
             sha_k=sha(k), sha_v=sha(v), sha_q_rope=sha(qr), sha_k_rope=sha(kr),
             sha_v_norm=sha(vn), o=o)


if __name__ == "__main__":
    qwen_t64()
    qwen_decode_small()
    reference_ramp_cases()
    gemma_t32()
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)))
