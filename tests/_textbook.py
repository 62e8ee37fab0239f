"""Independent float64 attention, RMSNorm and RoPE used to pin the oracle and the kernels.

These are the textbook formulas evaluated in float64 with numpy, written from the
mathematics (softmax(scale * Q K^T + causal mask) V, with query head h reading KV head
h // (H / Hkv)); they share no code with oracle/oracle.c.
"""
import numpy as np


def attention_f64(q, k, v, scale, causal=True, q_offset=0, window=0):
    """q [T, H, D], k/v [S, Hkv, D] -> o [T, H, D] in float64.

    Query row t sits at absolute position p = q_offset + t and may attend keys 0..=p when
    causal; with window > 0 only the keys p - window < j <= p."""
    q = np.asarray(q, np.float64)
    k = np.asarray(k, np.float64)
    v = np.asarray(v, np.float64)
    T, H, D = q.shape
    S, Hkv, _ = k.shape
    g = H // Hkv
    kr = np.repeat(k, g, axis=1)  # [S, H, D]: head h -> kv head h // g
    vr = np.repeat(v, g, axis=1)
    s = np.einsum("thd,shd->hts", q, kr) * scale  # [H, T, S]
    if causal:
        pos = q_offset + np.arange(T)[:, None]
        mask = np.arange(S)[None, :] > pos
        if window > 0:
            mask = mask | (np.arange(S)[None, :] <= pos - window)
        s = np.where(mask[None], -np.inf, s)
    s = s - s.max(axis=-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(axis=-1, keepdims=True)
    return np.einsum("hts,shd->thd", p, vr)


def rmsnorm_f64(x, w, dim, eps):
    x = np.asarray(x, np.float64).reshape(-1, dim)
    w = np.asarray(w, np.float64)
    return x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * w


def rope_f64(x, seq, n_heads, hd, theta, rope_angles=None, base_pos=0):
    """Half-split rotary: pairs (p, p + hd/2) rotated by angle (s + base_pos) * theta^(-2p/hd)
    for p < rope_angles; the remaining pairs pass through."""
    half = hd // 2
    ra = half if rope_angles is None else min(rope_angles, half)
    x = np.asarray(x, np.float64).reshape(seq, n_heads, hd)
    p = np.arange(half)
    ang = (base_pos + np.arange(seq))[:, None] * np.power(float(np.float32(theta)), -2.0 * p / hd)[None, :]
    ang = np.where(p[None, :] < ra, ang, 0.0)
    c = np.cos(ang)[:, None, :]
    s = np.sin(ang)[:, None, :]
    x1, x2 = x[..., :half], x[..., half:]
    return np.concatenate([x1 * c - x2 * s, x2 * c + x1 * s], axis=-1)


def rel_l2_f64(a, b):
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-12))


def ramp(n, off, step):
    """`off + i * step` in f32, as the reference's kernel tests build their inputs
    (crates/eyebrowse-kernels/src/attention.rs:170-172)."""
    return (np.float32(off) + np.arange(n, dtype=np.float32) * np.float32(step)).astype(np.float32)
